"""One serving step: schedule -> pack -> forward -> sample -> update
(reference runtime/model_runner.py:13-388).

``build_model_batch`` packs the scheduled requests (prefills first, then
decodes) into flat token/position arrays with ``query_start_loc`` offsets and
the paged-attention metadata: right-padded (-1) block tables, context lengths
and the slot of every scheduled token, slot = table[pos // B] * B + pos % B.

``execute_model_batch`` runs the model on those metadata. The reference runs
one ``forward_prefill_with_cache`` per prefill request; here every prefill of
the step goes through one packed forward (``forward_prefill_packed_with_cache``:
one varlen prefill launch per layer), and the decodes through one batched
decode forward, as in the reference. Logits come back in packed token order
whatever the order of phases in the batch. The batch checks are the
reference's, with its messages and order, evaluated with one host sync
instead of several per request; the same pass also runs the checks the
packed prefill forward and the batched decode forward would otherwise make
on their parts of the batch (positions, slots and distinct slots per phase,
with those forwards' messages), so both run with ``metadata_checked``. The
index lists reach the device through pinned memory without a wait: once a
forward is queued, a host sync or a pageable upload would stall the host until
its kernels finish, and the GPU would then idle while the host prepares the
next forward.

With ``decode_graphs`` (runtime/step_graphs.py) the decodes of a step
replay a HIP graph of the batched decode forward, recorded once per batch
size, instead of issuing its kernels from the host; with ``prefill_graphs``
a packed prefill whose shape repeats replays its recorded forward.

``run_generation_step`` also checks the decode workspaces once per step: a
split merge that gave up waiting (it only writes NaN) raises
``DecodeMergeError`` there instead of reaching the sampled tokens unnoticed.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ..kernels import paged_attention as kpa
from .paged_kv_cache import PagedKVCache
from .request import Request, RequestStatus
from .scheduler import Scheduler, SchedulerOutput


@dataclass
class ModelBatch:
    """Flattened model inputs of all requests in one scheduler step."""

    request_ids: list[str]
    input_token_ids: torch.Tensor
    positions: torch.Tensor
    query_start_loc: torch.Tensor
    request_phases: list[RequestStatus]
    context_lens: torch.Tensor
    block_tables: torch.Tensor
    slot_mapping: torch.Tensor


@dataclass
class GenerationStepResult:
    scheduler_output: SchedulerOutput
    model_batch: ModelBatch
    packed_logits: torch.Tensor
    sampled_token_ids: dict[str, int]
    finished_requests: list[Request]


def _check_blocks(request: Request, start: int, count: int, block_size: int) -> None:
    """The table must cover every scheduled position (reference :54-64)."""
    last = start + count - 1
    if count > 0 and last // block_size >= len(request.block_table):
        # The first position without a block, as the reference reports it.
        missing = max(start, len(request.block_table) * block_size)
        raise ValueError(f"Request {request.request_id} has no KV cache block "
                         f"for position {missing}")


def _slots(request: Request, start: int, count: int, block_size: int) -> list[int]:
    _check_blocks(request, start, count, block_size)
    table = request.block_table
    return [table[p // block_size] * block_size + p % block_size
            for p in range(start, start + count)]


def build_model_batch(scheduler_output: SchedulerOutput, block_size: int,
                      device: torch.device | str = "cpu") -> ModelBatch:
    """The step's packed inputs: prefill requests first, then decodes.

    On a HIP device the host does per-request work only (the reference's
    checks, the token ids, one (first position, count) pair and the padded
    block table per request), moves it in one copy, and one
    mlr_build_step_metadata launch expands positions, slot_mapping,
    query_start_loc and context_lens on the device. Other devices get the
    same tensors built on the host."""
    if block_size <= 0:
        raise ValueError("block_size must be greater than 0")
    entries: list[tuple[Request, RequestStatus, list[int], int]] = []
    for request in scheduler_output.prefill_requests:
        count = scheduler_output.num_scheduled_tokens[request.request_id]
        start = request.num_computed_tokens
        chunk = request.prompt_token_ids[start:start + count]
        if len(chunk) != count:
            raise ValueError(f"Request {request.request_id} expected {count} prefill "
                             f"tokens, got {len(chunk)}")
        _check_blocks(request, start, count, block_size)
        entries.append((request, RequestStatus.PREFILLING, chunk, start))
    for request in scheduler_output.decode_requests:
        if scheduler_output.num_scheduled_tokens[request.request_id] != 1:
            raise ValueError("Decode currently supports exactly one token per request")
        pending = request.pending_token_id
        if pending is None:
            raise ValueError(f"Decode request {request.request_id} has no pending token")
        _check_blocks(request, request.num_computed_tokens, 1, block_size)
        entries.append((request, RequestStatus.DECODING, [pending],
                        request.num_computed_tokens))
    dev = torch.device(device)
    if dev.type == "cuda" and entries:
        return _build_on_device(entries, block_size, dev)
    return _build_on_host(entries, block_size, dev)


def _build_on_host(entries, block_size: int, dev: torch.device) -> ModelBatch:
    tokens: list[int] = []
    positions: list[int] = []
    qsl = [0]
    ctx: list[int] = []
    slots: list[int] = []
    for request, _, new_tokens, start in entries:
        count = len(new_tokens)
        slots.extend(_slots(request, start, count, block_size))
        tokens.extend(new_tokens)
        positions.extend(range(start, start + count))
        qsl.append(qsl[-1] + count)
        ctx.append(start + count)
    tables = [list(e[0].block_table) for e in entries]
    width = max((len(t) for t in tables), default=0)
    padded = [t + [-1] * (width - len(t)) for t in tables]

    def long(values) -> torch.Tensor:
        return torch.tensor(values, dtype=torch.long, device=dev)

    return ModelBatch(
        request_ids=[e[0].request_id for e in entries],
        input_token_ids=long(tokens),
        positions=long(positions),
        query_start_loc=long(qsl),
        request_phases=[e[1] for e in entries],
        context_lens=long(ctx),
        block_tables=long(padded) if tables else torch.empty((0, 0), dtype=torch.long,
                                                              device=dev),
        slot_mapping=long(slots),
    )


def _build_on_device(entries, block_size: int, dev: torch.device) -> ModelBatch:
    import numpy as np

    from .. import _lib

    num_reqs = len(entries)
    counts = [len(e[2]) for e in entries]
    num_tokens = sum(counts)
    width = max(len(e[0].block_table) for e in entries)
    # One host buffer: token ids, then (first position, count) per request,
    # then the block tables padded with -1.
    host = np.empty(num_tokens + 2 * num_reqs + num_reqs * width, dtype=np.int64)
    tok = host[:num_tokens]
    info = host[num_tokens:num_tokens + 2 * num_reqs].reshape(num_reqs, 2)
    tab = host[num_tokens + 2 * num_reqs:].reshape(num_reqs, width)
    tab.fill(-1)
    at = 0
    for i, (request, _, new_tokens, start) in enumerate(entries):
        tok[at:at + counts[i]] = new_tokens
        at += counts[i]
        info[i, 0] = start
        info[i, 1] = counts[i]
        tab[i, :len(request.block_table)] = request.block_table
    buf = torch.from_numpy(host).to(dev)
    out = torch.empty(2 * num_tokens + 2 * num_reqs + 1, dtype=torch.long, device=dev)
    positions, slots = out[:num_tokens], out[num_tokens:2 * num_tokens]
    qsl = out[2 * num_tokens:2 * num_tokens + num_reqs + 1]
    ctx = out[2 * num_tokens + num_reqs + 1:]
    tables = buf[num_tokens + 2 * num_reqs:].view(num_reqs, width)
    lib = _lib.load()
    with torch.cuda.device(dev):
        status = lib.mlr_build_step_metadata(
            buf[num_tokens:].data_ptr(), tables.data_ptr(), width, width, num_reqs,
            num_tokens, block_size, positions.data_ptr(), slots.data_ptr(), qsl.data_ptr(),
            ctx.data_ptr(), _lib.stream_handle(dev))
    _lib.check(status, "mlr_build_step_metadata")
    return ModelBatch(
        request_ids=[e[0].request_id for e in entries],
        input_token_ids=buf[:num_tokens],
        positions=positions,
        query_start_loc=qsl,
        request_phases=[e[1] for e in entries],
        context_lens=ctx,
        block_tables=tables,
        slot_mapping=slots,
    )


def _upload(values, device: torch.device) -> torch.Tensor:
    """A host list of ints as an int64 tensor on `device`. For a GPU the list
    is staged in pinned memory and copied asynchronously on the current
    stream, so the host does not wait for the kernels already queued there
    (a copy from pageable memory would)."""
    if device.type != "cuda":
        return torch.tensor(values, dtype=torch.long, device=device)
    staged = torch.tensor(values, dtype=torch.long, pin_memory=True)
    return staged.to(device, non_blocking=True)


def _check_batch(model, batch: ModelBatch, kv_cache: PagedKVCache) -> tuple[list[int], int]:
    """The reference's execute_model_batch checks (:154-243), in its order,
    then the metadata checks of the two forwards that execute_model_batch runs
    on parts of the batch: the packed prefill's
    (TinyQwen2Model.check_prefill_packed_inputs) on the prefilling requests,
    then the batched decode's (Qwen2Attention._check_decode_metadata) on the
    decoding ones, with their messages and order; all of it with one host
    sync. Of those forwards' checks, the ones on query_start_loc, max_query_len
    and the block tables hold by construction or by the checks above; the rest
    are evaluated here over the whole batch: each token's position (prefill:
    context_len - num_tokens + its offset; decode: context_len - 1, the same
    formula for one token), its slot against the block table, and distinct
    slots among the prefill tokens and among the decode tokens. Returns the
    host copy of query_start_loc and the packed token count."""
    n = len(batch.request_ids)
    if len(batch.request_phases) != n:
        raise ValueError("request_phases length must match request_ids")
    if not n:
        raise ValueError("Cannot execute an empty ModelBatch")
    for name in ("input_token_ids", "positions", "slot_mapping"):
        if getattr(batch, name).ndim != 1:
            raise ValueError(f"{name} must be one-dimensional")
    num_tokens = batch.input_token_ids.numel()
    if batch.positions.numel() != num_tokens:
        raise ValueError("positions length must match input_token_ids")
    if batch.slot_mapping.numel() != num_tokens:
        raise ValueError("slot_mapping length must match input_token_ids")
    if batch.context_lens.ndim != 1:
        raise ValueError("context_lens must be one-dimensional")
    if batch.context_lens.numel() != n:
        raise ValueError("context_lens length must match request_ids")
    if batch.block_tables.ndim != 2:
        raise ValueError("block_tables must be two-dimensional")
    if batch.block_tables.shape[0] != n:
        raise ValueError("block_tables rows must match request_ids")
    index = {"input_token_ids": batch.input_token_ids, "positions": batch.positions,
             "query_start_loc": batch.query_start_loc, "context_lens": batch.context_lens,
             "block_tables": batch.block_tables, "slot_mapping": batch.slot_mapping}
    for name, tensor in index.items():
        if tensor.dtype is not torch.long:
            raise ValueError(f"{name} must use torch.long dtype")
    device = batch.input_token_ids.device
    for name, tensor in index.items():
        if tensor.device != device:
            raise ValueError(f"{name} must be on the same device as input_token_ids")
    param = next(model.parameters())
    if device != param.device:
        raise ValueError("ModelBatch and model must be on the same device")
    if kv_cache.device != param.device:
        raise ValueError("KV cache and model must be on the same device")
    if kv_cache.dtype != param.dtype:
        raise ValueError("KV cache dtype must match model dtype")
    if batch.query_start_loc.ndim != 1:
        raise ValueError("query_start_loc must be one-dimensional")
    if batch.query_start_loc.numel() != n + 1:
        raise ValueError("query_start_loc must contain one more entry than request_ids")

    # Everything the data-dependent checks need, in one transfer: the query
    # offsets, the context lengths and, per request, whether a block its
    # context uses lies outside the cache (blocks needed: ceil(ctx / bs), none
    # for ctx <= 0).
    bs, width = kv_cache.block_size, batch.block_tables.shape[1]
    required_dev = torch.div(batch.context_lens + (bs - 1), bs,
                             rounding_mode="floor").clamp_(min=0)
    used = torch.arange(width, device=device)[None, :] < required_dev[:, None]
    bad = (used & ((batch.block_tables < 0)
                   | (batch.block_tables >= kv_cache.num_blocks))).any(dim=1)
    flags = _step_metadata_flags(batch, bs, width, device)
    host = torch.cat([batch.query_start_loc, batch.context_lens, bad.long(),
                      flags.long()]).tolist()
    qsl, ctx, bad_rows = host[:n + 1], host[n + 1:2 * n + 1], host[2 * n + 1:3 * n + 1]
    flags = host[3 * n + 1:]
    if qsl[0] != 0:
        raise ValueError("query_start_loc must start at 0")
    if any(b <= a for a, b in zip(qsl, qsl[1:])):
        raise ValueError("query_start_loc must be strictly increasing")
    if qsl[-1] != num_tokens:
        raise ValueError("query_start_loc must end at the packed token count")
    required = [-(-c // bs) if c > 0 else 0 for c in ctx]
    for i, request_id in enumerate(batch.request_ids):
        if ctx[i] <= 0:
            raise ValueError(f"Request {request_id} context_len must be greater than 0")
        if width < required[i]:
            raise ValueError(f"Request {request_id} block_table has insufficient blocks")
        if bad_rows[i]:
            raise ValueError(f"Request {request_id} block_table contains an invalid "
                             "physical block")
    for i, phase in enumerate(batch.request_phases):
        if phase is RequestStatus.DECODING:
            if qsl[i + 1] - qsl[i] != 1:
                raise ValueError("Decode requires exactly one token per request")
        elif phase is not RequestStatus.PREFILLING:
            raise ValueError(f"Unsupported request phase {phase} for request "
                             f"{batch.request_ids[i]}")
    prefilling = [i for i, ph in enumerate(batch.request_phases)
                  if ph is RequestStatus.PREFILLING]
    if prefilling:
        if any(ctx[i] < qsl[i + 1] - qsl[i] for i in prefilling):
            raise ValueError("context_lens must cover each request's tokens")
        if flags[0]:
            raise ValueError("position_ids must run from context_len - num_tokens "
                             "to context_len - 1 for each request")
        if flags[1]:
            raise ValueError("slot_mapping must match block_tables and positions")
        if flags[2]:
            raise ValueError("packed tokens must use distinct write slots")
    if flags[3]:
        raise ValueError("decode positions must equal context_lens - 1")
    if flags[4]:
        raise ValueError("slot_mapping must match block_tables and positions")
    if flags[5]:
        raise ValueError("decode requests must use distinct write slots")
    return qsl, num_tokens


def _step_metadata_flags(batch: ModelBatch, bs: int, width: int,
                         device: torch.device) -> torch.Tensor:
    """Six device flags over the packed tokens: (prefill tokens) a position
    that is not context_len - num_tokens + offset, a slot that does not match
    the block table, a repeated slot; the same three for the decode tokens.
    Every index is clamped into range, so the gathers stay in bounds whatever
    the batch holds; flags that a malformed query_start_loc or block table
    makes meaningless are not read, as the checks before them raise."""
    n = len(batch.request_ids)
    num_tokens = batch.input_token_ids.numel()
    if num_tokens == 0 or width == 0:  # the checks before these raise
        return torch.zeros(6, dtype=torch.bool, device=device)
    qsl, ctx, tables = batch.query_start_loc, batch.context_lens, batch.block_tables
    positions, slots = batch.positions, batch.slot_mapping
    decoding = _upload([ph is RequestStatus.DECODING for ph in batch.request_phases],
                       device).bool()
    tokens = torch.arange(num_tokens, device=device)
    owner = torch.searchsorted(qsl[1:].contiguous(), tokens, right=True).clamp_(max=n - 1)
    lens = qsl[1:] - qsl[:-1]
    expected_pos = (ctx - lens)[owner] + tokens - qsl[:-1][owner]
    col = (positions // bs).clamp(0, width - 1)
    expected_slot = tables[owner, col] * bs + positions % bs
    dec = decoding[owner]
    bad_pos = positions != expected_pos
    bad_slot = slots != expected_slot
    # Repeated slots within a phase: the phase in the key's low bit.
    ordered = (slots * 2 + dec.long()).sort().values
    repeat = ordered[1:] == ordered[:-1]
    repeat_dec = (ordered[1:] & 1).bool()
    return torch.stack([(bad_pos & ~dec).any(), (bad_slot & ~dec).any(),
                        (repeat & ~repeat_dec).any(), (bad_pos & dec).any(),
                        (bad_slot & dec).any(), (repeat & repeat_dec).any()])


def execute_model_batch(model, batch: ModelBatch, kv_cache: PagedKVCache,
                        decode_graphs=None, prefill_graphs=None) -> torch.Tensor:
    """[num_packed_tokens, vocab_size] logits in packed token order.

    decode_graphs / prefill_graphs: a DecodeGraphs / PrefillGraphs
    (runtime/step_graphs.py) of this model and cache; the batch's decodes
    (prefills) then go through it, replaying recorded graphs instead of
    running the forward eagerly."""
    qsl, num_tokens = _check_batch(model, batch, kv_cache)
    for name, graphs in (("decode_graphs", decode_graphs), ("prefill_graphs", prefill_graphs)):
        if graphs is not None and (graphs.model is not model or graphs.kv_cache is not kv_cache):
            raise ValueError(f"{name} must belong to this model and KV cache")
    device = batch.input_token_ids.device
    logits = model.lm_head.weight.new_empty((num_tokens, model.lm_head.out_features))
    prefill = [i for i, ph in enumerate(batch.request_phases) if ph is RequestStatus.PREFILLING]
    decode = [i for i, ph in enumerate(batch.request_phases) if ph is RequestStatus.DECODING]

    packed = step = None
    if prefill:
        lens = [qsl[i + 1] - qsl[i] for i in prefill]
        contiguous = prefill == list(range(len(prefill)))
        if contiguous:  # build_model_batch's order: the prefill tokens lead
            rows = slice(0, qsl[len(prefill)])
            pick = lambda t: t[rows]  # noqa: E731
        else:
            idx = _upload([t for i in prefill for t in range(qsl[i], qsl[i + 1])], device)
            pick = lambda t: t.index_select(0, idx)  # noqa: E731
        req = _upload(prefill, device)
        offsets = [0]
        for n in lens:
            offsets.append(offsets[-1] + n)
        packed = (pick(batch.input_token_ids), pick(batch.positions), pick(batch.slot_mapping),
                  batch.block_tables.index_select(0, req), _upload(offsets, device),
                  batch.context_lens.index_select(0, req))
    if decode:
        req = _upload(decode, device)
        decode_rows = _upload([qsl[i] for i in decode], device)
        step = dict(input_ids=batch.input_token_ids.index_select(0, decode_rows).unsqueeze(1),
                    position_ids=batch.positions.index_select(0, decode_rows).unsqueeze(1),
                    slot_mapping=batch.slot_mapping.index_select(0, decode_rows),
                    block_tables=batch.block_tables.index_select(0, req),
                    context_lens=batch.context_lens.index_select(0, req))

    # _check_batch ran both forwards' metadata checks; the cache's shape
    # against the model is the one check of theirs left.
    model.model._check_cache(kv_cache)

    # Each forward's LM head writes its rows of `logits` directly where they
    # are contiguous (the prefills lead in build_model_batch's order and the
    # decodes follow), instead of into a new tensor copied in afterwards.
    if packed is not None:
        target = logits[rows] if contiguous else None
        if prefill_graphs is not None:
            out = prefill_graphs(*packed, max(lens), metadata_checked=True, out=target)
        else:
            out = model.logits(model.model.forward_prefill_packed_with_cache(
                *packed[:2], kv_cache, *packed[2:], max(lens), metadata_checked=True), target)
        if not contiguous:
            logits.index_copy_(0, idx, out)
    if step is not None:
        target = None
        if decode[-1] - decode[0] == len(decode) - 1:  # consecutive one-token requests
            target = logits[qsl[decode[0]]:qsl[decode[0]] + len(decode)]
        if decode_graphs is not None:
            out = decode_graphs(**step, metadata_checked=True, out=target)
        else:
            out = model.logits(model.model.forward_decode_batch_with_cache(
                kv_cache=kv_cache, **step, metadata_checked=True)[:, 0], target)
        if target is None:
            logits.index_copy_(0, decode_rows, out.reshape(len(decode), -1))
    return logits


def greedy_sample(packed_logits: torch.Tensor, batch: ModelBatch) -> dict[str, int]:
    """Argmax of each request's last scheduled token (reference :287-322)."""
    if packed_logits.ndim != 2:
        raise ValueError("packed_logits must have shape [total_tokens, vocab_size]")
    if packed_logits.shape[0] != batch.input_token_ids.shape[0]:
        raise ValueError("packed_logits token dimension must match ModelBatch tokens")
    if len(batch.request_ids) + 1 != batch.query_start_loc.numel():
        raise ValueError("query_start_loc must contain one more entry than request_ids")
    n = len(batch.request_ids)
    if n and packed_logits.shape[0]:
        # Each request's last row on the device, clamped so that the gather
        # stays in bounds whatever query_start_loc holds: the offsets and the
        # picks come back in one transfer, and the offsets are checked below.
        qsl_dev = batch.query_start_loc
        last = (qsl_dev[1:] - 1).clamp(0, packed_logits.shape[0] - 1)
        picks_dev = packed_logits.index_select(0, last).argmax(dim=-1)
        host = torch.cat([qsl_dev, picks_dev.to(qsl_dev.device)]).tolist()
        qsl, picks = host[:n + 1], host[n + 1:]
    else:
        qsl, picks = batch.query_start_loc.tolist(), []
    for i, request_id in enumerate(batch.request_ids):
        if qsl[i + 1] <= qsl[i]:
            raise ValueError(f"Request {request_id} must contain at least one query token")
    if not batch.request_ids:
        return {}
    return dict(zip(batch.request_ids, picks))


def run_generation_step(model, scheduler: Scheduler,
                        eos_token_id: int | None = None,
                        decode_graphs=None, prefill_graphs=None) -> GenerationStepResult:
    if not scheduler.waiting and not scheduler.running:
        raise ValueError("Cannot run generation step with no requests")
    scheduler_output = scheduler.schedule()
    if scheduler_output.is_empty:
        raise RuntimeError("Scheduler made no progress while unfinished requests remain")
    batch = build_model_batch(scheduler_output, block_size=scheduler.kv_cache.block_size,
                              device=scheduler.kv_cache.device)
    packed_logits = execute_model_batch(model=model, batch=batch, kv_cache=scheduler.kv_cache,
                                        decode_graphs=decode_graphs,
                                        prefill_graphs=prefill_graphs)
    sampled = greedy_sample(packed_logits, batch)
    if batch.input_token_ids.device.type == "cuda":
        # Before any sampled token is committed to the scheduler.
        kpa.check_decode_workspaces(batch.input_token_ids.device)
    eos = ({rid for rid, tok in sampled.items() if tok == eos_token_id}
           if eos_token_id is not None else set())
    finished = scheduler.update_after_model(scheduler_output=scheduler_output,
                                            sampled_token_ids=sampled,
                                            reached_eos_request_ids=eos)
    return GenerationStepResult(scheduler_output=scheduler_output, model_batch=batch,
                                packed_logits=packed_logits, sampled_token_ids=sampled,
                                finished_requests=finished)


def run_greedy_generation(model, scheduler: Scheduler,
                          eos_token_id: int | None = None,
                          decode_graphs=None, prefill_graphs=None) -> list[Request]:
    """Schedule-model-sample-update until every request has finished."""
    finished: list[Request] = []
    while scheduler.waiting or scheduler.running:
        finished.extend(run_generation_step(
            model, scheduler, eos_token_id=eos_token_id, decode_graphs=decode_graphs,
            prefill_graphs=prefill_graphs).finished_requests)
    return finished
