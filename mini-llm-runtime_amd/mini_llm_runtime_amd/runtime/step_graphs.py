"""The batched decode step, and repeated packed prefills, of a causal LM
replayed from HIP graphs.

The reference runs every decode step eagerly
(runtime/model_runner.py:execute_model_batch ->
TinyQwen2ForCausalLM.forward_decode_batch_with_cache, model/qwen2.py), so a
step costs the host time of issuing each layer's kernels: embedding, then per
layer RMSNorms, the QKV GEMM, the fused rotation + KV write + paged decode,
the output projection, the MLP and the residual adds, then the final norm and
the LM head, several hundred launches for a 24-layer model. At small batches
that host time is the whole step.

``DecodeGraphs`` records that step once per batch size into a HIP graph
(``torch.cuda.CUDAGraph``) over static input buffers and replays it. A call:

1. checks shapes, dtypes and devices, then the step's metadata against the
   cache with the model's own device-side checks
   (``Qwen2Attention._check_decode_metadata``: one host sync, the reference's
   messages and order, before anything is written);
2. copies token ids, positions, slots, context lengths and the block table
   into the batch size's static buffers on the current stream; the block
   table is right-padded with -1 to the fixed width ``max_blocks_per_seq``,
   so every replay's decode launch has the grid it was recorded with (the
   padded columns lie past every context and are never read);
3. replays the graph on the current stream.

The first call of a batch size records its graph: one eager step on the
runner's own stream (it sizes the decode workspace cached for that stream and
the model's concatenated QKV weights), then the capture on that stream with
the layers' metadata checks off (they were done in step 1). Nothing in the
recorded step allocates outside the graph's private pool or clears memory with
a memset: the decode workspace is returned to zero by the kernels themselves.

``record(batch_sizes)`` records graphs ahead of serving, as a server does at
start-up, so that no serving step pays for a recording: the dummy step of a
batch size puts row j at position j % block_size of a block the runner holds
(a context of j % block_size + 1 tokens), so every row writes its own slot and
nothing outside those blocks. The blocks come from the cache's allocator, as
a sequence of the runner's own, and go back with ``release()``.

A graph ends at the final norm's hidden states: the LM head runs after the
replay, into ``out`` when the caller passes one (the runner passes the decode
rows of its packed logits, so they are written once and not copied) and into
a new tensor otherwise. Graphs hold the weights and the cache as they were
recorded: replace a weight or the cache and call ``reset()``. Replays must not
overlap (one stream at a time): the graphs of one runner share its decode
workspace. A block table wider than ``max_blocks_per_seq`` runs the same step
eagerly (counted in ``eager_calls``).

``PrefillGraphs`` does the same for the packed prefill forward
(``forward_prefill_packed_with_cache``, logits of every packed token), whose
shape a server meets again and again (the same number of prompts of the same
lengths each step). A graph is keyed by the call's shape: tokens, requests,
longest query and block-table width (the prefill launch's grid follows from
them; the offsets, lengths, slots and tables are read on the device). A shape
runs eagerly until it is met for the ``record_at``-th time, and is recorded
then; at most ``max_graphs`` recordings are kept (least recently used
dropped), as each holds its static buffers (the hidden states, [tokens,
hidden], and the forward's intermediates in its private pool). As for the
decode, the LM head runs after the replay, into ``out`` when given. Only a runner's
first recording runs the eager step before its capture: the packed prefill
uses no decode workspace, and the model's cached weights and the stream's
GEMM state exist from then on. Every call runs the model's
own checks first (``check_prefill_packed_inputs``: one host sync, before
anything is written).
"""

from __future__ import annotations

from collections import OrderedDict

import torch

from ..model.qwen2_attention import Qwen2Attention
from .paged_kv_cache import PagedKVCache


class _Recorded:
    """Static inputs of one batch size and, once recorded, its graph."""

    def __init__(self, batch: int, width: int, device: torch.device) -> None:
        self.input_ids = torch.zeros(batch, 1, dtype=torch.long, device=device)
        self.position_ids = torch.zeros(batch, 1, dtype=torch.long, device=device)
        self.slot_mapping = torch.zeros(batch, dtype=torch.long, device=device)
        self.block_tables = torch.full((batch, width), -1, dtype=torch.long, device=device)
        self.context_lens = torch.ones(batch, dtype=torch.long, device=device)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.hidden: torch.Tensor | None = None

    def load(self, input_ids, position_ids, slot_mapping, block_tables, context_lens) -> None:
        width = block_tables.shape[1]
        self.input_ids.copy_(input_ids)
        self.position_ids.copy_(position_ids)
        self.slot_mapping.copy_(slot_mapping)
        self.context_lens.copy_(context_lens)
        self.block_tables[:, :width].copy_(block_tables)
        if width < self.block_tables.shape[1]:
            self.block_tables[:, width:].fill_(-1)


def _record(device, stream, step, warm=True):
    """With `warm`, one eager `step` on `stream` first (it sizes that stream's
    cached decode workspace and builds the model's concatenated weights and
    the stream's GEMM state outside the graph); then `step` recorded on
    `stream`: (graph, its output)."""
    current = torch.cuda.current_stream(device)
    stream.wait_stream(current)
    if warm:
        with torch.cuda.stream(stream):
            step()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        out = step()
    current.wait_stream(stream)
    return graph, out


def _check_pair(model, kv_cache) -> torch.device:
    device = kv_cache.device
    if device.type != "cuda":
        raise ValueError("step graphs need the KV cache on a HIP device")
    if model.lm_head.weight.device != device:
        raise ValueError("model and KV cache must be on the same device")
    config = model.model.config
    if kv_cache.num_layers != config.num_hidden_layers:
        raise ValueError("KV cache num_layers must match model layers")
    if kv_cache.num_kv_heads != config.num_key_value_heads:
        raise ValueError("KV cache num_kv_heads must match model num_key_value_heads")
    if kv_cache.head_dim != config.head_dim:
        raise ValueError("KV cache head_dim must match model head_dim")
    if kv_cache.dtype != model.lm_head.weight.dtype:
        raise ValueError("KV cache dtype must match the model's dtype")
    return device


class DecodeGraphs:
    """HIP-graph replay of ``model.forward_decode_batch_with_cache`` on one
    paged KV cache (see the module docstring).

    model: a TinyQwen2ForCausalLM on a HIP device, in eval mode.
    kv_cache: the PagedKVCache the steps read and write.
    max_blocks_per_seq: the block-table width every graph is recorded with;
        the longest context a replay serves is max_blocks_per_seq * block_size.
    """

    def __init__(self, model, kv_cache: PagedKVCache, max_blocks_per_seq: int) -> None:
        device = _check_pair(model, kv_cache)
        if int(max_blocks_per_seq) <= 0:
            raise ValueError("max_blocks_per_seq must be > 0")
        self.model = model
        self.kv_cache = kv_cache
        self.width = int(max_blocks_per_seq)
        self.device = device
        self.stream = torch.cuda.Stream(device)  # default priority
        self._recorded: dict[int, _Recorded] = {}
        self._scratch_key = ("decode_graphs", id(self))
        self.captures = 0
        self.replays = 0
        self.eager_calls = 0

    def reset(self) -> None:
        """Drop every recorded graph (after a weight or the cache changed)."""
        self._recorded.clear()

    def record(self, batch_sizes) -> None:
        """Record the graphs of `batch_sizes` (those not recorded yet) on
        dummy steps over the runner's own blocks (see the module docstring)."""
        sizes = sorted({int(b) for b in batch_sizes})
        if not sizes or sizes[0] <= 0:
            raise ValueError("batch sizes must be > 0")
        sizes = [b for b in sizes if b not in self._recorded]
        if not sizes:
            return
        cache, bs = self.kv_cache, self.kv_cache.block_size
        if self._scratch_key not in cache.block_tables:
            cache.add_sequence(self._scratch_key)
        if not cache.reserve_tokens(self._scratch_key, sizes[-1]):
            raise RuntimeError("KV cache has no free blocks for the dummy decode rows")
        blocks = torch.tensor(cache.block_tables[self._scratch_key], dtype=torch.long)
        cache.k_cache[:, blocks.to(self.device)] = 0
        cache.v_cache[:, blocks.to(self.device)] = 0
        for batch in sizes:
            rows = torch.arange(batch)
            offsets = rows % bs
            tables = blocks[rows // bs][:, None]
            r = _Recorded(batch, self.width, self.device)
            r.load(torch.zeros(batch, 1, dtype=torch.long), offsets[:, None],
                   tables[:, 0] * bs + offsets, tables, offsets + 1)
            self._record(r)
            self._recorded[batch] = r

    def release(self) -> None:
        """Drop every recorded graph and return the dummy rows' blocks."""
        self.reset()
        if self._scratch_key in self.kv_cache.block_tables:
            self.kv_cache.free_sequence(self._scratch_key)

    def _check(self, input_ids, position_ids, slot_mapping, block_tables, context_lens) -> int:
        if input_ids.ndim != 2 or input_ids.shape[1] != 1:
            raise ValueError("input_ids must have shape [B, 1] for decode")
        batch = input_ids.shape[0]
        if batch == 0:
            raise ValueError("decode batch must not be empty")
        if input_ids.dtype not in (torch.int32, torch.int64):
            raise TypeError("input_ids must have dtype torch.int32 or torch.int64")
        if position_ids.shape != (batch, 1):
            raise ValueError("position_ids must have shape [B, 1]")
        if slot_mapping.shape != (batch,):
            raise ValueError("slot_mapping must have shape [B]")
        if context_lens.shape != (batch,):
            raise ValueError("context_lens must have shape [B]")
        if block_tables.ndim != 2 or block_tables.shape[0] != batch or block_tables.shape[1] == 0:
            raise ValueError("block_tables must have shape [B, max_num_blocks]")
        for name, tensor in (("input_ids", input_ids), ("position_ids", position_ids),
                             ("slot_mapping", slot_mapping), ("context_lens", context_lens),
                             ("block_tables", block_tables)):
            if tensor.device != self.device:
                raise ValueError(f"{name} must be on the KV cache's device")
            if name != "input_ids" and tensor.dtype != torch.long:
                raise ValueError(f"{name} must use torch.long dtype")
        return batch

    def _step(self, r: _Recorded) -> torch.Tensor:
        return self.model.model.forward_decode_batch_with_cache(
            r.input_ids, r.position_ids, self.kv_cache, r.slot_mapping, r.block_tables,
            r.context_lens, metadata_checked=True)

    def _record(self, r: _Recorded) -> None:
        r.graph, r.hidden = _record(self.device, self.stream, lambda: self._step(r))
        self.captures += 1

    def _logits(self, hidden: torch.Tensor, out: torch.Tensor | None) -> torch.Tensor:
        if out is None:
            return self.model.logits(hidden)
        return self.model.logits(hidden[:, 0], out)

    def __call__(self, input_ids: torch.Tensor, position_ids: torch.Tensor,
                 slot_mapping: torch.Tensor, block_tables: torch.Tensor,
                 context_lens: torch.Tensor, *, metadata_checked: bool = False,
                 out: torch.Tensor | None = None) -> torch.Tensor:
        """[B, 1] token ids -> [B, 1, vocab_size] logits, or the logits
        written into `out` (a contiguous [B, vocab_size] tensor) and `out`
        returned.

        metadata_checked: the caller already ran the device-side metadata
        checks (Qwen2Attention._check_decode_metadata) on these tensors
        against this cache, so the call makes no host sync."""
        batch = self._check(input_ids, position_ids, slot_mapping, block_tables, context_lens)
        if block_tables.shape[1] > self.width:
            self.eager_calls += 1
            return self._logits(self.model.model.forward_decode_batch_with_cache(
                input_ids, position_ids, self.kv_cache, slot_mapping, block_tables,
                context_lens, metadata_checked=metadata_checked), out)
        if not metadata_checked:
            Qwen2Attention._check_decode_metadata(self.kv_cache, position_ids, slot_mapping,
                                                  block_tables, context_lens)
        r = self._recorded.get(batch)
        if r is None:
            r = _Recorded(batch, self.width, self.device)
            r.load(input_ids, position_ids, slot_mapping, block_tables, context_lens)
            self._record(r)
            self._recorded[batch] = r
        else:
            r.load(input_ids, position_ids, slot_mapping, block_tables, context_lens)
        r.graph.replay()
        self.replays += 1
        return self._logits(r.hidden, out)


class _PrefillRecorded:
    """Static inputs of one prefill shape and its graph."""

    def __init__(self, tokens: int, requests: int, width: int, device: torch.device) -> None:
        def zeros(*shape):
            return torch.zeros(*shape, dtype=torch.long, device=device)

        self.input_ids = zeros(tokens)
        self.position_ids = zeros(tokens)
        self.slot_mapping = zeros(tokens)
        self.block_tables = zeros(requests, width)
        self.query_start_loc = zeros(requests + 1)
        self.context_lens = zeros(requests)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.hidden: torch.Tensor | None = None

    def load(self, input_ids, position_ids, slot_mapping, block_tables, query_start_loc,
             context_lens) -> None:
        self.input_ids.copy_(input_ids)
        self.position_ids.copy_(position_ids)
        self.slot_mapping.copy_(slot_mapping)
        self.block_tables.copy_(block_tables)
        self.query_start_loc.copy_(query_start_loc)
        self.context_lens.copy_(context_lens)


class PrefillGraphs:
    """HIP-graph replay of ``model.forward_prefill_packed_with_cache`` for
    shapes met more than once (see the module docstring).

    model: a TinyQwen2ForCausalLM on a HIP device, in eval mode.
    kv_cache: the PagedKVCache the prefills write.
    max_graphs: recordings kept at once (least recently used dropped).
    record_at: the sighting of a shape that records it (1: the first).
    """

    def __init__(self, model, kv_cache: PagedKVCache, max_graphs: int = 8,
                 record_at: int = 3) -> None:
        self.device = _check_pair(model, kv_cache)
        if int(max_graphs) <= 0 or int(record_at) <= 0:
            raise ValueError("max_graphs and record_at must be > 0")
        self.record_at = int(record_at)
        self._warmed = False
        self.model = model
        self.kv_cache = kv_cache
        self.max_graphs = int(max_graphs)
        self.stream = torch.cuda.Stream(self.device)  # default priority
        self._recorded: OrderedDict[tuple, _PrefillRecorded] = OrderedDict()
        self._seen: dict[tuple, int] = {}
        self.captures = 0
        self.replays = 0
        self.eager_calls = 0

    def reset(self) -> None:
        """Drop every recorded graph (after a weight or the cache changed)."""
        self._recorded.clear()
        self._seen.clear()

    def __call__(self, input_ids: torch.Tensor, position_ids: torch.Tensor,
                 slot_mapping: torch.Tensor, block_tables: torch.Tensor,
                 query_start_loc: torch.Tensor, context_lens: torch.Tensor,
                 max_query_len: int, *, metadata_checked: bool = False,
                 out: torch.Tensor | None = None) -> torch.Tensor:
        """[T] token ids -> [T, vocab_size] logits, or the logits written
        into `out` (a contiguous [T, vocab_size] tensor) and `out` returned.

        metadata_checked: the caller already ran the model's
        check_prefill_packed_inputs on these tensors against this cache, so
        the call makes no host sync."""
        if not metadata_checked:
            self.model.model.check_prefill_packed_inputs(
                input_ids, position_ids, self.kv_cache, slot_mapping, block_tables,
                query_start_loc, context_lens, max_query_len)
        key = (input_ids.shape[0], context_lens.shape[0], int(max_query_len),
               block_tables.shape[1])
        args = (input_ids, position_ids, slot_mapping, block_tables, query_start_loc,
                context_lens)
        r = self._recorded.get(key)
        if r is None:
            seen = self._seen.get(key, 0) + 1
            if len(self._seen) >= 4096:
                self._seen.clear()
            self._seen[key] = seen
            if seen < self.record_at:
                self.eager_calls += 1
                return self.model.logits(self.model.model.forward_prefill_packed_with_cache(
                    *args[:2], self.kv_cache, *args[2:], max_query_len, metadata_checked=True),
                    out)
            r = _PrefillRecorded(key[0], key[1], key[3], self.device)
            r.load(*args)
            r.graph, r.hidden = _record(self.device, self.stream, lambda: (
                self.model.model.forward_prefill_packed_with_cache(
                    r.input_ids, r.position_ids, self.kv_cache, r.slot_mapping,
                    r.block_tables, r.query_start_loc, r.context_lens, key[2],
                    metadata_checked=True)), warm=not self._warmed)
            self._warmed = True
            self.captures += 1
            self._recorded[key] = r
            while len(self._recorded) > self.max_graphs:
                self._recorded.popitem(last=False)
        else:
            self._recorded.move_to_end(key)
            r.load(*args)
        r.graph.replay()
        self.replays += 1
        return self.model.logits(r.hidden, out)
