"""Paged attention on MI355X: the reference's kernel API over the HIP library.

Same functions, argument meaning and error messages as
``mini_llm_runtime.kernels.reference.paged_attention`` (the reference), so the
``Qwen2Attention`` paged methods call these unchanged. Every function checks
its arguments on the host first and then launches hand-written gfx950 kernels
through the C ABI (include/mlr_attn.h) on torch's current stream. Tensors must
be on a HIP device; nothing here falls back to PyTorch math.

Numerics (FP32 softmax statistics; P@V in FP32 for the chunk path):
- decode: scores are q.k rounded to the input dtype and scaled, softmax in
  FP32 (reference :246-251). The split-KV combine keeps unnormalised
  probabilities until the end, so BF16 results differ from the reference's
  BF16-rounded normalised probabilities (:251) by rounding only.
- chunk prefill: FP32 online softmax and FP32 P@V, output rounded once
  (reference :411-434).
"""

from __future__ import annotations

import math
from typing import Sequence

import torch

from .. import _lib

_DEFAULT_TILE = 64


def _as_index_tensor(values, device: torch.device) -> torch.Tensor:
    if isinstance(values, torch.Tensor):
        tensor = values.to(device=device, dtype=torch.long)
    else:
        tensor = torch.as_tensor(list(values), dtype=torch.long, device=device)
    return tensor


def _check_cache_pair(k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    if k_cache.ndim != 4 or v_cache.ndim != 4:
        raise ValueError(
            "k_cache and v_cache must have shape [num_blocks, block_size, Hkv, D]"
        )
    if k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must have the same shape")


def _require_kernel_layout(q: torch.Tensor, k_cache: torch.Tensor,
                           v_cache: torch.Tensor, what: str) -> None:
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError(f"{what}: k_cache and v_cache must be contiguous block pools")
    if q.dtype != k_cache.dtype or v_cache.dtype != k_cache.dtype:
        raise TypeError(f"{what}: q, k_cache and v_cache must share one dtype")


# Decode workspaces by (device, stream): zero-filled when allocated. The
# decode kernels exchange split partials through the workspace, a zero word
# meaning "not written yet"; it must be zero when a call starts, and every
# call leaves it zero. One workspace per stream keeps calls on different
# streams from sharing partials. A workspace that a larger one replaces stays
# allocated (in _RETIRED) for the life of the process: a graph captured
# earlier may still replay on its address.
_WORKSPACES: dict = {}
_RETIRED: list = []


class DecodeMergeError(RuntimeError):
    """A decode workspace's merge-failure flag was set: the multi-split
    decode outputs computed on it since the failure are NaN. The workspace
    has been cleared and is usable again."""


def decode_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A zero-initialised decode workspace of at least `nbytes` for the
    current stream of `device`, reused across calls.

    Under graph capture the cached workspace is used as it is: allocating or
    growing one there would only record its zero fill into the graph (the
    memory would hold garbage until the first replay), so that case raises
    and asks for an eager call of the same size first, or an explicit
    workspace.
    """
    stream = torch.cuda.current_stream(device).cuda_stream
    key = (device.index, stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            have = 0 if ws is None else ws.numel()
            raise RuntimeError(
                f"paged decode under graph capture needs a {nbytes}-byte decode workspace "
                f"for this stream and the cached one has {have} bytes; run one eager call "
                "of the same size on this stream before capturing, or pass workspace=")
        if ws is not None:
            _RETIRED.append(ws)
        ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def check_workspace(workspace: torch.Tensor) -> None:
    """Raise DecodeMergeError when `workspace`'s merge-failure flag is set
    (after clearing the workspace); synchronises torch's current stream and
    must run outside graph capture (mlr_paged_decode_workspace_check). Work
    that other streams queued on the workspace must have finished first
    (check_decode_workspaces synchronises the device for that)."""
    lib = _lib.load()
    device = workspace.device
    with torch.cuda.device(device):
        status = lib.mlr_paged_decode_workspace_check(
            workspace.data_ptr(), workspace.numel(), _lib.stream_handle(device))
    if status == _lib.MLR_ERR_MERGE:
        raise DecodeMergeError(lib.mlr_last_error().decode(errors="replace"))
    _lib.check(status, "mlr_paged_decode_workspace_check")


def check_decode_workspaces(device: torch.device | None = None) -> None:
    """Check every cached decode workspace (of `device`, or of all devices)
    for a merge failure, once the work queued on them has finished; raises
    DecodeMergeError if any flag was set, after clearing every flagged
    workspace. The model runner calls this once per step."""
    failures = []
    cached = [ws for (index, _stream), ws in list(_WORKSPACES.items())
              if device is None or index == device.index]
    for dev in {ws.device for ws in cached}:
        torch.cuda.synchronize(dev)  # the workspaces' own streams included
    for ws in cached:
        try:
            check_workspace(ws)
        except DecodeMergeError as exc:
            failures.append(str(exc))
    if failures:
        raise DecodeMergeError("; ".join(failures))


def decode_workspace_bytes(batch: int, num_q_heads: int, head_dim: int,
                           max_context: int, dtype: torch.dtype,
                           tokens_per_split: int = 0) -> int:
    lib = _lib.load()
    return int(lib.mlr_paged_decode_workspace_size(
        batch, num_q_heads, head_dim, max_context, tokens_per_split,
        _lib.dtype_code(dtype, "paged decode")))


def paged_decode_launch(q: torch.Tensor, k_cache: torch.Tensor,
                        v_cache: torch.Tensor, block_tables: torch.Tensor,
                        seq_lens: torch.Tensor, out: torch.Tensor | None = None,
                        *, scale: float | None = None, tokens_per_split: int = 0,
                        workspace: torch.Tensor | None = None,
                        new_k: torch.Tensor | None = None,
                        new_v: torch.Tensor | None = None,
                        slot_mapping: torch.Tensor | None = None) -> torch.Tensor:
    """Launch the split-KV decode on already-validated device operands.

    q [B, Hq, D]; k_cache/v_cache one contiguous layer [NB, BS, Hkv, D];
    block_tables [B, W] int64; seq_lens [B] int64, each in [1, W * BS].
    With new_k/new_v [B, Hkv, D] (cache dtype) and slot_mapping [B] int64, the
    decode step's KV write happens in the same call (mlr_paged_decode_append):
    slot_mapping[b] must be the slot of position seq_lens[b] - 1.
    A caller-provided `workspace` (uint8, at least decode_workspace_bytes)
    must be all-zero before its first use; each call leaves it reusable.
    Calls that share a workspace must not overlap.
    """
    device = _lib.require_hip(q, k_cache, v_cache, block_tables, seq_lens,
                              what="paged decode")
    lib = _lib.load()
    batch, num_q_heads, head_dim = q.shape
    num_blocks, block_size, num_kv_heads, _ = k_cache.shape
    if q.stride(-1) != 1:
        q = q.contiguous()
    if block_tables.dtype != torch.long:
        block_tables = block_tables.to(torch.long)
    if seq_lens.dtype != torch.long:
        seq_lens = seq_lens.to(torch.long)
    if block_tables.stride(-1) != 1:
        block_tables = block_tables.contiguous()
    seq_lens = seq_lens.contiguous()
    width = block_tables.shape[1]
    if out is None:
        out = torch.empty((batch, num_q_heads, head_dim), dtype=q.dtype, device=device)
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    dcode = _lib.dtype_code(q.dtype, "paged decode")
    ws_bytes = int(lib.mlr_paged_decode_workspace_size(
        batch, num_q_heads, head_dim, width * block_size, tokens_per_split, dcode))
    if workspace is None:
        workspace = decode_workspace(device, ws_bytes)
    elif workspace.numel() < ws_bytes:
        raise ValueError(f"decode workspace of {workspace.numel()} bytes is smaller than "
                         f"the {ws_bytes} bytes required")
    stream = _lib.stream_handle(device)
    common = (q.data_ptr(), q.stride(0), q.stride(1),
              k_cache.data_ptr(), v_cache.data_ptr(),
              num_blocks, block_size, num_kv_heads, head_dim,
              block_tables.data_ptr(), block_tables.stride(0), width,
              seq_lens.data_ptr(), batch, num_q_heads, float(scale), dcode,
              int(tokens_per_split), workspace.data_ptr(), workspace.numel())
    tail = (out.data_ptr(), out.stride(0), out.stride(1), stream)
    if new_k is None:
        with torch.cuda.device(device):
            status = lib.mlr_paged_decode(*common, *tail)
        _lib.check(status, "mlr_paged_decode")
        return out
    if new_k.dtype != k_cache.dtype or new_v.dtype != k_cache.dtype:
        new_k, new_v = new_k.to(k_cache.dtype), new_v.to(k_cache.dtype)
    if new_k.stride(-1) != 1 or new_k.stride() != new_v.stride():
        new_k, new_v = new_k.contiguous(), new_v.contiguous()
    slot_mapping = slot_mapping.to(torch.long).contiguous()
    with torch.cuda.device(device):
        status = lib.mlr_paged_decode_append(
            *common, new_k.data_ptr(), new_v.data_ptr(), new_k.stride(0),
            new_k.stride(1), slot_mapping.data_ptr(), *tail)
    _lib.check(status, "mlr_paged_decode_append")
    return out


def paged_attention_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: list[int],
    seq_len: int,
    block_size: int,
) -> torch.Tensor:
    """Single-request paged decode: q [Hq, D] -> [Hq, D].

    Reference: kernels/reference/paged_attention.py:6-105 (same validation).
    """
    if q.ndim != 2:
        raise ValueError("q must have shape [Hq, D]")
    _check_cache_pair(k_cache, v_cache)
    num_query_heads, head_dim = q.shape
    num_kv_heads = k_cache.shape[2]
    if head_dim != k_cache.shape[-1]:
        raise ValueError("q and KV cache must have the same head_dim")
    if num_query_heads % num_kv_heads != 0:
        raise ValueError("num_query_heads must be divisible by num_kv_heads")
    if seq_len <= 0:
        raise ValueError("seq_len must be greater than 0")
    required_blocks = (seq_len + block_size - 1) // block_size
    if len(block_table) < required_blocks:
        raise ValueError("block_table does not contain enough blocks for seq_len")
    if block_size != k_cache.shape[1]:
        raise ValueError("block_size does not match KV cache layout")
    used = [int(b) for b in list(block_table)[:required_blocks]]
    if any(b < 0 or b >= k_cache.shape[0] for b in used):
        raise ValueError("block_table contains an out-of-range physical block")
    _require_kernel_layout(q, k_cache, v_cache, "paged_attention_decode")
    device = _lib.require_hip(q, k_cache, v_cache, what="paged_attention_decode")
    table = torch.tensor([used], dtype=torch.long, device=device)
    lens = torch.tensor([seq_len], dtype=torch.long, device=device)
    out = paged_decode_launch(q.unsqueeze(0), k_cache, v_cache, table, lens)
    return out.squeeze(0)


def paged_attention_decode_batch_reference(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: list[list[int]],
    seq_lens: list[int],
    block_size: int,
) -> torch.Tensor:
    """Per-request loop over paged_attention_decode (reference :109-176)."""
    if q.ndim != 3:
        raise ValueError("q must have shape [B, Hq, D]")
    _check_cache_pair(k_cache, v_cache)
    num_query_heads, head_dim = q.shape[1], q.shape[-1]
    num_kv_heads = k_cache.shape[2]
    if head_dim != k_cache.shape[-1]:
        raise ValueError("q and KV cache must have the same head_dim")
    if num_query_heads % num_kv_heads != 0:
        raise ValueError("num_query_heads must be divisible by num_kv_heads")
    if len(block_tables) != q.shape[0]:
        raise ValueError("block_tables length must match batch size of q")
    if len(seq_lens) != q.shape[0]:
        raise ValueError("seq_lens length must match batch size of q")
    for i in range(q.shape[0]):
        required_blocks = (seq_lens[i] + block_size - 1) // block_size
        if len(block_tables[i]) < required_blocks:
            raise ValueError(
                f"block_table for batch {i} does not contain enough blocks "
                f"for seq_len {seq_lens[i]}")
    return torch.stack([
        paged_attention_decode(q[i], k_cache, v_cache, block_tables[i],
                               seq_lens[i], block_size)
        for i in range(q.shape[0])
    ], dim=0)


def paged_attention_decode_batch_parallel(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    block_size: int,
    *,
    validate: bool = True,
    tokens_per_split: int = 0,
) -> torch.Tensor:
    """Batched paged decode: q [B, Hq, D] -> [B, Hq, D].

    Reference: kernels/reference/paged_attention.py:178-254 (same validation
    messages). ``block_tables`` rows are -1-padded; only the first
    ceil(seq_len / block_size) entries of a row are read. With validate=True
    (default) one host sync checks that every row covers its sequence with
    in-range block ids, the condition under which the reference's gather is
    defined; callers that validated the step's metadata already pass False.
    """
    if q.ndim != 3:
        raise ValueError("q must have shape [B, Hq, D]")
    _check_cache_pair(k_cache, v_cache)
    num_query_heads, head_dim = q.shape[1], q.shape[-1]
    num_kv_heads = k_cache.shape[2]
    if head_dim != k_cache.shape[-1]:
        raise ValueError("q and KV cache must have the same head_dim")
    if num_query_heads % num_kv_heads != 0:
        raise ValueError("num_query_heads must be divisible by num_kv_heads")
    if len(block_tables) != q.shape[0]:
        raise ValueError("block_tables length must match batch size of q")
    if len(seq_lens) != q.shape[0]:
        raise ValueError("seq_lens length must match batch size of q")
    if block_size != k_cache.shape[1]:
        raise ValueError("block_size does not match KV cache layout")
    _require_kernel_layout(q, k_cache, v_cache, "paged_attention_decode_batch_parallel")
    device = _lib.require_hip(q, k_cache, v_cache,
                              what="paged_attention_decode_batch_parallel")
    block_tables = _as_index_tensor(block_tables, device)
    seq_lens = _as_index_tensor(seq_lens, device)
    if block_tables.ndim != 2:
        raise ValueError("block_tables must have shape [B, max_num_blocks]")
    if validate:
        _validate_tables(block_tables, seq_lens, block_size, k_cache.shape[0])
    return paged_decode_launch(q, k_cache, v_cache, block_tables, seq_lens,
                               tokens_per_split=tokens_per_split)


def _validate_tables(block_tables: torch.Tensor, seq_lens: torch.Tensor,
                     block_size: int, num_blocks: int) -> None:
    """One device reduction and one host sync for all table checks."""
    width = block_tables.shape[1]
    required = (seq_lens + block_size - 1) // block_size
    columns = torch.arange(width, device=block_tables.device)
    used = columns[None, :] < required[:, None]
    bad_ids = used & ((block_tables < 0) | (block_tables >= num_blocks))
    flags = torch.stack([
        (seq_lens <= 0).any(),
        (required > width).any(),
        bad_ids.any(),
    ]).cpu()
    if bool(flags[0]):
        raise ValueError("seq_lens must be greater than 0")
    if bool(flags[1]):
        raise ValueError("block_tables have insufficient blocks for seq_lens")
    if bool(flags[2]):
        raise ValueError("block_tables contain an invalid physical block")


def paged_prefill_launch(q: torch.Tensor, k_cache: torch.Tensor,
                         v_cache: torch.Tensor, block_tables: torch.Tensor,
                         query_start_loc: torch.Tensor, context_lens: torch.Tensor,
                         max_query_len: int, *, tile_size: int = _DEFAULT_TILE,
                         scale: float | None = None,
                         out: torch.Tensor | None = None) -> torch.Tensor:
    """Varlen chunk prefill on already-validated device operands.

    q [total_q, Hq, D]; block_tables [S, W] int64; query_start_loc [S+1] and
    context_lens [S] int64. The chunk keys must already be in the cache.
    """
    device = _lib.require_hip(q, k_cache, v_cache, block_tables, query_start_loc,
                              context_lens, what="paged prefill")
    lib = _lib.load()
    total_q, num_q_heads, head_dim = q.shape
    num_blocks, block_size, num_kv_heads, _ = k_cache.shape
    if q.stride(-1) != 1:
        q = q.contiguous()
    block_tables = block_tables.to(torch.long).contiguous()
    query_start_loc = query_start_loc.to(torch.long).contiguous()
    context_lens = context_lens.to(torch.long).contiguous()
    if out is None:
        out = torch.empty((total_q, num_q_heads, head_dim), dtype=q.dtype, device=device)
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    if total_q == 0:
        return out
    with torch.cuda.device(device):
        status = lib.mlr_paged_prefill(
            q.data_ptr(), q.stride(0), q.stride(1),
            k_cache.data_ptr(), v_cache.data_ptr(),
            num_blocks, block_size, num_kv_heads, head_dim,
            block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1],
            query_start_loc.data_ptr(), context_lens.data_ptr(),
            context_lens.shape[0], int(max_query_len), num_q_heads, float(scale),
            _lib.dtype_code(q.dtype, "paged prefill"), int(tile_size),
            out.data_ptr(), out.stride(0), out.stride(1),
            _lib.stream_handle(device))
    _lib.check(status, "mlr_paged_prefill")
    return out


def paged_attention_prefill_chunk_tiled(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: Sequence[int] | torch.Tensor,
    prefix_len: int,
    context_len: int,
    block_size: int,
    tile_size: int,
) -> torch.Tensor:
    """Chunk prefill for one sequence: q [C, Hq, D] -> [C, Hq, D].

    Reference: kernels/reference/paged_attention.py:346-434 (same validation).
    Keys [0, context_len) of the sequence must already be in the cache.
    """
    if tile_size <= 0:
        raise ValueError("tile_size must be greater than 0")
    if context_len != prefix_len + q.shape[0]:
        raise ValueError("context_len must equal prefix_len + q.shape[0]")
    q_num_heads = q.shape[1]
    kv_num_heads = k_cache.shape[2]
    if q_num_heads % kv_num_heads != 0:
        raise ValueError("q_num_heads must be divisible by kv_num_heads")
    if q.ndim != 3:
        raise ValueError("q must have shape [chunk_len, Hq, D]")
    _check_cache_pair(k_cache, v_cache)
    if q.shape[-1] != k_cache.shape[-1]:
        raise ValueError("q and KV cache must have the same head_dim")
    if block_size != k_cache.shape[1]:
        raise ValueError("block_size does not match KV cache layout")
    if prefix_len < 0:
        raise ValueError("prefix_len cannot be negative")
    _require_kernel_layout(q, k_cache, v_cache, "paged_attention_prefill_chunk_tiled")
    device = _lib.require_hip(q, k_cache, v_cache,
                              what="paged_attention_prefill_chunk_tiled")
    chunk_len = q.shape[0]
    if chunk_len == 0:
        return torch.empty_like(q)
    required_blocks = (context_len + block_size - 1) // block_size
    if isinstance(block_table, torch.Tensor):
        table = block_table.to(device=device, dtype=torch.long).reshape(-1)
        if table.numel() < required_blocks:
            raise IndexError("block_table does not cover context_len")
        used = table[:required_blocks]
        if bool(((used < 0) | (used >= k_cache.shape[0])).any().cpu()):
            raise ValueError("block_table contains an out-of-range physical block")
    else:
        entries = [int(b) for b in block_table]
        if len(entries) < required_blocks:
            raise IndexError("block_table does not cover context_len")
        if any(b < 0 or b >= k_cache.shape[0] for b in entries[:required_blocks]):
            raise ValueError("block_table contains an out-of-range physical block")
        table = torch.tensor(entries[:required_blocks], dtype=torch.long, device=device)
    table = table.contiguous()
    lib = _lib.load()
    if q.stride(-1) != 1:
        q = q.contiguous()
    out = torch.empty_like(q, memory_format=torch.contiguous_format)
    num_blocks, _, num_kv_heads, head_dim = k_cache.shape
    with torch.cuda.device(device):
        status = lib.mlr_paged_prefill_chunk(
            q.data_ptr(), q.stride(0), q.stride(1),
            k_cache.data_ptr(), v_cache.data_ptr(),
            num_blocks, block_size, num_kv_heads, head_dim,
            table.data_ptr(), table.numel(), int(prefix_len), int(context_len),
            q_num_heads, 1.0 / math.sqrt(head_dim),
            _lib.dtype_code(q.dtype, "paged_attention_prefill_chunk_tiled"),
            int(tile_size), out.data_ptr(), out.stride(0), out.stride(1),
            _lib.stream_handle(device))
    _lib.check(status, "mlr_paged_prefill_chunk")
    return out


def paged_attention_prefill_varlen(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    query_start_loc: torch.Tensor,
    context_lens: torch.Tensor,
    block_size: int,
    tile_size: int = _DEFAULT_TILE,
    *,
    max_query_len: int | None = None,
) -> torch.Tensor:
    """Chunk prefill for a packed batch (ModelBatch layout, one launch).

    q [total_q, Hq, D] holds sequence s's rows at
    [query_start_loc[s], query_start_loc[s+1]); its prefix length is
    context_lens[s] - query_len_s. No reference counterpart: the reference runs
    chunk prefill one sequence at a time (kernels/reference/paged_attention.py
    :346-434); this is the packed form of the same computation.
    """
    if q.ndim != 3:
        raise ValueError("q must have shape [total_tokens, Hq, D]")
    _check_cache_pair(k_cache, v_cache)
    if block_size != k_cache.shape[1]:
        raise ValueError("block_size does not match KV cache layout")
    if q.shape[1] % k_cache.shape[2] != 0:
        raise ValueError("q_num_heads must be divisible by kv_num_heads")
    if tile_size <= 0:
        raise ValueError("tile_size must be greater than 0")
    _require_kernel_layout(q, k_cache, v_cache, "paged_attention_prefill_varlen")
    device = _lib.require_hip(q, k_cache, v_cache,
                              what="paged_attention_prefill_varlen")
    block_tables = _as_index_tensor(block_tables, device)
    query_start_loc = _as_index_tensor(query_start_loc, device)
    context_lens = _as_index_tensor(context_lens, device)
    qlens = query_start_loc[1:] - query_start_loc[:-1]
    if max_query_len is None:
        max_query_len = int(qlens.max().item()) if qlens.numel() else 0
    return paged_prefill_launch(q, k_cache, v_cache, block_tables, query_start_loc,
                                context_lens, max_query_len, tile_size=tile_size)


def paged_kv_read_floor(k_cache: torch.Tensor, v_cache: torch.Tensor,
                        block_tables: torch.Tensor, context_lens: torch.Tensor,
                        tokens_per_item: int = 320,
                        out: torch.Tensor | None = None) -> torch.Tensor:
    """Diagnostic (no reference counterpart): read every context token's K and
    V slot row through the block table and return the XOR checksums of the
    32-bit words read, one int32 per (sequence, item of `tokens_per_item`
    tokens). The time of this call is the memory floor of a decode step on
    the same block list. Operands as for paged_decode_launch."""
    device = _lib.require_hip(k_cache, v_cache, block_tables, context_lens,
                              what="paged KV read floor")
    lib = _lib.load()
    num_blocks, block_size = k_cache.shape[0], k_cache.shape[1]
    row_bytes = k_cache[0, 0].numel() * k_cache.element_size()
    block_tables = block_tables.to(torch.long).contiguous()
    context_lens = context_lens.to(torch.long).contiguous()
    batch, width = block_tables.shape
    n = int(lib.mlr_paged_kv_read_floor_outputs(batch, width, block_size, tokens_per_item))
    if out is None:
        out = torch.empty(max(n, 1), dtype=torch.int32, device=device)
    with torch.cuda.device(device):
        status = lib.mlr_paged_kv_read_floor(
            k_cache.data_ptr(), v_cache.data_ptr(), num_blocks, block_size, row_bytes,
            block_tables.data_ptr(), block_tables.stride(0), width, context_lens.data_ptr(),
            batch, tokens_per_item, out.data_ptr(), out.numel(), _lib.stream_handle(device))
    _lib.check(status, "mlr_paged_kv_read_floor")
    return out
