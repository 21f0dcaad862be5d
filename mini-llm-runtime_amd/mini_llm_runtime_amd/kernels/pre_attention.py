"""Fused pre-attention step: projection bias, rotary embedding, KV-cache write.

``qkv_rope_write`` takes the output of one QKV projection GEMM over the
concatenated [q | k | v] weights and, in one launch (``mlr_qkv_rope_write``),
adds the optional bias, rotates the q and k heads at their positions, returns
the rotated q and writes k and v into one layer of the paged cache. It
replaces the reference's per-layer sequence Qwen2RotaryEmbedding ->
apply_rotary_pos_emb -> kv_cache.write_slots (model/qwen2.py:125-209,
:605-613, :737-746), with the same rounding in the model dtype.

``qkv_rope_decode`` goes one step further for a decode step: the same
rotation and KV write and the batched paged decode in one launch
(``mlr_paged_decode_qkv``).

Checks are on shapes, dtypes and devices only; slot values are the caller's
to validate (``PagedKVCache.check_slots`` runs the reference's write_slots
checks). A slot outside the pool is not written.
"""

from __future__ import annotations

import torch

from .. import _lib
from ..runtime.paged_kv_cache import PagedKVCache
from . import paged_attention as kpa

_SUPPORTED = (torch.float32, torch.float16, torch.bfloat16)

# FP32 copies of rotary inv_freq buffers held in another dtype (a model cast
# to bf16 casts its buffers), so that a call does not launch a conversion.
# An entry keeps its source tensor alive, so the source's storage cannot be
# reused while cached, and records the source's version counter, so an
# in-place change of the buffer is seen.
_FREQ32: dict = {}
_FREQ32_MAX = 64


def _freq_fp32(inv_freq: torch.Tensor) -> torch.Tensor:
    if inv_freq.dtype == torch.float32 and inv_freq.is_contiguous():
        return inv_freq
    key = (inv_freq.data_ptr(), inv_freq.dtype, inv_freq.device, inv_freq.stride())
    hit = _FREQ32.get(key)
    if hit is not None and hit[0] is inv_freq and hit[1] == inv_freq._version:
        return hit[2]
    freq = inv_freq.to(torch.float32).contiguous()
    if len(_FREQ32) >= _FREQ32_MAX:
        _FREQ32.clear()
    _FREQ32[key] = (inv_freq, inv_freq._version, freq)
    return freq


def qkv_rope_write(qkv: torch.Tensor, positions: torch.Tensor, inv_freq: torch.Tensor,
                   kv_cache: PagedKVCache, layer_idx: int, slot_mapping: torch.Tensor,
                   num_q_heads: int, *, bias: torch.Tensor | None = None,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """qkv [T, (Hq + 2 Hkv) * D] -> rotated q [T, Hq, D]; k, v to the cache.

    positions: int64 [T]; inv_freq: the rotary module's buffer [D / 2] (used
    as FP32, exactly as the reference promotes it); slot_mapping int32/int64
    [T]; bias [(Hq + 2 Hkv) * D] or None.
    """
    if layer_idx < 0 or layer_idx >= kv_cache.num_layers:
        raise IndexError("Unexpected layer_idx")
    hkv, d = kv_cache.num_kv_heads, kv_cache.head_dim
    if num_q_heads <= 0 or num_q_heads % hkv != 0:
        raise ValueError("num_q_heads must be a positive multiple of the cache's KV heads")
    width = (num_q_heads + 2 * hkv) * d
    if qkv.ndim != 2 or qkv.shape[1] != width:
        raise ValueError(f"qkv must have shape [num_tokens, {width}], got {tuple(qkv.shape)}")
    if qkv.shape[0] > 0 and qkv.stride(1) != 1:
        raise ValueError("qkv rows must be contiguous")
    tokens = qkv.shape[0]
    if positions.shape != (tokens,) or positions.dtype != torch.long:
        raise ValueError("positions must be an int64 tensor of shape [num_tokens]")
    if slot_mapping.shape != (tokens,):
        raise ValueError("slot_mapping must have shape [num_tokens]")
    if slot_mapping.dtype not in (torch.int32, torch.int64):
        raise TypeError("slot_mapping must use an integer index dtype")
    if inv_freq.shape != (d // 2,):
        raise ValueError(f"inv_freq must have shape [{d // 2}]")
    if qkv.dtype not in _SUPPORTED:
        raise TypeError(f"qkv dtype {qkv.dtype} is not supported")
    if qkv.dtype != kv_cache.dtype:
        raise TypeError("qkv dtype must match the KV cache dtype")
    if bias is not None and (bias.shape != (width,) or bias.dtype != qkv.dtype):
        raise ValueError(f"bias must have shape [{width}] and the qkv dtype")
    if out is None:
        out = torch.empty((tokens, num_q_heads, d), dtype=qkv.dtype, device=qkv.device)
    elif (out.shape != (tokens, num_q_heads, d) or out.dtype != qkv.dtype
          or (tokens > 0 and (out.stride(2) != 1 or out.stride(1) != d))):
        raise ValueError("out must be [num_tokens, num_q_heads, head_dim] with contiguous heads")
    tensors = [qkv, positions, inv_freq, slot_mapping, out, kv_cache.k_cache]
    if bias is not None:
        tensors.append(bias)
    device = _lib.require_hip(*tensors, what="qkv_rope_write")
    if tokens == 0:
        return out
    layer_k, layer_v = kv_cache.get_layer_cache(layer_idx)
    if not (layer_k.is_contiguous() and layer_v.is_contiguous()):
        raise ValueError("KV cache layers must be contiguous")
    freq = _freq_fp32(inv_freq)
    bias_c = bias.contiguous() if bias is not None else None
    lib = _lib.load()
    with torch.cuda.device(device):
        status = lib.mlr_qkv_rope_write(
            qkv.data_ptr(), qkv.stride(0), bias_c.data_ptr() if bias_c is not None else None,
            positions.data_ptr(), freq.data_ptr(), slot_mapping.data_ptr(),
            _lib.INDEX_CODES[slot_mapping.dtype], out.data_ptr(), out.stride(0),
            layer_k.data_ptr(), layer_v.data_ptr(), kv_cache.num_blocks * kv_cache.block_size,
            tokens, num_q_heads, hkv, d, _lib.dtype_code(qkv.dtype, "qkv_rope_write"),
            _lib.stream_handle(device))
    _lib.check(status, "mlr_qkv_rope_write")
    return out


def qkv_rope_decode_fusable(qkv_dtype: torch.dtype, kv_cache: PagedKVCache,
                            num_q_heads: int) -> bool:
    """Shapes ``qkv_rope_decode`` covers: bf16 or fp16, head_dim 64 or 128, at
    most 16 query heads per KV head, block_size a multiple of 16, the cache in
    the model dtype. Other shapes run qkv_rope_write and then the decode."""
    hkv = kv_cache.num_kv_heads
    return (qkv_dtype in (torch.bfloat16, torch.float16) and kv_cache.dtype == qkv_dtype
            and kv_cache.head_dim in (64, 128) and num_q_heads % hkv == 0
            and 0 < num_q_heads // hkv <= 16 and kv_cache.block_size % 16 == 0)


def qkv_rope_decode(qkv: torch.Tensor, inv_freq: torch.Tensor, kv_cache: PagedKVCache,
                    layer_idx: int, slot_mapping: torch.Tensor, block_tables: torch.Tensor,
                    context_lens: torch.Tensor, num_q_heads: int, *,
                    out: torch.Tensor | None = None,
                    scale: float | None = None, tokens_per_split: int = 0,
                    workspace: torch.Tensor | None = None) -> torch.Tensor:
    """One decode step of a layer after its QKV projection, in one launch
    (``mlr_paged_decode_qkv``): qkv [B, (Hq + 2 Hkv) * D], the projection's
    output with its bias -> attention output [B, Hq, D]; the rotated k and v
    of each request are written to slot_mapping[b] of the layer's cache on
    the way.

    Each request's token sits at position context_lens[b] - 1 and
    slot_mapping[b] is that position's slot; the caller validates this
    metadata (Qwen2Attention does, with the reference's checks). Results equal
    ``qkv_rope_write`` at those positions (without its bias) followed by the
    batched decode bit for bit. Only shapes ``qkv_rope_decode_fusable`` accepts.
    """
    if layer_idx < 0 or layer_idx >= kv_cache.num_layers:
        raise IndexError("Unexpected layer_idx")
    hkv, d = kv_cache.num_kv_heads, kv_cache.head_dim
    if not qkv_rope_decode_fusable(qkv.dtype, kv_cache, num_q_heads):
        raise ValueError("qkv_rope_decode needs bf16 or fp16, head_dim 64 or 128, at most 16 query "
                         "heads per KV head and a block_size multiple of 16")
    width = (num_q_heads + 2 * hkv) * d
    if qkv.ndim != 2 or qkv.shape[1] != width or qkv.shape[0] == 0:
        raise ValueError(f"qkv must have shape [batch, {width}] with batch > 0, "
                         f"got {tuple(qkv.shape)}")
    batch = qkv.shape[0]
    if qkv.stride(1) != 1 or qkv.stride(0) % 8 != 0 or qkv.data_ptr() % 16 != 0:
        # The kernel reads 16-byte aligned row chunks; a fresh copy is aligned.
        qkv = qkv.clone(memory_format=torch.contiguous_format)
    if inv_freq.shape != (d // 2,):
        raise ValueError(f"inv_freq must have shape [{d // 2}]")
    for name, tensor in (("slot_mapping", slot_mapping), ("context_lens", context_lens)):
        if tensor.shape != (batch,) or tensor.dtype != torch.long:
            raise ValueError(f"{name} must be an int64 tensor of shape [batch]")
    if (block_tables.ndim != 2 or block_tables.shape[0] != batch
            or block_tables.dtype != torch.long):
        raise ValueError("block_tables must be an int64 tensor of shape [batch, max_blocks]")
    device = _lib.require_hip(qkv, inv_freq, slot_mapping, context_lens, block_tables,
                              kv_cache.k_cache, what="qkv_rope_decode")
    layer_k, layer_v = kv_cache.get_layer_cache(layer_idx)
    if not (layer_k.is_contiguous() and layer_v.is_contiguous()):
        raise ValueError("KV cache layers must be contiguous")
    if out is None:
        out = torch.empty((batch, num_q_heads, d), dtype=qkv.dtype, device=device)
    elif out.shape != (batch, num_q_heads, d) or out.dtype != qkv.dtype or out.stride(2) != 1:
        raise ValueError("out must be [batch, num_q_heads, head_dim] with contiguous rows")
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    slot_mapping, context_lens = slot_mapping.contiguous(), context_lens.contiguous()
    freq = _freq_fp32(inv_freq)
    width_blocks = block_tables.shape[1]
    if scale is None:
        scale = d ** -0.5
    dcode = _lib.dtype_code(qkv.dtype, "qkv_rope_decode")
    lib = _lib.load()
    ws_bytes = int(lib.mlr_paged_decode_workspace_size(
        batch, num_q_heads, d, width_blocks * kv_cache.block_size, tokens_per_split, dcode))
    if workspace is None:
        workspace = kpa.decode_workspace(device, ws_bytes)
    elif workspace.numel() < ws_bytes:
        raise ValueError(f"decode workspace of {workspace.numel()} bytes is smaller than "
                         f"the {ws_bytes} bytes required")
    with torch.cuda.device(device):
        status = lib.mlr_paged_decode_qkv(
            qkv.data_ptr(), qkv.stride(0), freq.data_ptr(), layer_k.data_ptr(), layer_v.data_ptr(), kv_cache.num_blocks,
            kv_cache.block_size, hkv, d, block_tables.data_ptr(), block_tables.stride(0),
            width_blocks, context_lens.data_ptr(), slot_mapping.data_ptr(), batch,
            num_q_heads, float(scale), dcode, int(tokens_per_split), workspace.data_ptr(),
            workspace.numel(), out.data_ptr(), out.stride(0), out.stride(1),
            _lib.stream_handle(device))
    _lib.check(status, "mlr_paged_decode_qkv")
    return out
