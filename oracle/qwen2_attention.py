"""CPU restatement of the reference's Qwen2 attention callers (oracle; tests only).

Follows src/mini_llm_runtime/model/qwen2.py:
- rotary embedding (:125-170): inv_freq = 1 / theta^(2i/D), angles
  position * inv_freq duplicated over both halves, cos/sin cast to the
  activation dtype; rotate_half and apply_rotary_pos_emb (:173-209);
- q/k/v projections with bias and the bias-free o_proj (:211-236, :276-280);
- forward_prefill_with_cache (:372-439): write the prompt's K/V, dense causal
  attention (:323-370) over the fresh K/V;
- forward_decode_with_cache (:441-536): write, single-request paged decode;
- forward_decode_batch_with_cache (:538-622): write, batched paged decode;
- forward_prefill_chunk_with_cache (:624-767): write, tiled chunk prefill.
Validation is not restated here (the product's messages are tested on their
own); these functions compute what the reference computes for valid input.

Weights are a dict of tensors: q_w [Hq*D, H], q_b, k_w [Hkv*D, H], k_b, v_w,
v_b, o_w [H, H]. Pinned by tests/test_oracle_pins.py against a float64
textbook (RoPE as a rotation of the pairs (x_i, x_{i+D/2}) by position *
theta^(-2i/D), then textbook attention).
"""

from __future__ import annotations

import torch

from . import paged_attention as pa


def rope_tables(positions: torch.Tensor, head_dim: int, theta: float, dtype,
                freq_dtype: torch.dtype | None = None):
    """cos, sin [..., D] for integer positions (reference :125-170).

    inv_freq is an FP32 buffer of the rotary module (:135-141); a module cast
    with .to(freq_dtype) holds it rounded to that dtype, and the FP32
    positions then multiply the rounded values (type promotion, :164-167)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    if freq_dtype is not None:
        inv_freq = inv_freq.to(freq_dtype).to(torch.float32)
    angles = positions.to(torch.float32).unsqueeze(-1) * inv_freq
    angles = torch.cat((angles, angles), dim=-1)
    return angles.cos().to(dtype), angles.sin().to(dtype)


def rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [..., heads, D] rotated with cos/sin [..., D] (reference :173-209)."""
    half = x.shape[-1] // 2
    turned = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * cos.to(x.dtype).unsqueeze(-2) + turned * sin.to(x.dtype).unsqueeze(-2)


def project(hidden: torch.Tensor, w: dict, hq: int, hkv: int, d: int):
    lead = hidden.shape[:-1]
    q = torch.nn.functional.linear(hidden, w["q_w"], w["q_b"]).reshape(lead + (hq, d))
    k = torch.nn.functional.linear(hidden, w["k_w"], w["k_b"]).reshape(lead + (hkv, d))
    v = torch.nn.functional.linear(hidden, w["v_w"], w["v_b"]).reshape(lead + (hkv, d))
    return q, k, v


def qkv_rope(hidden, positions, w, hq, hkv, d, theta, freq_dtype=None):
    q, k, v = project(hidden, w, hq, hkv, d)
    cos, sin = rope_tables(positions, d, theta, hidden.dtype, freq_dtype)
    return rotate(q, cos, sin), rotate(k, cos, sin), v


def _unpack(cfg):
    """cfg = (hq, hkv, d, theta) or (hq, hkv, d, theta, freq_dtype): the last
    is the dtype the rotary module was cast to (None or absent: FP32)."""
    hq, hkv, d, theta, *rest = cfg
    return hq, hkv, d, theta, (rest[0] if rest else None)


def dense_causal(q, k, v, scale):
    """[1, S, Hq, D] x [1, S, Hkv, D] causal attention (reference :323-370)."""
    group = q.shape[-2] // k.shape[-2]
    k = k.repeat_interleave(group, dim=-2)
    v = v.repeat_interleave(group, dim=-2)
    s = q.shape[1]
    qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    scores = (qt @ kt.transpose(-2, -1)) * scale
    scores = scores.masked_fill(~torch.tril(torch.ones(s, s, dtype=torch.bool)), float("-inf"))
    sm = torch.float32 if scores.dtype in (torch.float16, torch.bfloat16) else scores.dtype
    weights = torch.softmax(scores, dim=-1, dtype=sm).to(vt.dtype)
    out = (weights @ vt).transpose(1, 2)
    return out.reshape(out.shape[0], s, -1)


def prefill_whole(hidden, positions, cache, layer, slots, w, cfg):
    hq, hkv, d, theta, fdt = _unpack(cfg)
    q, k, v = qkv_rope(hidden, positions, w, hq, hkv, d, theta, fdt)
    cache.write_slots(slots, k.squeeze(0), v.squeeze(0), layer)
    out = dense_causal(q, k, v, d ** -0.5)
    return torch.nn.functional.linear(out, w["o_w"])


def decode_single(hidden, positions, cache, layer, slots, block_table, context_len, w, cfg):
    hq, hkv, d, theta, fdt = _unpack(cfg)
    q, k, v = qkv_rope(hidden, positions, w, hq, hkv, d, theta, fdt)
    cache.write_slots(slots, k.squeeze(1), v.squeeze(1), layer)
    kc, vc = cache.get_layer_cache(layer)
    out = pa.decode_single(q[0, 0], kc, vc, block_table, context_len, cache.block_size)
    return torch.nn.functional.linear(out.reshape(1, 1, hq * d), w["o_w"])


def decode_batch(hidden, positions, cache, layer, slots, block_tables, context_lens, w, cfg):
    hq, hkv, d, theta, fdt = _unpack(cfg)
    batch = hidden.shape[0]
    q, k, v = qkv_rope(hidden, positions, w, hq, hkv, d, theta, fdt)
    cache.write_slots(slots, k.squeeze(1), v.squeeze(1), layer)
    kc, vc = cache.get_layer_cache(layer)
    out = pa.decode_batch_parallel(q.squeeze(1), kc, vc, block_tables, context_lens,
                                   cache.block_size)
    return torch.nn.functional.linear(out.reshape(batch, 1, hq * d), w["o_w"])


def prefill_chunk(hidden, positions, cache, layer, slots, block_table, prefix_len,
                  context_len, tile_size, w, cfg):
    hq, hkv, d, theta, fdt = _unpack(cfg)
    chunk = hidden.shape[1]
    q, k, v = qkv_rope(hidden, positions, w, hq, hkv, d, theta, fdt)
    cache.write_slots(slots, k.squeeze(0), v.squeeze(0), layer)
    kc, vc = cache.get_layer_cache(layer)
    out = pa.prefill_chunk_tiled(q.squeeze(0), kc, vc, block_table, prefix_len, context_len,
                                 cache.block_size, tile_size)
    return torch.nn.functional.linear(out.reshape(1, chunk, hq * d), w["o_w"])
