"""Fused pre-attention step (mlr_qkv_rope_write: bias + rotary embedding + KV
write) on the GPU.

Two references:
- the unfused PyTorch sequence of the reference's attention callers
  (Qwen2RotaryEmbedding -> apply_rotary_pos_emb -> write_slots,
  model/qwen2.py:125-209, :605-613) run on the same GPU: bit-exact, since the
  kernel repeats its rounding operation by operation and uses the same device
  cos/sin;
- the oracle (oracle/qwen2_attention.py rope_tables + rotate, OracleKVCache
  write) on the CPU: FP32 within 1e-5; in half precision the CPU and GPU
  cos/sin may differ in the last FP32 bit, which can move a rounding of cos,
  sin or a product, so the bound is two ulps of the terms |x_lo| + |x_hi|.
"""

from __future__ import annotations

import pytest
import torch

from mini_llm_runtime_amd.kernels.pre_attention import qkv_rope_write
from mini_llm_runtime_amd.model.qwen2_attention import Qwen2RotaryEmbedding, apply_rotary_pos_emb
from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache
from oracle import qwen2_attention as oqa
from oracle.paged_kv_cache import OracleKVCache

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
SHAPES = [(14, 2, 64), (4, 4, 128), (8, 1, 64), (2, 1, 16), (28, 4, 128)]  # (Hq, Hkv, D)
THETA = 1_000_000.0
ULP = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}


def make_case(seed, tokens, hq, hkv, d, dtype, with_bias, index_dtype, num_blocks=40, bs=16):
    gen = torch.Generator().manual_seed(seed)
    width = (hq + 2 * hkv) * d
    qkv = torch.randn(tokens, width, generator=gen).to(dtype)
    bias = torch.randn(width, generator=gen).to(dtype) if with_bias else None
    # Positions past Qwen2.5's 32768: the rotation has no table bound.
    positions = torch.randint(0, 40000, (tokens,), generator=gen)
    slots = torch.randperm(num_blocks * bs, generator=gen)[:tokens].to(index_dtype)
    pool = torch.randn(2, 1, num_blocks, bs, hkv, d, generator=gen).to(dtype)
    return qkv, bias, positions, slots, pool


def gpu_cache(pool, device):
    _, layers, nb, bs, hkv, d = pool.shape
    cache = PagedKVCache(layers, nb, bs, hkv, d, dtype=pool.dtype, device=device)
    cache.k_cache.copy_(pool[0])
    cache.v_cache.copy_(pool[1])
    return cache


def split_heads(x, hq, hkv, d):
    t = x.shape[0]
    return (x[:, :hq * d].reshape(t, hq, d), x[:, hq * d:(hq + hkv) * d].reshape(t, hkv, d),
            x[:, (hq + hkv) * d:].reshape(t, hkv, d))


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
# 1030 and 2048 tokens take four tokens per workgroup (1030: a partial last one).
@pytest.mark.parametrize("tokens", [1, 37, 300, 1030, 2048])
@pytest.mark.parametrize("with_bias", [False, True], ids=["nobias", "bias"])
def test_bit_exact_against_unfused_torch_path(device, dtype, shape, tokens, with_bias):
    hq, hkv, d = shape
    index_dtype = torch.int32 if tokens % 2 else torch.int64
    qkv, bias, positions, slots, pool = make_case(tokens + d, tokens, hq, hkv, d, dtype,
                                                  with_bias, index_dtype,
                                                  num_blocks=max(40, tokens // 16 + 8))
    rot = Qwen2RotaryEmbedding(d, THETA).to(device)
    qkv_d, pos_d, slots_d = qkv.to(device), positions.to(device), slots.to(device)
    bias_d = bias.to(device) if bias is not None else None

    # Unfused: the reference's ops with torch on the same device.
    ref_cache = gpu_cache(pool, device)
    x = qkv_d + bias_d if bias_d is not None else qkv_d
    q, k, v = split_heads(x, hq, hkv, d)
    cos, sin = rot(q, pos_d)
    q_ref, k_ref = apply_rotary_pos_emb(q, k, cos, sin)
    ref_cache.write_slots(slots_d, k_ref, v, layer_idx=0)

    cache = gpu_cache(pool, device)
    q_out = qkv_rope_write(qkv_d, pos_d, rot.inv_freq, cache, 0, slots_d, hq, bias=bias_d)
    torch.cuda.synchronize()
    assert torch.equal(q_out.cpu(), q_ref.cpu())
    assert torch.equal(cache.k_cache.cpu(), ref_cache.k_cache.cpu())
    assert torch.equal(cache.v_cache.cpu(), ref_cache.v_cache.cpu())


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("shape", SHAPES[:2], ids=lambda s: "x".join(map(str, s)))
def test_matches_oracle(device, dtype, shape):
    hq, hkv, d = shape
    tokens = 129
    qkv, bias, positions, slots, pool = make_case(7, tokens, hq, hkv, d, dtype, True,
                                                  torch.int64)
    x = qkv + bias
    q, k, v = split_heads(x, hq, hkv, d)
    cos, sin = oqa.rope_tables(positions, d, THETA, dtype)
    q_want, k_want = oqa.rotate(q, cos, sin), oqa.rotate(k, cos, sin)
    oracle = OracleKVCache(1, pool.shape[2], pool.shape[3], hkv, d, dtype=dtype)
    oracle.k_cache.copy_(pool[0])
    oracle.v_cache.copy_(pool[1])
    oracle.write_slots(slots, k_want, v, 0)

    rot = Qwen2RotaryEmbedding(d, THETA).to(device)
    cache = gpu_cache(pool, device)
    q_out = qkv_rope_write(qkv.to(device), positions.to(device), rot.inv_freq, cache, 0,
                           slots.to(device), hq, bias=bias.to(device))

    def close(got, want, x):
        """FP32: 1e-5. Half precision: a one-ulp change of cos or sin moves
        each product by at most one ulp of that product, so the bound is two
        ulps of |x_lo| + |x_hi| (the terms, not the possibly cancelling sum)."""
        got, want = got.cpu().double(), want.double()
        if dtype == torch.float32:
            return (got - want).abs().max().item() <= 1e-5
        half = d // 2
        x = x.double()
        mag = x.abs() + torch.cat((x[..., half:], x[..., :half]), dim=-1).abs()
        return bool(((got - want).abs() <= 2 * ULP[dtype] * mag).all())

    assert close(q_out, q_want, q)
    written = slots.tolist()
    assert close(cache.k_cache[0].view(-1, hkv, d)[written], k_want, k)
    keep = torch.ones(cache.k_cache[0].view(-1, hkv, d).shape[0], dtype=torch.bool)
    keep[written] = False
    assert torch.equal(cache.k_cache[0].view(-1, hkv, d).cpu()[keep],
                       oracle.k_cache[0].view(-1, hkv, d)[keep])
    assert torch.equal(cache.v_cache.cpu(), oracle.v_cache)


@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_out_of_range_slots_are_skipped_and_q_still_written(device, index_dtype):
    hq, hkv, d, dtype = 4, 2, 64, torch.bfloat16
    qkv, _, positions, _, pool = make_case(5, 4, hq, hkv, d, dtype, False, index_dtype)
    num_slots = pool.shape[2] * pool.shape[3]
    slots = torch.tensor([-1, num_slots, 3, 2 ** 30], dtype=index_dtype)
    rot = Qwen2RotaryEmbedding(d, THETA).to(device)
    cache = gpu_cache(pool, device)
    q_out = qkv_rope_write(qkv.to(device), positions.to(device), rot.inv_freq, cache, 0,
                           slots.to(device), hq)
    q, k, v = split_heads(qkv.to(device), hq, hkv, d)
    cos, sin = rot(q, positions.to(device))
    q_ref, k_ref = apply_rotary_pos_emb(q, k, cos, sin)
    assert torch.equal(q_out.cpu(), q_ref.cpu())
    want_k, want_v = pool[0, 0].clone(), pool[1, 0].clone()
    want_k.view(-1, hkv, d)[3] = k_ref[2].cpu()
    want_v.view(-1, hkv, d)[3] = v[2].cpu()
    assert torch.equal(cache.k_cache[0].cpu(), want_k)
    assert torch.equal(cache.v_cache[0].cpu(), want_v)


def test_empty_batch_and_strided_rows(device):
    hq, hkv, d, dtype = 2, 1, 64, torch.float32
    rot = Qwen2RotaryEmbedding(d, THETA).to(device)
    cache = PagedKVCache(1, 4, 16, hkv, d, dtype=dtype, device=device)
    empty = torch.empty(0, (hq + 2 * hkv) * d, device=device)
    out = qkv_rope_write(empty, torch.empty(0, dtype=torch.long, device=device), rot.inv_freq,
                         cache, 0, torch.empty(0, dtype=torch.long, device=device), hq)
    assert out.shape == (0, hq, d)
    # Rows taken from a wider buffer (row stride > row width).
    gen = torch.Generator().manual_seed(1)
    wide = torch.randn(9, (hq + 2 * hkv) * d + 40, generator=gen).to(device)
    qkv = wide[:, :(hq + 2 * hkv) * d]
    positions = torch.arange(100, 109, device=device)
    slots = torch.arange(9, device=device) * 3
    q_out = qkv_rope_write(qkv, positions, rot.inv_freq, cache, 0, slots, hq)
    q, k, v = split_heads(qkv.contiguous(), hq, hkv, d)
    cos, sin = rot(q, positions)
    q_ref, k_ref = apply_rotary_pos_emb(q, k, cos, sin)
    assert torch.equal(q_out.cpu(), q_ref.cpu())
    assert torch.equal(cache.k_cache[0].view(-1, hkv, d)[slots].cpu(), k_ref.cpu())
    assert torch.equal(cache.v_cache[0].view(-1, hkv, d)[slots].cpu(), v.cpu())


def test_bf16_module_inv_freq_is_used_as_stored(device):
    """A model cast to bf16 casts the rotary buffer too; the reference then
    promotes those bf16 frequencies to FP32 (model/qwen2.py:163-167). The
    kernel takes the buffer as stored."""
    hq, hkv, d, dtype = 4, 2, 64, torch.bfloat16
    qkv, _, positions, slots, pool = make_case(9, 33, hq, hkv, d, dtype, False, torch.int64)
    rot = Qwen2RotaryEmbedding(d, THETA).to(device=device, dtype=torch.bfloat16)
    assert rot.inv_freq.dtype == torch.bfloat16
    cache = gpu_cache(pool, device)
    q_out = qkv_rope_write(qkv.to(device), positions.to(device), rot.inv_freq, cache, 0,
                           slots.to(device), hq)
    q, k, _ = split_heads(qkv.to(device), hq, hkv, d)
    cos, sin = rot(q, positions.to(device))
    q_ref, _ = apply_rotary_pos_emb(q, k, cos, sin)
    assert torch.equal(q_out.cpu(), q_ref.cpu())
