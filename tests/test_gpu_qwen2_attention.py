"""Qwen2Attention's paged methods on the GPU against the oracle's restatement.

Same weights on both sides (the module's own seeded initialisation, copied
into the oracle's weight dict). Checked per method: the layer output, the K/V
rows written to the cache, and that every other slot is left untouched
(bit-for-bit; written slots hold exactly the K/V rows of the module's own
projection and rotation on the GPU).
Tolerances on the layer output (projections, RoPE, attention, o_proj):
1e-5 max-abs for FP32, 2e-2 for BF16.
"""

from __future__ import annotations

import types

import pytest
import torch

import oracle.qwen2_attention as oqa
from mini_llm_runtime_amd.model.qwen2_attention import Qwen2Attention, apply_rotary_pos_emb
from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache
from oracle.paged_kv_cache import OracleKVCache

pytestmark = pytest.mark.gpu

QWEN05B = types.SimpleNamespace(hidden_size=896, num_attention_heads=14,
                                num_key_value_heads=2, head_dim=64, rope_theta=1_000_000.0)
SMALL = types.SimpleNamespace(hidden_size=64, num_attention_heads=4, num_key_value_heads=2,
                              head_dim=16, rope_theta=10_000.0)
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


def make_module(cfg, dtype, device, seed=0):
    torch.manual_seed(seed)
    module = Qwen2Attention(cfg).to(dtype)
    w = {"q_w": module.qkv_proj.q_proj.weight, "q_b": module.qkv_proj.q_proj.bias,
         "k_w": module.qkv_proj.k_proj.weight, "k_b": module.qkv_proj.k_proj.bias,
         "v_w": module.qkv_proj.v_proj.weight, "v_b": module.qkv_proj.v_proj.bias,
         "o_w": module.o_proj.weight}
    w = {k: v.detach().clone() for k, v in w.items()}
    return module.to(device), w


def oracle_cfg(cfg, dtype):
    """The oracle's (hq, hkv, d, theta, freq_dtype): make_module casts the
    module to `dtype`, and with it the rotary inv_freq buffer, as a reference
    module cast with .to(dtype) holds it."""
    return (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.rope_theta,
            dtype)


def paired_caches(cfg, dtype, device, num_blocks, bs, seed):
    """A device cache and an oracle cache holding the same random pools."""
    gen = torch.Generator().manual_seed(seed)
    shape = (1, num_blocks, bs, cfg.num_key_value_heads, cfg.head_dim)
    k = (torch.randn(shape, generator=gen) * 0.5).to(dtype)
    v = (torch.randn(shape, generator=gen) * 0.5).to(dtype)
    dev = PagedKVCache(1, num_blocks, bs, cfg.num_key_value_heads, cfg.head_dim, dtype=dtype,
                       device=device)
    ora = OracleKVCache(1, num_blocks, bs, cfg.num_key_value_heads, cfg.head_dim, dtype=dtype)
    dev.k_cache.copy_(k)
    dev.v_cache.copy_(v)
    ora.k_cache.copy_(k)
    ora.v_cache.copy_(v)
    return dev, ora


def check_caches(dev, ora, written_slots, rows_k, rows_v):
    """Untouched slots keep their bits; written slots hold exactly the K/V rows
    the module computed on the GPU (rows_k/rows_v [T, Hkv, D], slot order).
    The oracle computes its rows with CPU GEMMs, which round differently, so
    its rows are compared through the layer output instead."""
    got_k = dev.k_cache[0].cpu().reshape(-1, dev.num_kv_heads, dev.head_dim)
    got_v = dev.v_cache[0].cpu().reshape(-1, dev.num_kv_heads, dev.head_dim)
    want_k = ora.k_cache[0].reshape(-1, dev.num_kv_heads, dev.head_dim)
    want_v = ora.v_cache[0].reshape(-1, dev.num_kv_heads, dev.head_dim)
    written = torch.zeros(got_k.shape[0], dtype=torch.bool)
    idx = torch.as_tensor(written_slots)
    written[idx] = True
    assert torch.equal(got_k[~written], want_k[~written])
    assert torch.equal(got_v[~written], want_v[~written])
    assert torch.equal(got_k[idx], rows_k.cpu())
    assert torch.equal(got_v[idx], rows_v.cpu())


def module_rows(module, hidden, positions, device, fused=True):
    """The K/V rows the module writes for these inputs, [T, Hkv, D].

    The cache paths project with one GEMM over the concatenated [q | k | v]
    weights and rotate in the fused kernel, which repeats the PyTorch
    rotation bit for bit (tests/test_gpu_pre_attention.py); the whole-prompt
    prefill keeps the three projections (fused=False)."""
    hidden, positions = hidden.to(device), positions.to(device)
    if not fused:
        _, k, v = module._qkv_rope(hidden, positions)
        return k.reshape(-1, *k.shape[-2:]), v.reshape(-1, *v.shape[-2:])
    weight, bias = module._qkv_weights()
    x = torch.nn.functional.linear(hidden.reshape(-1, hidden.shape[-1]), weight, bias)
    hq, hkv, d = module.num_attention_heads, module.num_key_value_heads, module.head_dim
    q = x[:, :hq * d].reshape(-1, hq, d)
    k = x[:, hq * d:(hq + hkv) * d].reshape(-1, hkv, d)
    v = x[:, (hq + hkv) * d:].reshape(-1, hkv, d)
    cos, sin = module.rotary_embedding(q, positions.reshape(-1))
    _, k = apply_rotary_pos_emb(q, k, cos, sin)
    return k, v


def max_abs(a, b):
    return (a.detach().double().cpu() - b.detach().double().cpu()).abs().max().item()


@pytest.mark.parametrize("cfg,dtype", [(SMALL, torch.float32), (QWEN05B, torch.bfloat16),
                                       (QWEN05B, torch.float32)],
                         ids=["small-fp32", "qwen05b-bf16", "qwen05b-fp32"])
def test_decode_batch_with_cache(device, cfg, dtype):
    module, w = make_module(cfg, dtype, device)
    bs, nblocks = 16, 96
    lens = [1, 17, 130, 255, 64]
    gen = torch.Generator().manual_seed(3)
    perm = torch.randperm(nblocks, generator=gen).tolist()
    need = [(n + bs - 1) // bs for n in lens]
    tables, at = [], 0
    for n in need:
        tables.append(perm[at:at + n])
        at += n
    width = max(need) + 1
    bt = torch.tensor([t + [-1] * (width - len(t)) for t in tables])
    ctx = torch.tensor(lens)
    pos = (ctx - 1).unsqueeze(1)
    slots = torch.tensor([tables[b][(n - 1) // bs] * bs + (n - 1) % bs
                          for b, n in enumerate(lens)])
    hidden = torch.randn(len(lens), 1, cfg.hidden_size, generator=gen).to(dtype)
    dev, ora = paired_caches(cfg, dtype, device, nblocks, bs, seed=5)
    got = module.forward_decode_batch_with_cache(hidden.to(device), pos.to(device), dev, 0,
                                                 slots.to(device), bt.to(device), ctx.to(device))
    want = oqa.decode_batch(hidden, pos, ora, 0, slots, bt, ctx, w, oracle_cfg(cfg, dtype))
    print(f"decode batch {cfg.hidden_size} {dtype}: max-abs {max_abs(got, want):.3e}")
    assert max_abs(got, want) <= TOL[dtype]
    check_caches(dev, ora, slots.tolist(), *module_rows(module, hidden, pos, device))


@pytest.mark.parametrize("cfg,dtype", [(SMALL, torch.float32), (QWEN05B, torch.bfloat16)],
                         ids=["small-fp32", "qwen05b-bf16"])
def test_decode_single_with_cache(device, cfg, dtype):
    module, w = make_module(cfg, dtype, device)
    bs, nblocks = 16, 16
    table = [7, 2, 11, 4]
    n = 50
    slot = torch.tensor([table[(n - 1) // bs] * bs + (n - 1) % bs])
    gen = torch.Generator().manual_seed(9)
    hidden = torch.randn(1, 1, cfg.hidden_size, generator=gen).to(dtype)
    pos = torch.tensor([[n - 1]])
    dev, ora = paired_caches(cfg, dtype, device, nblocks, bs, seed=6)
    got = module.forward_decode_with_cache(hidden.to(device), pos.to(device), dev, 0,
                                           slot.to(device), table, n)
    want = oqa.decode_single(hidden, pos, ora, 0, slot, table, n, w, oracle_cfg(cfg, dtype))
    assert max_abs(got, want) <= TOL[dtype]
    check_caches(dev, ora, slot.tolist(), *module_rows(module, hidden, pos, device))


@pytest.mark.parametrize("cfg,dtype,prefix,chunk,tile",
                         [(SMALL, torch.float32, 0, 21, 4), (SMALL, torch.float32, 37, 9, 16),
                          (QWEN05B, torch.bfloat16, 300, 128, 64),
                          (QWEN05B, torch.bfloat16, 0, 77, 16)],
                         ids=["small-fp32-first", "small-fp32-prefix", "qwen05b-bf16-prefix",
                              "qwen05b-bf16-first"])
def test_prefill_chunk_with_cache(device, cfg, dtype, prefix, chunk, tile):
    module, w = make_module(cfg, dtype, device)
    bs = 16
    context = prefix + chunk
    need = (context + bs - 1) // bs
    nblocks = need + 5
    gen = torch.Generator().manual_seed(prefix + chunk)
    table = torch.randperm(nblocks, generator=gen)[:need].tolist()
    positions = torch.arange(prefix, context).unsqueeze(0)
    slots = torch.tensor([table[p // bs] * bs + p % bs for p in range(prefix, context)])
    hidden = torch.randn(1, chunk, cfg.hidden_size, generator=gen).to(dtype)
    dev, ora = paired_caches(cfg, dtype, device, nblocks, bs, seed=8)
    got = module.forward_prefill_chunk_with_cache(hidden.to(device), positions.to(device), dev,
                                                  0, slots.to(device), table, prefix, context,
                                                  tile)
    want = oqa.prefill_chunk(hidden, positions, ora, 0, slots, table, prefix, context, tile, w,
                             oracle_cfg(cfg, dtype))
    print(f"prefill chunk {cfg.hidden_size} {dtype} p{prefix} c{chunk}: "
          f"max-abs {max_abs(got, want):.3e}")
    assert max_abs(got, want) <= TOL[dtype]
    check_caches(dev, ora, slots.tolist(), *module_rows(module, hidden, positions, device))


@pytest.mark.parametrize("cfg,dtype,seq", [(SMALL, torch.float32, 23),
                                           (QWEN05B, torch.bfloat16, 200)],
                         ids=["small-fp32", "qwen05b-bf16"])
def test_prefill_whole_with_cache(device, cfg, dtype, seq):
    module, w = make_module(cfg, dtype, device)
    bs, nblocks = 16, 40
    gen = torch.Generator().manual_seed(seq)
    table = torch.randperm(nblocks, generator=gen)[:(seq + bs - 1) // bs].tolist()
    slots = torch.tensor([table[p // bs] * bs + p % bs for p in range(seq)])
    positions = torch.arange(seq).unsqueeze(0)
    hidden = torch.randn(1, seq, cfg.hidden_size, generator=gen).to(dtype)
    dev, ora = paired_caches(cfg, dtype, device, nblocks, bs, seed=4)
    got = module.forward_prefill_with_cache(hidden.to(device), positions.to(device), dev, 0,
                                            slots.to(device))
    want = oqa.prefill_whole(hidden, positions, ora, 0, slots, w, oracle_cfg(cfg, dtype))
    assert max_abs(got, want) <= TOL[dtype]
    check_caches(dev, ora, slots.tolist(),
                 *module_rows(module, hidden, positions, device, fused=False))


def test_decode_steps_follow_the_prefill(device):
    """Prefill a prompt, then decode three tokens, each step's K/V written by
    the fused pre-attention step; the whole sequence matches the oracle run
    step by step."""
    cfg, dtype = SMALL, torch.float32
    module, w = make_module(cfg, dtype, device)
    bs, nblocks = 4, 12
    table = [5, 0, 9, 3, 7]
    prompt = 9
    gen = torch.Generator().manual_seed(2)
    dev, ora = paired_caches(cfg, dtype, device, nblocks, bs, seed=1)
    hidden = torch.randn(1, prompt, cfg.hidden_size, generator=gen)
    slots = torch.tensor([table[p // bs] * bs + p % bs for p in range(prompt)])
    positions = torch.arange(prompt).unsqueeze(0)
    got = module.forward_prefill_with_cache(hidden.to(device), positions.to(device), dev, 0,
                                            slots.to(device))
    want = oqa.prefill_whole(hidden, positions, ora, 0, slots, w, oracle_cfg(cfg, dtype))
    assert max_abs(got, want) <= TOL[dtype]
    written = slots.tolist()
    rows = [module_rows(module, hidden, positions, device, fused=False)]
    bt = torch.tensor([table])
    for step in range(3):
        n = prompt + step + 1
        slot = torch.tensor([table[(n - 1) // bs] * bs + (n - 1) % bs])
        x = torch.randn(1, 1, cfg.hidden_size, generator=gen)
        pos = torch.tensor([[n - 1]])
        ctx = torch.tensor([n])
        got = module.forward_decode_batch_with_cache(x.to(device), pos.to(device), dev, 0,
                                                     slot.to(device), bt.to(device),
                                                     ctx.to(device))
        want = oqa.decode_batch(x, pos, ora, 0, slot, bt, ctx, w, oracle_cfg(cfg, dtype))
        assert max_abs(got, want) <= TOL[dtype], f"step {step}"
        written += slot.tolist()
        rows.append(module_rows(module, x, pos, device))
    check_caches(dev, ora, written, torch.cat([r[0] for r in rows]),
                 torch.cat([r[1] for r in rows]))


def _device_decode_case(device, dtype=torch.float32):
    """The reference's make_decode_case (tests/model/test_qwen2_batch_decode.py:
    15-31): two decode requests over a 6-block, block-size-2 pool of layer 1,
    here on the device."""
    cfg = types.SimpleNamespace(hidden_size=64, num_attention_heads=4, num_key_value_heads=2,
                                head_dim=16, rope_theta=1_000_000.0)
    torch.manual_seed(42)
    module = Qwen2Attention(cfg).to(dtype=dtype).to(device)
    cache = PagedKVCache(2, 6, 2, 2, 16, dtype=dtype, device=device)
    cache.k_cache.normal_()
    cache.v_cache.normal_()
    inputs = dict(
        hidden_states=torch.randn(2, 1, 64, dtype=dtype, device=device),
        position_ids=torch.tensor([[2], [4]], device=device),
        layer_idx=1,
        slot_mapping=torch.tensor([0, 8], device=device),
        block_tables=torch.tensor([[2, 0, -1], [1, 3, 4]], device=device),
        context_lens=torch.tensor([3, 5], device=device),
    )
    return module, cache, inputs


@pytest.mark.parametrize("field,value,message", [
    ("hidden_states", torch.zeros(2, 2, 64), "hidden_states must have shape"),
    ("position_ids", torch.tensor([[1], [4]]), "decode positions"),
    ("context_lens", torch.tensor([0, 5]), "greater than 0"),
    ("block_tables", torch.tensor([[2, 0], [1, 3]]), "insufficient blocks"),
    ("block_tables", torch.tensor([[2, -1, -1], [1, 3, 4]]), "invalid physical block"),
    ("slot_mapping", torch.tensor([1, 8]), "slot_mapping must match"),
    ("slot_mapping", torch.tensor([8, 8]), "slot_mapping must match"),
    ("context_lens", torch.tensor([3., 5.]), "torch.long dtype"),
])
def test_device_batch_decode_rejects_metadata_before_cache_write(device, field, value,
                                                                 message):
    """Reference tests/model/test_qwen2_batch_decode.py:74-94 on a device
    cache: the metadata checks run on the device (one reduction, one host
    sync) before the fused write and the decode launch, so a rejected call
    leaves both layers of the cache bit-identical."""
    module, cache, inputs = _device_decode_case(device)
    old_k, old_v = cache.k_cache.clone(), cache.v_cache.clone()
    inputs[field] = value.to(device)
    with pytest.raises(ValueError, match=message):
        with torch.no_grad():
            module.forward_decode_batch_with_cache(kv_cache=cache, **inputs)
    torch.cuda.synchronize()
    assert torch.equal(cache.k_cache, old_k)
    assert torch.equal(cache.v_cache, old_v)


def test_device_batch_decode_accepts_the_unmutated_case(device):
    """The same case without a mutation runs and writes exactly the two slots
    of layer 1 (the other slots and layer 0 keep their bits)."""
    module, cache, inputs = _device_decode_case(device)
    old_k = cache.k_cache.clone()
    with torch.no_grad():
        out = module.forward_decode_batch_with_cache(kv_cache=cache, **inputs)
    assert out.shape == (2, 1, 64) and torch.isfinite(out).all()
    changed = (cache.k_cache != old_k).reshape(2, 12, -1).any(-1).cpu()
    assert not changed[0].any()
    assert changed[1].nonzero().flatten().tolist() == [0, 8]
