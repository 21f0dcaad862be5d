"""One-launch decode step (mlr_paged_decode_qkv: rotary embedding of q and the
new key + KV write + paged decode after the QKV projection) on the GPU.

The fused call must equal the two launches it replaces bit for bit: the
pre-attention step mlr_qkv_rope_write at positions context_lens - 1 (itself
bit-exact against the reference's PyTorch rotation and checked against the
oracle in test_gpu_pre_attention.py), then the batched decode. Both the
output and the cache rows written are compared with torch.equal, and the
decode output is checked against the oracle's decode (max-abs 2e-2, BF16
inputs with FP32 softmax). The cases reach every kernel layout the launcher
picks: head_dim 64 with one load batch per wave, a fifth tile in LDS (one KV
head or a pair per workgroup) and double-buffered loads; head_dim 128 with one
or two load batches per wave, with and without KV-head pairs.
"""

from __future__ import annotations

import pytest
import torch

import oracle.paged_attention as opa
from mini_llm_runtime_amd.kernels import paged_attention as kpa
from mini_llm_runtime_amd.kernels import pre_attention as kpre
from mini_llm_runtime_amd.model.qwen2_attention import Qwen2RotaryEmbedding
from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache
from oracle_pins import random_paged

pytestmark = pytest.mark.gpu

THETA = 1_000_000.0
BS = 16

# Contexts that give 24 sequences enough (sequence, split) items for the
# KV-head-pair kernels at head_dim 64 (320-token splits) and 128.
LENS64 = [3520, 1, 16, 17, 321, 640, 641, 2999, 3201, 150, 1280, 2048,
          900, 3333, 77, 2500, 319, 320, 1919, 3100, 2222, 1234, 555, 3456]
LENS128 = [2000, 1, 17, 640, 1999, 129, 700, 1500, 33, 1024, 1100, 385]

CASES = [
    # (id, hq, hkv, d, lens, tokens_per_split)
    ("d64-one-batch", 14, 2, 64, [1, 16, 17, 300, 1000, 257], 64),
    ("d64-lds-tile", 14, 2, 64, [300, 384, 770, 5, 321, 640], 320),
    ("d64-lds-pairs", 14, 2, 64, LENS64, 0),
    ("d64-lds-pairs-g8", 16, 2, 64, LENS64, 320),
    ("d64-double", 16, 4, 64, [300, 384, 770, 5, 1500], 384),
    ("d64-mha", 8, 8, 64, [33, 64, 500, 2000], 0),
    ("d64-group16", 32, 2, 64, [1, 700, 2100], 0),
    ("d128-one-batch", 8, 1, 128, [5, 129, 700, 64], 64),
    ("d128-double", 16, 1, 128, [5, 129, 700, 64, 1000], 176),
    ("d128-pairs", 28, 4, 128, LENS128, 128),
    ("d128-pairs-double", 28, 4, 128, LENS128, 176),
]


def _case(hq, hkv, d, lens, seed, dtype=torch.bfloat16):
    _, kc, vc, bt, sl, tables = random_paged(lens, hq, hkv, d, BS, dtype=dtype,
                                             seed=seed, fill=0.0)
    gen = torch.Generator().manual_seed(seed + 7)
    qkv = torch.randn(len(lens), (hq + 2 * hkv) * d, generator=gen).to(dtype)
    slots = torch.tensor([tables[b][(n - 1) // BS] * BS + (n - 1) % BS
                          for b, n in enumerate(lens)])
    return qkv, kc, vc, bt, sl, slots, tables


def _cache(kc, vc, device):
    nb, bs, hkv, d = kc.shape
    cache = PagedKVCache(1, nb, bs, hkv, d, dtype=kc.dtype, device=device)
    cache.k_cache[0].copy_(kc)
    cache.v_cache[0].copy_(vc)
    return cache


def _two_launches(qkv, inv_freq, cache, bt, sl, slots, hq, tokens_per_split):
    q = kpre.qkv_rope_write(qkv, sl - 1, inv_freq, cache, 0, slots, hq)
    k, v = cache.get_layer_cache(0)
    return kpa.paged_decode_launch(q, k, v, bt, sl, tokens_per_split=tokens_per_split), q


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("cid,hq,hkv,d,lens,tokens_per_split", CASES,
                         ids=[c[0] for c in CASES])
def test_one_launch_equals_rope_write_then_decode(device, cid, hq, hkv, d, lens,
                                                  tokens_per_split, dtype):
    qkv, kc, vc, bt, sl, slots, tables = _case(hq, hkv, d, lens, seed=len(lens) * 31 + d + hq,
                                               dtype=dtype)
    inv_freq = Qwen2RotaryEmbedding(d, THETA).inv_freq.to(device)
    qkv, bt, sl, slots = (t.to(device) for t in (qkv, bt, sl, slots))

    two_cache = _cache(kc, vc, device)
    want, q = _two_launches(qkv, inv_freq, two_cache, bt, sl, slots, hq, tokens_per_split)
    one_cache = _cache(kc, vc, device)
    got = kpre.qkv_rope_decode(qkv, inv_freq, one_cache, 0, slots, bt, sl, hq,
                               tokens_per_split=tokens_per_split)
    assert torch.equal(one_cache.k_cache, two_cache.k_cache)
    assert torch.equal(one_cache.v_cache, two_cache.v_cache)
    assert torch.equal(got, want)

    k, v = two_cache.get_layer_cache(0)
    oracle = opa.decode_batch_loop(q.cpu(), k.cpu(), v.cpu(), tables, lens, BS)
    assert torch.isfinite(got).all()
    assert (got.double().cpu() - oracle.double()).abs().max().item() <= 2e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_half_inv_freq_and_strided_qkv_rows(device, dtype):
    """A model cast to bf16 (fp16) holds inv_freq in bf16 (fp16), used as its
    FP32 value as qkv_rope_write does, and qkv rows may come from a wider
    buffer."""
    hq, hkv, d, lens = 14, 2, 64, [40, 1, 333]
    qkv, kc, vc, bt, sl, slots, _ = _case(hq, hkv, d, lens, seed=3, dtype=dtype)
    inv_freq = Qwen2RotaryEmbedding(d, THETA).inv_freq.to(device, dtype)
    wide = torch.zeros(len(lens), qkv.shape[1] + 64, dtype=dtype)
    wide[:, :qkv.shape[1]] = qkv
    wide, bt, sl, slots = (t.to(device) for t in (wide, bt, sl, slots))
    rows = wide[:, :qkv.shape[1]]

    two_cache = _cache(kc, vc, device)
    want, _ = _two_launches(rows.contiguous(), inv_freq, two_cache, bt, sl, slots, hq, 0)
    one_cache = _cache(kc, vc, device)
    got = kpre.qkv_rope_decode(rows, inv_freq, one_cache, 0, slots, bt, sl, hq)
    assert torch.equal(one_cache.k_cache, two_cache.k_cache)
    assert torch.equal(one_cache.v_cache, two_cache.v_cache)
    assert torch.equal(got, want)


def test_misaligned_qkv_rows_are_copied(device):
    """Rows that start 2 bytes past a 16-byte boundary (a view one element
    into a wider buffer) are copied to an aligned buffer first."""
    hq, hkv, d, lens = 14, 2, 64, [77, 5]
    qkv, kc, vc, bt, sl, slots, _ = _case(hq, hkv, d, lens, seed=5)
    inv_freq = Qwen2RotaryEmbedding(d, THETA).inv_freq.to(device)
    wide = torch.zeros(len(lens), qkv.shape[1] + 8, dtype=torch.bfloat16)
    wide[:, 1:qkv.shape[1] + 1] = qkv
    wide, bt, sl, slots = (t.to(device) for t in (wide, bt, sl, slots))
    rows = wide[:, 1:qkv.shape[1] + 1]
    assert rows.data_ptr() % 16 != 0

    two_cache = _cache(kc, vc, device)
    want, _ = _two_launches(rows.contiguous(), inv_freq, two_cache, bt, sl, slots, hq, 0)
    one_cache = _cache(kc, vc, device)
    got = kpre.qkv_rope_decode(rows, inv_freq, one_cache, 0, slots, bt, sl, hq)
    assert torch.equal(one_cache.k_cache, two_cache.k_cache)
    assert torch.equal(got, want)


def test_repeated_steps_reuse_the_workspace(device):
    """Three decode steps in a row on one cache: each step's new row is read
    back by the next, and the shared workspace is left clean each time."""
    hq, hkv, d = 14, 2, 64
    lens = [300, 17, 1000, 64]
    qkv, kc, vc, bt, sl, _, tables = _case(hq, hkv, d, [n + 3 for n in lens], seed=11)
    inv_freq = Qwen2RotaryEmbedding(d, THETA).inv_freq.to(device)
    bt = bt.to(device)
    one_cache, two_cache = _cache(kc, vc, device), _cache(kc, vc, device)
    gen = torch.Generator().manual_seed(12)
    for step in range(3):
        ctx = torch.tensor([n + step + 1 for n in lens])
        slots = torch.tensor([tables[b][(n - 1) // BS] * BS + (n - 1) % BS
                              for b, n in enumerate(ctx.tolist())])
        qkv = torch.randn(len(lens), qkv.shape[1], generator=gen).bfloat16().to(device)
        ctx, slots = ctx.to(device), slots.to(device)
        want, _ = _two_launches(qkv, inv_freq, two_cache, bt, ctx, slots, hq, 0)
        got = kpre.qkv_rope_decode(qkv, inv_freq, one_cache, 0, slots, bt, ctx, hq)
        assert torch.equal(got, want), step
    assert torch.equal(one_cache.k_cache, two_cache.k_cache)
    assert torch.equal(one_cache.v_cache, two_cache.v_cache)


def test_shapes_outside_the_kernel_are_rejected(device):
    cache = PagedKVCache(1, 8, BS, 2, 32, dtype=torch.bfloat16, device=device)
    assert not kpre.qkv_rope_decode_fusable(torch.bfloat16, cache, 4)
    qkv = torch.zeros(1, 8 * 32, dtype=torch.bfloat16, device=device)
    one = torch.ones(1, dtype=torch.long, device=device)
    with pytest.raises(ValueError, match="head_dim 64 or 128"):
        kpre.qkv_rope_decode(qkv, torch.ones(16, device=device), cache, 0, one - 1,
                             torch.zeros(1, 1, dtype=torch.long, device=device), one, 4)


def test_one_launch_step_in_graph_replays(device):
    """The one-launch step captured in a HIP graph and replayed four times,
    with new projection rows copied in eagerly between replays: every replay
    equals an eager call on a copy of the cache, output and cache bits."""
    hq, hkv, d = 14, 2, 64
    lens = [33, 600, 1500, 4000, 257]
    qkv, kc, vc, bt, sl, slots, _ = _case(hq, hkv, d, lens, seed=41)
    inv_freq = Qwen2RotaryEmbedding(d, THETA).inv_freq.to(device)
    qkv, bt, sl, slots = (t.to(device) for t in (qkv, bt, sl, slots))
    cache = _cache(kc, vc, device)
    out = torch.empty(len(lens), hq, d, dtype=torch.bfloat16, device=device)
    ws = torch.zeros(kpa.decode_workspace_bytes(len(lens), hq, d, bt.shape[1] * BS,
                                                torch.bfloat16),
                     dtype=torch.uint8, device=device)
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        kpre.qkv_rope_decode(qkv, inv_freq, cache, 0, slots, bt, sl, hq, out=out, workspace=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        kpre.qkv_rope_decode(qkv, inv_freq, cache, 0, slots, bt, sl, hq, out=out, workspace=ws)
    gen = torch.Generator().manual_seed(4)
    for _ in range(4):
        qkv.copy_(torch.randn(qkv.shape, generator=gen).to(torch.bfloat16).to(device))
        eager_cache = _cache(cache.k_cache[0].clone(), cache.v_cache[0].clone(), device)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = kpre.qkv_rope_decode(qkv, inv_freq, eager_cache, 0, slots, bt, sl, hq)
        assert torch.equal(out, eager)
        assert torch.equal(cache.k_cache, eager_cache.k_cache)
        assert torch.equal(cache.v_cache, eager_cache.v_cache)


def test_qwen05b_b64_served_step_matches_oracle(device):
    """The served decode step (what forward_decode_batch_with_cache runs after
    its QKV GEMM) at full size: batch 64, 14/2 heads, head_dim 64, contexts
    U[128, 4096] in a 24,576-block pool. qkv_rope_decode against the oracle's
    rotary embedding (rope_tables + rotate at position ctx - 1, the
    reference's model/qwen2.py:125-209 restated), write_slots and
    decode_batch_parallel: output within 2e-2 on every (sequence, head) row,
    written V rows bit-exact, written K rows within two bf16 ulps of the
    terms of the oracle's (cos/sin come from the device's and the host's
    libraries); and
    equal bit for bit to mlr_qkv_rope_write followed by the decode."""
    import oracle.qwen2_attention as oqa
    from mini_llm_runtime_amd import workloads

    wl = workloads.bf16_decode_qwen05b_b64()
    hq, hkv, d = 14, 2, 64
    gen = torch.Generator().manual_seed(64)
    qkv = torch.randn(64, (hq + 2 * hkv) * d, generator=gen).bfloat16()
    q = qkv[:, :hq * d].reshape(64, hq, d)
    k_new = qkv[:, hq * d:(hq + hkv) * d].reshape(64, hkv, d)
    v_new = qkv[:, (hq + hkv) * d:].reshape(64, hkv, d)
    cos, sin = oqa.rope_tables(wl.context_lens - 1, d, THETA, torch.bfloat16)
    q_rot, k_rot = oqa.rotate(q, cos, sin), oqa.rotate(k_new, cos, sin)
    kc, vc = wl.k_cache.clone(), wl.v_cache.clone()
    kc.view(-1, hkv, d).index_copy_(0, wl.slot_mapping, k_rot)
    vc.view(-1, hkv, d).index_copy_(0, wl.slot_mapping, v_new)
    want = opa.decode_batch_parallel(q_rot, kc, vc, wl.block_tables, wl.context_lens, BS)

    inv_freq = Qwen2RotaryEmbedding(d, THETA).inv_freq.to(device)
    qkv_d, bt, sl, slots = (t.to(device) for t in (qkv, wl.block_tables, wl.context_lens,
                                                      wl.slot_mapping))
    one_cache = _cache(wl.k_cache, wl.v_cache, device)
    got = kpre.qkv_rope_decode(qkv_d, inv_freq, one_cache, 0, slots, bt, sl, hq)
    err = (got.double().cpu() - want.double()).abs().max().item()
    print(f"qwen05b_b64 served step max-abs vs oracle: {err:.3e}")
    assert torch.isfinite(got).all()
    assert err <= 2e-2
    k_rows = one_cache.k_cache[0].view(-1, hkv, d).index_select(0, slots).cpu()
    v_rows = one_cache.v_cache[0].view(-1, hkv, d).index_select(0, slots).cpu()
    assert torch.equal(v_rows, v_new)
    # A one-ulp change of cos or sin moves each product by at most one ulp
    # of that product: two bf16 ulps (2^-7 relative) of the terms
    # |x_lo| + |x_hi|, not of their possibly cancelling sum.
    x = k_new.double()
    mag = x.abs() + torch.cat((x[..., d // 2:], x[..., :d // 2]), dim=-1).abs()
    assert ((k_rows.double() - k_rot.double()).abs() <= 2 * 2.0 ** -7 * mag).all()

    two_cache = _cache(wl.k_cache, wl.v_cache, device)
    pair, _ = _two_launches(qkv_d, inv_freq, two_cache, bt, sl, slots, hq, 0)
    assert torch.equal(one_cache.k_cache, two_cache.k_cache)
    assert torch.equal(got, pair)


def _random_served_case(seed):
    """Shape of a seeded served-step case: head_dim, KV heads, GQA group,
    batch, context lengths (edge lengths mixed in) and split size."""
    gen = torch.Generator().manual_seed(9100 + seed)

    def pick(values):
        return values[int(torch.randint(len(values), (1,), generator=gen))]

    d = pick([64, 64, 128])
    hkv = pick([1, 2, 2, 4])
    group = pick([1, 2, 4, 7, 8, 16])
    batch = int(torch.randint(1, 25, (1,), generator=gen))
    lens = torch.randint(1, 3001, (batch,), generator=gen).tolist()
    edges = [1, 15, 16, 17, 319, 320, 321, 640]
    for i in range(0, batch, 3):
        lens[i] = pick(edges)
    return d, hkv * group, hkv, lens, pick([0, 0, 64, 128, 176, 320])


@pytest.mark.parametrize("seed", range(12))
def test_random_served_steps_equal_the_two_launches(device, seed):
    """Seeded random shapes of the one-launch served step: equal to
    mlr_qkv_rope_write followed by the decode bit for bit (output and cache),
    and within 2e-2 of the oracle's decode."""
    _check_random_served(device, seed, torch.bfloat16)


@pytest.mark.parametrize("seed", range(6))
def test_random_served_steps_fp16(device, seed):
    """The same in fp16 (other draws)."""
    _check_random_served(device, 100 + seed, torch.float16)


def _check_random_served(device, seed, dtype):
    d, hq, hkv, lens, ts = _random_served_case(seed)
    shape = (f"seed {seed} {str(dtype)[6:]}: d={d} hq={hq} hkv={hkv} batch={len(lens)} "
             f"ts={ts} lens={lens}")
    qkv, kc, vc, bt, sl, slots, tables = _case(hq, hkv, d, lens, seed=500 + seed, dtype=dtype)
    inv_freq = Qwen2RotaryEmbedding(d, THETA).inv_freq.to(device)
    qkv, bt, sl, slots = (t.to(device) for t in (qkv, bt, sl, slots))

    two_cache = _cache(kc, vc, device)
    want, q = _two_launches(qkv, inv_freq, two_cache, bt, sl, slots, hq, ts)
    one_cache = _cache(kc, vc, device)
    got = kpre.qkv_rope_decode(qkv, inv_freq, one_cache, 0, slots, bt, sl, hq,
                               tokens_per_split=ts)
    assert torch.equal(one_cache.k_cache, two_cache.k_cache), shape
    assert torch.equal(one_cache.v_cache, two_cache.v_cache), shape
    assert torch.equal(got, want), shape

    k, v = two_cache.get_layer_cache(0)
    oracle = opa.decode_batch_loop(q.cpu(), k.cpu(), v.cpu(), tables, lens, BS)
    assert torch.isfinite(got).all(), shape
    assert (got.double().cpu() - oracle.double()).abs().max().item() <= 2e-2, shape
