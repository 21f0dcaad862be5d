"""Batched paged decode on the GPU against the oracle (CPU).

Tolerances (max-abs): 1e-5 for FP32 and FP64 inputs, 2e-2 for BF16 and FP16
inputs with FP32 softmax. Every case also checks that padded block-table
entries and unwritten (NaN) pool rows never reach the result.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle.paged_attention as opa
from mini_llm_runtime_amd import workloads
from mini_llm_runtime_amd.kernels import paged_attention as kpa
from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache
from oracle_pins import random_paged

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.float64: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.double().cpu() - b.double().cpu()).abs().max().item()


def run_decode(q, kc, vc, bt, sl, bs, device, **kw):
    return kpa.paged_attention_decode_batch_parallel(
        q.to(device), kc.to(device), vc.to(device), bt.to(device), sl.to(device), bs, **kw)


@pytest.mark.parametrize(
    "hq,hkv,seq_lens,tables",
    [
        (4, 2, [3, 5], [[2, 0, -1], [1, 3, 4]]),
        (2, 2, [3, 5], [[2, 0, -1], [1, 3, 4]]),
        (4, 1, [3, 5], [[2, 0, -1], [1, 3, 4]]),
        (4, 2, [3, 4], [[2, 0], [1, 3]]),
    ],
    ids=["gqa-ragged", "mha-ragged", "mqa-ragged", "seq-length-equals-heads"],
)
def test_reference_batch_cases(device, hq, hkv, seq_lens, tables):
    torch.manual_seed(42)
    q = torch.randn(len(seq_lens), hq, 8)
    kc = torch.randn(5, 2, hkv, 8)
    vc = torch.randn_like(kc)
    bt, sl = torch.tensor(tables), torch.tensor(seq_lens)
    want = opa.decode_batch_parallel(q, kc, vc, bt, sl, 2)
    got = run_decode(q, kc, vc, bt, sl, 2, device)
    assert max_abs(got, want) <= 1e-5


def test_fp32_decode_b4_with_new_token_write(device):
    """FP32 decode, batch 4, GQA 7:1, contexts {17, 64, 130, 255} (max-abs 1e-5)."""
    wl = workloads.fp32_decode_b4()
    cache = PagedKVCache(1, 64, 16, 2, 64, dtype=torch.float32, device=device)
    cache.k_cache[0].copy_(wl.k_cache)
    cache.v_cache[0].copy_(wl.v_cache)
    cache.write_slots(wl.slot_mapping.to(device), wl.new_k.to(device), wl.new_v.to(device))
    ref_k, ref_v = wl.k_cache.clone(), wl.v_cache.clone()
    ref_k.view(-1, 2, 64).index_copy_(0, wl.slot_mapping, wl.new_k)
    ref_v.view(-1, 2, 64).index_copy_(0, wl.slot_mapping, wl.new_v)
    assert torch.equal(cache.k_cache[0].cpu(), ref_k)
    want = opa.decode_batch_parallel(wl.q, ref_k, ref_v, wl.block_tables, wl.context_lens, 16)
    k_layer, v_layer = cache.get_layer_cache(0)
    got = kpa.paged_attention_decode_batch_parallel(
        wl.q.to(device), k_layer, v_layer, wl.block_tables.to(device),
        wl.context_lens.to(device), 16)
    assert max_abs(got, want) <= 1e-5
    for b in range(4):
        single = kpa.paged_attention_decode(wl.q[b].to(device), k_layer, v_layer,
                                            wl.tables[b], int(wl.context_lens[b]), 16)
        assert max_abs(single, want[b]) <= 1e-5


CASES = [
    # (dtype, hq, hkv, d, block_size, seq_lens)
    (torch.bfloat16, 14, 2, 64, 16, [1, 15, 16, 17, 300, 1000]),   # MFMA, G=7
    (torch.bfloat16, 16, 2, 64, 16, [100, 321, 640, 2000]),        # MFMA, KV pair, G=8
    (torch.bfloat16, 16, 4, 64, 16, [5, 320, 1290]),               # MFMA, two KV pairs
    (torch.bfloat16, 28, 4, 128, 16, [33, 700, 2049]),             # MFMA, D=128
    (torch.bfloat16, 8, 8, 64, 16, [5, 100]),                      # MFMA, G=1
    (torch.bfloat16, 32, 2, 64, 32, [64, 513]),                    # MFMA, G=16, BS=32
    (torch.bfloat16, 14, 2, 64, 8, [9, 130]),                      # generic (BS=8)
    (torch.bfloat16, 40, 2, 64, 16, [77]),                         # generic (G=20)
    (torch.bfloat16, 8, 2, 96, 16, [50, 200]),                     # generic (D=96)
    (torch.float16, 14, 2, 64, 16, [31, 257, 1000]),               # fp16 MFMA, LDS tile
    (torch.float16, 16, 2, 64, 16, [100, 321, 640, 2000]),         # fp16 MFMA, KV pair
    (torch.float16, 28, 4, 128, 16, [33, 700, 2049]),              # fp16 MFMA, D=128
    (torch.float16, 8, 8, 64, 16, [5, 100]),                       # fp16 MFMA, G=1
    (torch.float16, 32, 2, 64, 32, [64, 513]),                     # fp16 MFMA, G=16, BS=32
    (torch.float16, 14, 2, 64, 8, [9, 130]),                       # generic (BS=8)
    # FP32 MFMA, merged splits; 18 work items: eight waves per KV head
    (torch.float32, 14, 2, 64, 16, [1, 255, 600]),
    (torch.float32, 28, 4, 128, 16, [33, 700, 2049]),              # FP32 MFMA, D=128
    (torch.float32, 32, 2, 64, 32, [64, 513, 1]),                  # G=16, BS=32, eight waves
    (torch.float32, 14, 2, 64, 8, [9, 130]),                       # generic (BS=8)
    (torch.float32, 6, 3, 40, 5, [7, 23]),
    (torch.float64, 4, 2, 16, 4, [3, 19]),
]


@pytest.mark.parametrize("dtype,hq,hkv,d,bs,lens", CASES,
                         ids=[f"{str(c[0])[6:]}-{c[1]}x{c[2]}-d{c[3]}-bs{c[4]}" for c in CASES])
def test_decode_matches_oracle(device, dtype, hq, hkv, d, bs, lens):
    # Unwritten rows are NaN: the kernel must never read them. The oracle's
    # tensorized path would (it multiplies block-0 filler by zero), so the
    # per-request oracle loop, which reads only live rows, is the reference.
    q, kc, vc, bt, sl, tables = random_paged(lens, hq, hkv, d, bs, dtype=dtype, seed=len(lens))
    want = opa.decode_batch_loop(q, kc, vc, tables, lens, bs)
    got = run_decode(q, kc, vc, bt, sl, bs, device)
    assert torch.isfinite(got).all()
    assert max_abs(got, want) <= TOL[dtype]


# 272..384: splits of 5-6 tiles per wave, whose last one or two tiles go
# through LDS (head_dim 64).
@pytest.mark.parametrize("tokens_per_split", [16, 48, 256, 272, 320, 384, 512, 4096])
def test_split_size_does_not_change_the_result(device, tokens_per_split):
    q, kc, vc, bt, sl, tables = random_paged([40, 777, 1500], 14, 2, 64, 16,
                                             dtype=torch.bfloat16, seed=5)
    want = opa.decode_batch_loop(q, kc, vc, tables, [40, 777, 1500], 16)
    got = run_decode(q, kc, vc, bt, sl, 16, device, tokens_per_split=tokens_per_split)
    assert max_abs(got, want) <= 2e-2


@pytest.mark.parametrize("dtype,lens,tokens_per_split", [
    (torch.bfloat16, [1, 16, 17, 300, 1000, 257], 0),     # fused in the MFMA kernel
    (torch.bfloat16, [33, 64, 500], 64),
    (torch.bfloat16, [300, 384, 770, 5], 384),              # new token in an LDS tile
    (torch.float16, [1, 16, 17, 300, 1000, 257], 0),      # fp16, fused in the MFMA kernel
    (torch.float16, [33, 64, 500, 2000], 128),
    (torch.float32, [5, 255, 256], 0),                     # fused in the FP32 MFMA kernel
    (torch.float32, [300, 384, 770, 5, 1000, 2049], 64),   # FP32, splits merged in-launch
])
def test_decode_append_equals_write_then_decode(device, dtype, lens, tokens_per_split):
    """mlr_paged_decode_append: same cache bits and same output bits as
    write_slots followed by paged decode."""
    q, kc, vc, bt, sl, tables = random_paged(lens, 14, 2, 64, 16, dtype=dtype, seed=21,
                                             fill=0.0)
    gen = torch.Generator().manual_seed(5)
    new_k = torch.randn(len(lens), 2, 64, generator=gen).to(dtype)
    new_v = torch.randn(len(lens), 2, 64, generator=gen).to(dtype)
    slots = torch.tensor([tables[b][(n - 1) // 16] * 16 + (n - 1) % 16
                          for b, n in enumerate(lens)])
    q, bt, sl, slots_d = (t.to(device) for t in (q, bt, sl, slots))
    k1, v1 = kc.to(device), vc.to(device)
    k2, v2 = kc.to(device), vc.to(device)
    nk, nv = new_k.to(device), new_v.to(device)
    fused = kpa.paged_decode_launch(q, k1, v1, bt, sl, new_k=nk, new_v=nv,
                                    slot_mapping=slots_d, tokens_per_split=tokens_per_split)
    k2.view(-1, 2, 64).index_copy_(0, slots_d, nk)
    v2.view(-1, 2, 64).index_copy_(0, slots_d, nv)
    plain = kpa.paged_decode_launch(q, k2, v2, bt, sl, tokens_per_split=tokens_per_split)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    assert torch.equal(fused, plain)
    want = opa.decode_batch_loop(q.cpu(), k2.cpu(), v2.cpu(), tables, lens, 16)
    assert max_abs(fused, want) <= TOL[dtype]


def _fused_and_plain_vs_oracle(device, lens, hq, hkv, d, tokens_per_split, seed,
                               dtype=torch.bfloat16):
    """The fused write against write-then-decode (same cache bits, same output
    bits) and the decode against the oracle."""
    q, kc, vc, bt, sl, tables = random_paged(lens, hq, hkv, d, 16, dtype=dtype,
                                             seed=seed, fill=0.0)
    gen = torch.Generator().manual_seed(seed + 1)
    new_k = torch.randn(len(lens), hkv, d, generator=gen).to(dtype)
    new_v = torch.randn(len(lens), hkv, d, generator=gen).to(dtype)
    slots = torch.tensor([tables[b][(n - 1) // 16] * 16 + (n - 1) % 16
                          for b, n in enumerate(lens)])
    q, bt, sl, slots_d = (t.to(device) for t in (q, bt, sl, slots))
    k1, v1 = kc.to(device), vc.to(device)
    k2, v2 = kc.to(device), vc.to(device)
    nk, nv = new_k.to(device), new_v.to(device)
    fused = kpa.paged_decode_launch(q, k1, v1, bt, sl, new_k=nk, new_v=nv,
                                    slot_mapping=slots_d, tokens_per_split=tokens_per_split)
    k2.view(-1, hkv, d).index_copy_(0, slots_d, nk)
    v2.view(-1, hkv, d).index_copy_(0, slots_d, nv)
    plain = kpa.paged_decode_launch(q, k2, v2, bt, sl, tokens_per_split=tokens_per_split)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    assert torch.equal(fused, plain)
    want = opa.decode_batch_loop(q.cpu(), k2.cpu(), v2.cpu(), tables, lens, 16)
    assert torch.isfinite(plain).all()
    assert max_abs(plain, want) <= TOL[dtype]


# Every FP32 instantiation the launcher picks (tiles per wave =
# ceil(tokens_per_split / 64)): head_dim 64 with up to four tiles in one load
# batch, or double-buffered batches of two; head_dim 128 with one tile, or
# double-buffered single tiles. GQA groups 7, 1 and 8; contexts from one token
# to 4000 (up to 63 splits merged in the launch).
FP32_LENS = [4000, 1, 17, 64, 65, 255, 256, 257, 640, 1500, 2049, 3333]


@pytest.mark.parametrize("d,hq,hkv,tokens_per_split", [
    (64, 14, 2, 64),     # one tile per wave
    (64, 14, 2, 256),    # four tiles in one batch (the fp32_decode_b4 layout)
    (64, 14, 2, 512),    # double-buffered batches of two
    (64, 8, 8, 272),     # GQA group 1, double-buffered
    (64, 16, 2, 0),      # GQA group 8, default split
    (128, 28, 4, 64),    # head_dim 128, one tile
    (128, 28, 4, 256),   # head_dim 128, double-buffered
    (128, 16, 2, 0),     # head_dim 128, GQA group 8, default split
], ids=lambda v: str(v))
def test_fp32_every_layout_matches_oracle(device, d, hq, hkv, tokens_per_split):
    """FP32 on the matrix-core kernel: the fused write equals write-then-decode
    bit for bit, and the decode is within 1e-5 of the oracle."""
    _fused_and_plain_vs_oracle(device, FP32_LENS, hq, hkv, d, tokens_per_split, seed=61 + d,
                               dtype=torch.float32)


# Enough (sequence, split) items that the launcher gives every workgroup a
# pair of KV heads (batch x splits x Hkv/2 at least the GPU's 256 CUs).
# Head_dim 128: one load batch per wave at 128 tokens per split,
# double-buffered at 176.
PAIR128_LENS = [2000, 1, 17, 640, 1999, 129, 700, 1500, 33, 1024, 1100, 385]


@pytest.mark.parametrize("tokens_per_split", [128, 176])
def test_head_dim_128_kv_head_pairs(device, tokens_per_split):
    """Head_dim 128, 28/4 heads."""
    _fused_and_plain_vs_oracle(device, PAIR128_LENS, 28, 4, 128, tokens_per_split, seed=13)


# Head_dim 64 at the default 320-token splits (a fifth tile per wave in LDS):
# 24 sequences up to 3520 tokens (11 splits) with one pair of KV heads, and
# 12 with two pairs.
PAIR64_LENS = [3520, 1, 16, 17, 321, 640, 641, 2999, 3201, 150, 1280, 2048,
               900, 3333, 77, 2500, 319, 320, 1919, 3100, 2222, 1234, 555, 3456]


@pytest.mark.parametrize("hq,hkv,lens", [
    (16, 2, PAIR64_LENS),          # GQA group 8: the merge's 16 query-head rows full
    (14, 2, PAIR64_LENS),          # Qwen2.5-0.5B heads
    (16, 4, PAIR64_LENS[:12]),     # two KV-head pairs per item
], ids=["16x2", "14x2", "16x4"])
def test_head_dim_64_kv_head_pairs(device, hq, hkv, lens):
    _fused_and_plain_vs_oracle(device, lens, hq, hkv, 64, 0, seed=29)


# Seeded random batches of 24-40 sequences with contexts U[1, 4000] (plus a
# 4000-token, a split-boundary and a one-token sequence), sized so the
# launcher takes the KV-head-pair kernels: Qwen2.5-0.5B heads, GQA groups of
# 8 and 4, two KV-head pairs per item (12/4), and head_dim 128.
PAIR_SHAPES = [(14, 2, 64), (16, 2, 64), (8, 2, 64), (12, 4, 64), (28, 4, 128), (14, 2, 64)]


@pytest.mark.parametrize("seed", range(len(PAIR_SHAPES)))
def test_kv_head_pairs_random_batches(device, seed):
    hq, hkv, d = PAIR_SHAPES[seed]
    gen = torch.Generator().manual_seed(1000 + seed)
    batch = int(torch.randint(24, 41, (1,), generator=gen))
    lens = torch.randint(1, 4001, (batch,), generator=gen).tolist()
    lens[:3] = [4000, 320 * (1 + seed % 3), 1]
    _fused_and_plain_vs_oracle(device, lens, hq, hkv, d, 0, seed=200 + seed)


def test_batch_permutation_is_bitwise_invariant(device):
    q, kc, vc, bt, sl, _ = random_paged([64, 129, 1024, 3000, 17], 14, 2, 64, 16,
                                        dtype=torch.bfloat16, seed=9)
    base = run_decode(q, kc, vc, bt, sl, 16, device)
    perm = torch.tensor([3, 0, 4, 2, 1])
    moved = run_decode(q[perm], kc, vc, bt[perm], sl[perm], 16, device)
    assert torch.equal(moved, base[perm.to(device)])


def test_qwen05b_b64_decode_with_write(device):
    """BF16 decode at Qwen2.5-0.5B shape, batch 64, contexts U[128, 4096]."""
    wl = workloads.bf16_decode_qwen05b_b64()
    kc, vc = wl.k_cache.clone(), wl.v_cache.clone()
    kc.view(-1, 2, 64).index_copy_(0, wl.slot_mapping, wl.new_k)
    vc.view(-1, 2, 64).index_copy_(0, wl.slot_mapping, wl.new_v)
    cache = PagedKVCache(1, kc.shape[0], 16, 2, 64, dtype=torch.bfloat16, device=device)
    cache.k_cache[0].copy_(wl.k_cache)
    cache.v_cache[0].copy_(wl.v_cache)
    cache.write_slots(wl.slot_mapping.to(device), wl.new_k.to(device), wl.new_v.to(device))
    k_layer, v_layer = cache.get_layer_cache(0)
    got = kpa.paged_attention_decode_batch_parallel(
        wl.q.to(device), k_layer, v_layer, wl.block_tables.to(device),
        wl.context_lens.to(device), 16)
    want = opa.decode_batch_parallel(wl.q, kc, vc, wl.block_tables, wl.context_lens, 16)
    err = max_abs(got, want)
    print(f"qwen05b_b64 decode max-abs vs oracle: {err:.3e}")
    assert err <= 2e-2


def test_qwen05b_b64_append_step_matches_oracle(device):
    """The timed decode step at full size (batch 64, contexts U[128, 4096]):
    paged_decode_launch with new_k/new_v/slot_mapping, i.e.
    mlr_paged_decode_append, the 64-token KV write folded into the split
    decode. Its cache equals the oracle's write_slots bit for bit, its output
    is within 2e-2 of the oracle's write_slots + decode_batch_parallel on
    every (sequence, head) row, and it equals mlr_kv_write followed by
    mlr_paged_decode on the GPU bit for bit."""
    wl = workloads.bf16_decode_qwen05b_b64()
    kc, vc = wl.k_cache.clone(), wl.v_cache.clone()
    kc.view(-1, 2, 64).index_copy_(0, wl.slot_mapping, wl.new_k)
    vc.view(-1, 2, 64).index_copy_(0, wl.slot_mapping, wl.new_v)
    want = opa.decode_batch_parallel(wl.q, kc, vc, wl.block_tables, wl.context_lens, 16)
    q, bt, sl = wl.q.to(device), wl.block_tables.to(device), wl.context_lens.to(device)
    slots = wl.slot_mapping.to(device)

    fused = PagedKVCache(1, kc.shape[0], 16, 2, 64, dtype=torch.bfloat16, device=device)
    fused.k_cache[0].copy_(wl.k_cache)
    fused.v_cache[0].copy_(wl.v_cache)
    k_layer, v_layer = fused.get_layer_cache(0)
    got = kpa.paged_decode_launch(q, k_layer, v_layer, bt, sl, new_k=wl.new_k.to(device),
                                  new_v=wl.new_v.to(device), slot_mapping=slots)
    assert torch.equal(k_layer.cpu(), kc) and torch.equal(v_layer.cpu(), vc)
    err = max_abs(got, want)
    print(f"qwen05b_b64 append step max-abs vs oracle: {err:.3e}")
    assert torch.isfinite(got).all()
    assert err <= 2e-2

    pair = PagedKVCache(1, kc.shape[0], 16, 2, 64, dtype=torch.bfloat16, device=device)
    pair.k_cache[0].copy_(wl.k_cache)
    pair.v_cache[0].copy_(wl.v_cache)
    pair.write_slots(slots, wl.new_k.to(device), wl.new_v.to(device))
    k2, v2 = pair.get_layer_cache(0)
    assert torch.equal(got, kpa.paged_decode_launch(q, k2, v2, bt, sl))


def _textbook_row(q_row, kc, vc, table, length, kv_head, bs):
    """float64 attention of one query row over one sequence (vectorised)."""
    pos = torch.arange(length)
    blocks = torch.tensor(table)[pos // bs]
    k = kc[blocks, pos % bs, kv_head].double()
    v = vc[blocks, pos % bs, kv_head].double()
    logits = k @ q_row.double() / math.sqrt(q_row.shape[0])
    w = torch.exp(logits - logits.max())
    return ((w / w.sum()) @ v).numpy()


@pytest.fixture(scope="module")
def qwen7b_32k():
    return workloads.bf16_decode_qwen7b_32k()


def _textbook_rows(q, kc, vc, table, length, bs):
    """float64 attention of every query head of one sequence, [Hq, D]."""
    hq, d = q.shape
    hkv = kc.shape[2]
    group = hq // hkv
    pos = torch.arange(length)
    blocks = torch.tensor(table)[pos // bs]
    k = kc[blocks, pos % bs].double()            # [S, Hkv, D]
    v = vc[blocks, pos % bs].double()
    qg = q.double().view(hkv, group, d)          # query head h reads KV head h // group
    logits = torch.einsum("skd,kgd->kgs", k, qg) / math.sqrt(d)
    w = torch.softmax(logits, dim=-1)
    return torch.einsum("kgs,skd->kgd", w, v).reshape(hq, d)


@pytest.fixture(scope="module")
def qwen7b_32k_textbook(qwen7b_32k):
    wl = qwen7b_32k
    return torch.stack([_textbook_rows(wl.q[b], wl.k_cache, wl.v_cache, wl.tables[b],
                                       int(wl.context_lens[b]), 16)
                        for b in range(wl.q.shape[0])])


def test_textbook_rows_match_the_row_form(qwen7b_32k, qwen7b_32k_textbook):
    """The vectorised float64 reference equals the one-row form on a few rows."""
    wl = qwen7b_32k
    for b, h in ((0, 0), (3, 13), (7, 27)):
        one = _textbook_row(wl.q[b, h], wl.k_cache, wl.v_cache, wl.tables[b], 32768, h // 7, 16)
        assert np.abs(qwen7b_32k_textbook[b, h].numpy() - one).max() <= 1e-12


@pytest.mark.parametrize("splits", [4, 8, 16, 32])
def test_qwen7b_32k_split_sweep(device, qwen7b_32k, qwen7b_32k_textbook, splits):
    """BF16 decode at Qwen2.5-7B shape, context 32768, split count swept;
    every (sequence, query head) row against float64 attention."""
    wl = qwen7b_32k
    ts = math.ceil(32768 / splits / 16) * 16
    got = run_decode(wl.q, wl.k_cache, wl.v_cache, wl.block_tables, wl.context_lens, 16,
                     device, tokens_per_split=ts).double().cpu()
    err = (got - qwen7b_32k_textbook).abs()
    print(f"qwen7b_32k splits {splits}: max-abs over {err.shape[0] * err.shape[1]} rows "
          f"{err.max().item():.3e}")
    assert err.max().item() <= 2e-2


@pytest.mark.parametrize(
    "hq,hkv,seq_lens,tables",
    [
        (4, 2, [3, 5], [[2, 0, -1], [1, 3, 4]]),
        (2, 2, [3, 5], [[2, 0, -1], [1, 3, 4]]),
        (4, 1, [3, 5], [[2, 0, -1], [1, 3, 4]]),
        (4, 2, [3, 4], [[2, 0], [1, 3]]),
    ],
    ids=["gqa-ragged", "mha-ragged", "mqa-ragged", "seq-length-equals-heads"],
)
def test_per_request_loop_matches_oracle_loop(device, hq, hkv, seq_lens, tables):
    """paged_attention_decode_batch_reference (the per-request loop, reference
    kernels/reference/paged_attention.py:109-176) against the oracle's loop,
    and equal to the batched decode (tests/kernels/test_paged_attention_batch.py:
    10-43 of the reference)."""
    torch.manual_seed(42)
    q = torch.randn(len(seq_lens), hq, 8)
    kc = torch.randn(5, 2, hkv, 8)
    vc = torch.randn_like(kc)
    want = opa.decode_batch_loop(q, kc, vc, tables, seq_lens, 2)
    got = kpa.paged_attention_decode_batch_reference(
        q.to(device), kc.to(device), vc.to(device), tables, seq_lens, 2)
    assert got.shape == q.shape and got.device.type == "cuda"
    assert max_abs(got, want) <= 1e-5
    batched = run_decode(q, kc, vc, torch.tensor(tables), torch.tensor(seq_lens), 2, device)
    assert max_abs(got, batched) <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_per_request_loop_qwen05b_shape(device, dtype):
    """The per-request loop at Qwen2.5-0.5B head shape on ragged contexts,
    against the oracle loop (1e-5 FP32, 2e-2 BF16)."""
    lens = [1, 17, 300, 1000]
    q, kc, vc, _, _, tables = random_paged(lens, 14, 2, 64, 16, dtype=dtype, seed=31)
    want = opa.decode_batch_loop(q, kc, vc, tables, lens, 16)
    got = kpa.paged_attention_decode_batch_reference(
        q.to(device), kc.to(device), vc.to(device), tables, lens, 16)
    assert torch.isfinite(got).all()
    assert max_abs(got, want) <= TOL[dtype]


@pytest.mark.parametrize("tokens_per_split", [0, 64, 272])
def test_single_launch_merge_reuses_its_workspace(device, tokens_per_split):
    """The matrix-core decode merges a sequence's splits in the same launch
    (the workgroup of the last split waits for the others' partial words in
    the workspace, zero meaning "not written yet"). Five calls with fresh
    inputs on one workspace: each matches the oracle, and the whole workspace
    is back at zero after each."""
    lens = [1, 16, 17, 255, 256, 257, 1000, 2049, 4096, 3000, 40, 700]
    batch, hq, hkv = len(lens), 14, 2
    ws_bytes = kpa.decode_workspace_bytes(batch, hq, 64, 4096, torch.bfloat16,
                                          tokens_per_split)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=device)
    for seed in range(5):
        q, kc, vc, bt, sl, tables = random_paged(lens, hq, hkv, 64, 16, dtype=torch.bfloat16,
                                                 seed=100 + seed)
        width = bt.shape[1]
        bt = torch.nn.functional.pad(bt, (0, 256 - width), value=-1)  # 4096-token tables
        want = opa.decode_batch_loop(q, kc, vc, tables, lens, 16)
        got = kpa.paged_decode_launch(q.to(device), kc.to(device), vc.to(device),
                                      bt.to(device), sl.to(device),
                                      tokens_per_split=tokens_per_split, workspace=ws)
        assert torch.isfinite(got).all()
        assert max_abs(got, want) <= 2e-2, seed
        assert int(torch.count_nonzero(ws)) == 0, seed


def test_single_launch_merge_in_graph_replays(device):
    """A captured decode replayed several times, with new queries copied in
    eagerly between replays: every replay equals an eager call bit for bit
    (the workspace words the merge uses return to zero inside each replay)."""
    lens = [33, 600, 1500, 4000, 257]
    q, kc, vc, bt, sl, _ = random_paged(lens, 14, 2, 64, 16, dtype=torch.bfloat16, seed=77)
    q, kc, vc, bt, sl = (t.to(device) for t in (q, kc, vc, bt, sl))
    out = torch.empty_like(q)
    ws = torch.zeros(kpa.decode_workspace_bytes(5, 14, 64, bt.shape[1] * 16, torch.bfloat16),
                     dtype=torch.uint8, device=device)
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        kpa.paged_decode_launch(q, kc, vc, bt, sl, out, workspace=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        kpa.paged_decode_launch(q, kc, vc, bt, sl, out, workspace=ws)
    gen = torch.Generator().manual_seed(3)
    for _ in range(4):
        q.copy_(torch.randn(q.shape, generator=gen).to(torch.bfloat16).to(device))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = kpa.paged_decode_launch(q, kc, vc, bt, sl)
        assert torch.equal(replayed, eager)


def test_workspace_survives_calls_of_other_shapes(device):
    """One workspace through calls of different batch sizes, head layouts,
    dtypes (the generic kernel writes partials too) and split sizes, large
    then small then large again: every call matches the oracle and the whole
    workspace is zero after each (both kernels return the partial words they
    wrote to zero once merged)."""
    ws = torch.zeros(kpa.decode_workspace_bytes(64, 28, 128, 8192, torch.bfloat16, 16),
                     dtype=torch.uint8, device=device)
    calls = [
        ([4096, 300, 2000, 17] * 8, 14, 2, 64, torch.bfloat16, 0),
        ([40, 900], 14, 2, 64, torch.float32, 16),
        ([33, 257], 8, 8, 64, torch.bfloat16, 16),
        ([700, 1500, 64], 28, 4, 128, torch.bfloat16, 0),
        ([4096, 300, 2000, 17] * 8, 14, 2, 64, torch.bfloat16, 0),
        ([3000, 1] * 16, 14, 2, 64, torch.bfloat16, 64),
    ]
    for i, (lens, hq, hkv, d, dtype, ts) in enumerate(calls):
        q, kc, vc, bt, sl, tables = random_paged(lens, hq, hkv, d, 16, dtype=dtype, seed=40 + i)
        want = opa.decode_batch_loop(q, kc, vc, tables, lens, 16)
        got = kpa.paged_decode_launch(q.to(device), kc.to(device), vc.to(device), bt.to(device),
                                      sl.to(device), tokens_per_split=ts, workspace=ws)
        assert max_abs(got, want) <= TOL[dtype], i
        assert int(torch.count_nonzero(ws)) == 0, i


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_merge_distrusts_a_flagged_workspace(device, dtype):
    """The workspace's first word is what a merge that waited past its limit
    leaves behind (set here from the host; every kernel exits normally).
    Such a workspace is not trusted: every sequence whose splits are merged
    gets NaN, and sequences that fit one split are still exact."""
    lens = [100, 1000, 3000, 320, 321, 17]
    ts = 320
    q, kc, vc, bt, sl, tables = random_paged(lens, 14, 2, 64, 16, dtype=dtype, seed=5)
    ws = torch.zeros(kpa.decode_workspace_bytes(len(lens), 14, 64, bt.shape[1] * 16,
                                                dtype, ts),
                     dtype=torch.uint8, device=device)
    ws[:4].view(torch.int32).fill_(1)
    got = kpa.paged_decode_launch(q.to(device), kc.to(device), vc.to(device), bt.to(device),
                                  sl.to(device), tokens_per_split=ts, workspace=ws)
    want = opa.decode_batch_loop(q, kc, vc, tables, lens, 16)
    got = got.float().cpu()
    for i, n in enumerate(lens):
        if n <= ts:
            assert max_abs(got[i], want[i]) <= TOL[dtype], i
        else:
            assert torch.isnan(got[i]).all(), i


def _flag_case(device):
    lens = [100, 1000, 3000, 320, 321, 17]
    q, kc, vc, bt, sl, tables = random_paged(lens, 14, 2, 64, 16, dtype=torch.bfloat16, seed=5)
    want = opa.decode_batch_loop(q, kc, vc, tables, lens, 16)
    args = tuple(t.to(device) for t in (q, kc, vc, bt, sl))
    return lens, args, want


def test_flagged_workspace_is_reported_and_cleared(device):
    """mlr_paged_decode_workspace_check on a workspace whose merge-failure
    flag is set (from the host, as a merge that waited past its limit would
    leave it; every kernel exits normally): it raises DecodeMergeError, the
    whole workspace is zero afterwards (the flag and the partial rows the
    distrusting merges left behind), and the next decode on it is exact.
    A clean workspace passes."""
    lens, args, want = _flag_case(device)
    ts = 320
    ws = torch.zeros(kpa.decode_workspace_bytes(len(lens), 14, 64, args[3].shape[1] * 16,
                                                torch.bfloat16, ts),
                     dtype=torch.uint8, device=device)
    kpa.check_workspace(ws)  # clean: no error
    ws[:4].view(torch.int32).fill_(1)
    got = kpa.paged_decode_launch(*args, tokens_per_split=ts, workspace=ws)
    assert torch.isnan(got[1]).all()
    assert int(torch.count_nonzero(ws[256:])) > 0  # partials of distrusted merges
    with pytest.raises(kpa.DecodeMergeError, match="gave up waiting"):
        kpa.check_workspace(ws)
    assert int(torch.count_nonzero(ws)) == 0
    kpa.check_workspace(ws)
    got = kpa.paged_decode_launch(*args, tokens_per_split=ts, workspace=ws)
    assert max_abs(got, want) <= 2e-2
    assert int(torch.count_nonzero(ws)) == 0


def test_cached_workspace_flag_raises_in_the_step_check(device):
    """The per-stream workspace the Python layer keeps: a set flag makes
    check_decode_workspaces (called by run_generation_step once per step)
    raise DecodeMergeError; the workspace is cleared and later calls are
    exact. The test runs on a stream of its own, so its cached workspace is
    the one it flags."""
    lens, args, want = _flag_case(device)
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        kpa.paged_decode_launch(*args, tokens_per_split=320)
        ws = kpa.decode_workspace(device, 256)  # this stream's cached workspace
        ws[:4].view(torch.int32).fill_(1)
        got = kpa.paged_decode_launch(*args, tokens_per_split=320)
        assert torch.isnan(got[1]).all()
        with pytest.raises(kpa.DecodeMergeError):
            kpa.check_decode_workspaces(device)
        assert int(torch.count_nonzero(ws)) == 0
        kpa.check_decode_workspaces(device)
        got = kpa.paged_decode_launch(*args, tokens_per_split=320)
        assert max_abs(got, want) <= 2e-2
    torch.cuda.synchronize()


def test_workspace_check_is_refused_under_capture(device):
    """The check synchronises the host, so it refuses a stream under graph
    capture (before touching the stream) instead of breaking the capture."""
    ws = torch.zeros(4096, dtype=torch.uint8, device=device)
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        with pytest.raises(RuntimeError, match="captured"):
            kpa.check_workspace(ws)
        ws.add_(0)  # keeps the graph non-empty
    torch.cuda.synchronize()


def test_cached_workspace_under_graph_capture(device):
    """Decode without workspace= inside graph capture. A cached workspace that
    is too small is not replaced inside the capture (that would record only
    its zero fill, leaving it uninitialised until a replay): the call raises
    and asks for an eager call first. After an eager call of the captured
    size on the same stream, capture uses the cached workspace, and every
    replay (new queries copied in eagerly between replays) equals an eager
    call bit for bit. A workspace that a larger one replaced stays allocated
    (graphs captured on it keep a live address)."""
    small = [40, 700]
    big = [33, 600, 1500, 4000, 257]
    qs, kcs, vcs, bts, sls, _ = random_paged(small, 14, 2, 64, 16, dtype=torch.bfloat16, seed=76)
    q, kc, vc, bt, sl, _ = random_paged(big, 14, 2, 64, 16, dtype=torch.bfloat16, seed=77)
    qs, kcs, vcs, bts, sls = (t.to(device) for t in (qs, kcs, vcs, bts, sls))
    q, kc, vc, bt, sl = (t.to(device) for t in (q, kc, vc, bt, sl))
    out = torch.empty_like(q)
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        kpa.paged_decode_launch(qs, kcs, vcs, bts, sls)  # caches a small workspace
        small_ws = kpa.decode_workspace(device, 256)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        with pytest.raises(RuntimeError, match="eager call"):
            kpa.paged_decode_launch(q, kc, vc, bt, sl, out)
        out.add_(0)  # keeps the graph non-empty
    with torch.cuda.stream(stream):
        kpa.paged_decode_launch(q, kc, vc, bt, sl, out)  # grows the cached workspace
        grown = kpa.decode_workspace(device, 256)
    torch.cuda.synchronize()
    assert grown.numel() > small_ws.numel()
    assert any(r is small_ws for r in kpa._RETIRED)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        kpa.paged_decode_launch(q, kc, vc, bt, sl, out)
    gen = torch.Generator().manual_seed(4)
    for _ in range(4):
        q.copy_(torch.randn(q.shape, generator=gen).to(torch.bfloat16).to(device))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = kpa.paged_decode_launch(q, kc, vc, bt, sl)
        assert torch.equal(replayed, eager)
