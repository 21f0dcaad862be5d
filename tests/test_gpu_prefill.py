"""Paged chunk prefill on the GPU against the oracle's tiled restatement (CPU).

Tolerances (max-abs): 1e-5 for FP32/FP64, 2e-2 for BF16/FP16 (FP32 softmax).
Pools are NaN-filled outside the written context, so a stray read fails.
"""

from __future__ import annotations

import itertools

import pytest
import torch

import oracle.paged_attention as opa
from mini_llm_runtime_amd import workloads
from mini_llm_runtime_amd.kernels import paged_attention as kpa
from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache
from oracle_pins import build_pool

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.float64: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def max_abs(a, b):
    return (a.double().cpu() - b.double().cpu()).abs().max().item()


def make_case(hq, hkv, prefix, chunk, d, bs, dtype, seed, spare=2):
    gen = torch.Generator().manual_seed(seed)
    context = prefix + chunk
    n_blocks = (context + bs - 1) // bs
    table = torch.randperm(n_blocks + spare, generator=gen)[:n_blocks].tolist()
    k = torch.randn(context, hkv, d, generator=gen).to(dtype)
    v = torch.randn(context, hkv, d, generator=gen).to(dtype)
    q = torch.randn(chunk, hq, d, generator=gen).to(dtype)
    kc, vc = build_pool(k, v, table, bs, n_blocks + spare)
    return q, kc, vc, table


@pytest.mark.parametrize("hq,hkv", [(2, 2), (4, 2), (4, 1)], ids=["mha", "gqa", "mqa"])
@pytest.mark.parametrize("prefix", [0, 5], ids=["first-chunk", "with-prefix"])
@pytest.mark.parametrize("tile", [1, 4, 16])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_reference_chunk_grid(device, hq, hkv, prefix, tile, dtype):
    # The reference's grid (tests/kernels/test_paged_attention.py:249-351).
    q, kc, vc, table = make_case(hq, hkv, prefix, 4, 8, 3, dtype, seed=0)
    want = opa.prefill_chunk_tiled(q, kc, vc, table, prefix, prefix + 4, 3, tile)
    got = kpa.paged_attention_prefill_chunk_tiled(
        q.to(device), kc.to(device), vc.to(device), table, prefix, prefix + 4, 3, tile)
    assert got.shape == q.shape and got.dtype == q.dtype
    assert torch.isfinite(got).all()
    assert max_abs(got, want) <= TOL[dtype]


CASES = [
    # (dtype, hq, hkv, d, bs, prefix, chunk, tile)
    (torch.bfloat16, 14, 2, 64, 16, 0, 512, 64),
    (torch.bfloat16, 14, 2, 64, 16, 1000, 77, 128),
    (torch.bfloat16, 28, 4, 128, 16, 300, 200, 16),
    (torch.bfloat16, 8, 8, 64, 32, 17, 100, 64),
    (torch.float16, 14, 2, 64, 16, 100, 130, 64),                  # fp16 matrix cores
    (torch.float16, 28, 4, 128, 16, 300, 200, 16),                 # fp16, D=128
    (torch.float16, 8, 8, 64, 32, 17, 100, 64),                    # fp16, G=1, BS=32
    (torch.float16, 14, 2, 64, 16, 1000, 77, 128),
    (torch.float32, 14, 2, 64, 16, 250, 70, 64),                   # FP32 matrix cores
    (torch.float32, 28, 4, 128, 16, 300, 200, 16),                 # FP32, D=128
    (torch.float32, 8, 8, 64, 32, 17, 100, 64),                    # FP32, G=1, BS=32
    (torch.float32, 14, 2, 64, 16, 1000, 77, 128),
    (torch.float32, 6, 3, 40, 5, 11, 29, 7),
    (torch.float64, 4, 2, 16, 4, 9, 13, 4),
]


@pytest.mark.parametrize("dtype,hq,hkv,d,bs,prefix,chunk,tile", CASES,
                         ids=[f"{str(c[0])[6:]}-{c[1]}x{c[2]}-d{c[3]}-p{c[5]}-c{c[6]}"
                              for c in CASES])
def test_chunk_matches_oracle(device, dtype, hq, hkv, d, bs, prefix, chunk, tile):
    q, kc, vc, table = make_case(hq, hkv, prefix, chunk, d, bs, dtype, seed=chunk)
    want = opa.prefill_chunk_tiled(q, kc, vc, table, prefix, prefix + chunk, bs, tile)
    got = kpa.paged_attention_prefill_chunk_tiled(
        q.to(device), kc.to(device), vc.to(device), table, prefix, prefix + chunk, bs, tile)
    assert torch.isfinite(got).all()
    assert max_abs(got, want) <= TOL[dtype]


@pytest.mark.parametrize("tile", [16, 64, 128])
def test_chunk512_x8_varlen_with_kv_write(device, tile):
    """BF16 chunk prefill, 8 sequences x 512-token chunk, prefixes U[0, 3584]."""
    wl = workloads.bf16_prefill_chunk512_x8()
    nb = wl.k_cache.shape[0]
    cache = PagedKVCache(1, nb, 16, 2, 64, dtype=torch.bfloat16, device=device)
    cache.k_cache[0].copy_(wl.k_cache)
    cache.v_cache[0].copy_(wl.v_cache)
    cache.write_slots(wl.slot_mapping.to(device), wl.chunk_k.to(device),
                      wl.chunk_v.to(device))
    kc, vc = wl.k_cache.clone(), wl.v_cache.clone()
    kc.view(-1, 2, 64).index_copy_(0, wl.slot_mapping, wl.chunk_k)
    vc.view(-1, 2, 64).index_copy_(0, wl.slot_mapping, wl.chunk_v)
    assert torch.equal(cache.k_cache[0].cpu(), kc)
    k_layer, v_layer = cache.get_layer_cache(0)
    got = kpa.paged_attention_prefill_varlen(
        wl.q.to(device), k_layer, v_layer, wl.block_tables.to(device),
        wl.query_start_loc.to(device), wl.context_lens.to(device), 16, tile).cpu()
    worst = 0.0
    for s in range(len(wl.prefix_lens)):  # every sequence of the batch
        lo, hi = int(wl.query_start_loc[s]), int(wl.query_start_loc[s + 1])
        p = wl.prefix_lens[s]
        want = opa.prefill_chunk_tiled(wl.q[lo:hi], kc, vc, wl.tables[s], p, p + hi - lo,
                                       16, tile)
        worst = max(worst, max_abs(got[lo:hi], want))
    print(f"chunk512_x8 tile {tile}: max-abs vs oracle over all {len(wl.prefix_lens)} "
          f"sequences {worst:.3e}")
    assert worst <= 2e-2


def test_varlen_equals_per_sequence_calls(device):
    """Packing sequences into one launch changes nothing, bit for bit."""
    wl = workloads.bf16_prefill_chunk512_x8(num_seqs=3, chunk=96, max_prefix=300)
    kc, vc = wl.k_cache.clone(), wl.v_cache.clone()
    kc.view(-1, 2, 64).index_copy_(0, wl.slot_mapping, wl.chunk_k)
    vc.view(-1, 2, 64).index_copy_(0, wl.slot_mapping, wl.chunk_v)
    kc, vc = kc.to(device), vc.to(device)
    packed = kpa.paged_attention_prefill_varlen(
        wl.q.to(device), kc, vc, wl.block_tables.to(device), wl.query_start_loc.to(device),
        wl.context_lens.to(device), 16, 64)
    for s in range(3):
        lo, hi = int(wl.query_start_loc[s]), int(wl.query_start_loc[s + 1])
        p = wl.prefix_lens[s]
        single = kpa.paged_attention_prefill_chunk_tiled(
            wl.q[lo:hi].to(device), kc, vc, wl.tables[s], p, p + hi - lo, 16, 64)
        assert torch.equal(single, packed[lo:hi])


# BF16 shapes at the edges of the matrix-core kernel's tiling: 32-query waves,
# 128-query workgroups, 64-key tiles, 16-row copy spans and blocks larger
# than a key tile.
EDGE_CASES = [
    # (hq, hkv, d, bs, prefix, chunk)
    (14, 2, 64, 16, 0, 1),
    (14, 2, 64, 16, 3, 31),
    (8, 1, 64, 64, 64, 129),
    (16, 2, 128, 256, 700, 300),
    (8, 8, 128, 32, 1, 257),
    (4, 2, 64, 128, 4095, 65),
]


@pytest.mark.parametrize("hq,hkv,d,bs,prefix,chunk", EDGE_CASES,
                         ids=[f"{c[0]}x{c[1]}-d{c[2]}-bs{c[3]}-p{c[4]}-c{c[5]}"
                              for c in EDGE_CASES])
def test_bf16_tiling_edges_match_oracle(device, hq, hkv, d, bs, prefix, chunk):
    q, kc, vc, table = make_case(hq, hkv, prefix, chunk, d, bs, torch.bfloat16,
                                 seed=prefix + chunk)
    want = opa.prefill_chunk_tiled(q, kc, vc, table, prefix, prefix + chunk, bs, 64)
    got = kpa.paged_attention_prefill_chunk_tiled(
        q.to(device), kc.to(device), vc.to(device), table, prefix, prefix + chunk, bs, 64)
    assert torch.isfinite(got).all()
    assert max_abs(got, want) <= 2e-2


@pytest.mark.parametrize("hq,hkv,d,bs,prefix,chunk", EDGE_CASES,
                         ids=[f"{c[0]}x{c[1]}-d{c[2]}-bs{c[3]}-p{c[4]}-c{c[5]}"
                              for c in EDGE_CASES])
def test_fp16_tiling_edges_match_oracle(device, hq, hkv, d, bs, prefix, chunk):
    """The same tiling edges in fp16 (the matrix-core kernel's fp16 operands)."""
    q, kc, vc, table = make_case(hq, hkv, prefix, chunk, d, bs, torch.float16,
                                 seed=prefix + chunk)
    want = opa.prefill_chunk_tiled(q, kc, vc, table, prefix, prefix + chunk, bs, 64)
    got = kpa.paged_attention_prefill_chunk_tiled(
        q.to(device), kc.to(device), vc.to(device), table, prefix, prefix + chunk, bs, 64)
    assert torch.isfinite(got).all()
    assert max_abs(got, want) <= 2e-2


@pytest.mark.parametrize("hq,hkv,d,bs,prefix,chunk", EDGE_CASES,
                         ids=[f"{c[0]}x{c[1]}-d{c[2]}-bs{c[3]}-p{c[4]}-c{c[5]}"
                              for c in EDGE_CASES])
def test_fp32_tiling_edges_match_oracle(device, hq, hkv, d, bs, prefix, chunk):
    """The same tiling edges in FP32 (the FP32 matrix-core kernel: 16-query
    waves, 64-query workgroups, 16-key blocks), within 1e-5."""
    q, kc, vc, table = make_case(hq, hkv, prefix, chunk, d, bs, torch.float32,
                                 seed=prefix + chunk)
    want = opa.prefill_chunk_tiled(q, kc, vc, table, prefix, prefix + chunk, bs, 64)
    got = kpa.paged_attention_prefill_chunk_tiled(
        q.to(device), kc.to(device), vc.to(device), table, prefix, prefix + chunk, bs, 64)
    assert torch.isfinite(got).all()
    assert max_abs(got, want) <= 1e-5


def test_bf16_ragged_varlen_matches_oracle(device):
    """One launch over sequences of 1..300 queries with unrelated prefixes."""
    hq, hkv, d, bs = 14, 2, 64, 16
    qlens, prefixes = [1, 33, 128, 300, 7, 129], [0, 100, 5, 1000, 63, 2047]
    gen = torch.Generator().manual_seed(11)
    ctxs = [p + c for p, c in zip(prefixes, qlens)]
    nblk = [(c + bs - 1) // bs for c in ctxs]
    total_blocks = sum(nblk) + 3
    perm = torch.randperm(total_blocks, generator=gen).tolist()
    tables, at = [], 0
    for n in nblk:
        tables.append(perm[at:at + n])
        at += n
    kc = torch.full((total_blocks, bs, hkv, d), float("nan"), dtype=torch.bfloat16)
    vc = torch.full_like(kc, float("nan"))
    qs = []
    for s, ctx in enumerate(ctxs):
        k = torch.randn(ctx, hkv, d, generator=gen).to(torch.bfloat16)
        v = torch.randn(ctx, hkv, d, generator=gen).to(torch.bfloat16)
        for pos in range(ctx):
            kc[tables[s][pos // bs], pos % bs] = k[pos]
            vc[tables[s][pos // bs], pos % bs] = v[pos]
        qs.append(torch.randn(qlens[s], hq, d, generator=gen).to(torch.bfloat16))
    q = torch.cat(qs)
    width = max(nblk)
    bt = torch.tensor([t + [0] * (width - len(t)) for t in tables], dtype=torch.long)
    qsl = torch.tensor([0] + list(itertools.accumulate(qlens)), dtype=torch.long)
    got = kpa.paged_attention_prefill_varlen(
        q.to(device), kc.to(device), vc.to(device), bt.to(device), qsl.to(device),
        torch.tensor(ctxs, dtype=torch.long).to(device), bs, 64).cpu()
    for s in range(len(qlens)):
        lo, hi = int(qsl[s]), int(qsl[s + 1])
        want = opa.prefill_chunk_tiled(q[lo:hi], kc, vc, tables[s], prefixes[s], ctxs[s], bs, 64)
        assert max_abs(got[lo:hi], want) <= 2e-2, f"sequence {s}"


@pytest.mark.parametrize("num_seqs", [40, 300])
def test_bf16_many_sequences_match_oracle(device, num_seqs):
    """Workgroups past twice the CU count (40 sequences: 1120 workgroups, the
    rank pairing covers only the first 2 x CUs) and more work items than the
    prologue ranks (300 sequences x 2 query tiles: the unranked order). Every
    (sequence, head) must still be computed exactly once."""
    hq, hkv, d, bs = 14, 2, 64, 16
    gen = torch.Generator().manual_seed(num_seqs)
    qlens = torch.randint(1, 201, (num_seqs,), generator=gen).tolist()
    prefixes = torch.randint(0, 501, (num_seqs,), generator=gen).tolist()
    ctxs = [p + c for p, c in zip(prefixes, qlens)]
    nblk = [(c + bs - 1) // bs for c in ctxs]
    total_blocks = sum(nblk) + 3
    perm = torch.randperm(total_blocks, generator=gen).tolist()
    tables, at = [], 0
    for n in nblk:
        tables.append(perm[at:at + n])
        at += n
    kc = torch.full((total_blocks, bs, hkv, d), float("nan"), dtype=torch.bfloat16)
    vc = torch.full_like(kc, float("nan"))
    qs = []
    for s, ctx in enumerate(ctxs):
        pos = torch.arange(ctx)
        blocks = torch.tensor(tables[s])[pos // bs]
        kc[blocks, pos % bs] = torch.randn(ctx, hkv, d, generator=gen).to(torch.bfloat16)
        vc[blocks, pos % bs] = torch.randn(ctx, hkv, d, generator=gen).to(torch.bfloat16)
        qs.append(torch.randn(qlens[s], hq, d, generator=gen).to(torch.bfloat16))
    q = torch.cat(qs)
    width = max(nblk)
    bt = torch.tensor([t + [-1] * (width - len(t)) for t in tables], dtype=torch.long)
    qsl = torch.tensor([0] + list(itertools.accumulate(qlens)), dtype=torch.long)
    got = kpa.paged_attention_prefill_varlen(
        q.to(device), kc.to(device), vc.to(device), bt.to(device), qsl.to(device),
        torch.tensor(ctxs, dtype=torch.long).to(device), bs, 64).cpu()
    assert torch.isfinite(got).all()
    for s in range(num_seqs):
        lo, hi = int(qsl[s]), int(qsl[s + 1])
        want = opa.prefill_chunk_tiled(q[lo:hi], kc, vc, tables[s], prefixes[s], ctxs[s], bs, 64)
        assert max_abs(got[lo:hi], want) <= 2e-2, f"sequence {s}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("d,bs", [(64, 16), (128, 32), (40, 5)], ids=["d64", "d128", "generic"])
def test_out_of_range_block_masks_its_tokens(device, d, bs, dtype):
    """An out-of-range block id in the table hides that block's keys."""
    from oracle import textbook
    hq, hkv, prefix, chunk = 4, 2, 70, 40
    q, kc, vc, table = make_case(hq, hkv, prefix, chunk, d, bs, dtype, seed=5)
    bad_blk = 1  # a prefix block: its keys are visible to every query
    context = prefix + chunk
    visible = [[j <= prefix + i and j // bs != bad_blk for j in range(context)]
               for i in range(chunk)]
    want = torch.zeros(chunk, hq, d, dtype=torch.float64)
    for h in range(hq):
        k, v = textbook.logical_kv(kc.float().numpy(), vc.float().numpy(), table, context,
                                   h // (hq // hkv))
        want[:, h] = torch.from_numpy(textbook.attend(q[:, h].float().numpy(), k, v, visible))
    broken = list(table)
    broken[bad_blk] = kc.shape[0] + 7
    bt = torch.tensor([broken], dtype=torch.long)
    got = kpa.paged_prefill_launch(
        q.to(device), kc.to(device), vc.to(device), bt.to(device),
        torch.tensor([0, chunk], dtype=torch.long).to(device),
        torch.tensor([context], dtype=torch.long).to(device), chunk).cpu()
    assert torch.isfinite(got).all()
    assert max_abs(got, want) <= TOL[dtype]
