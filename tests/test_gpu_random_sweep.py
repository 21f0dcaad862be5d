"""Seeded random shapes through the decode and prefill kernels, against the
oracle on the CPU.

Each case draws its dtype, head_dim, KV heads, GQA group, block size, batch,
context lengths and split size from its seed, so together the cases cross the
matrix-core and generic kernels, one and two KV heads per workgroup, every
load-batch layout and the in-launch merge of up to hundreds of splits. Decode
cases with the fused KV write also check that the write and the output equal
write-then-decode bit for bit. Every case names its shape in its failure
message.

Tolerances. Decode: max-abs 1e-5 for FP32 and 2e-2 for BF16 and FP16 against
the oracle, as elsewhere (the kernel rounds scores and probabilities as the
reference does). Prefill, FP32: max-abs 1e-5 against the oracle. Prefill,
BF16: the kernel and the reference round differently (the reference rounds
q.k to bf16, the kernel rounds q * scale * log2(e) and P), and random shapes
reach outputs far larger than the configured workloads do: a query with a
one-token prefix sees one or two keys, and its output is a V row itself, up
to about 3.5. There two roundings that are each within bf16 resolution of
the exact result can differ by more than 2e-2 (measured on the CPU for one
such case: oracle 0.019 from float64 attention, an emulation of the kernel's
roundings 0.0085). So each element is checked against float64 attention
within 2e-2 plus half a bf16 ulp of its value (2^-8 |x|), and against the
oracle within 2e-2 plus one ulp (2^-7 |x|). The fp16 sweep draws the same
kinds of shapes in fp16, with fp16's half ulp and ulp (2^-11, 2^-10).
"""

from __future__ import annotations

import itertools

import pytest
import torch

import oracle.paged_attention as opa
from mini_llm_runtime_amd.kernels import paged_attention as kpa
from oracle_pins import random_paged

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def max_abs(a, b):
    return (a.double().cpu() - b.double().cpu()).abs().max().item()


def pick(gen, values):
    return values[int(torch.randint(len(values), (1,), generator=gen))]


def decode_case(seed):
    gen = torch.Generator().manual_seed(7000 + seed)
    dtype = pick(gen, [torch.bfloat16, torch.bfloat16, torch.float32, torch.float32,
                       torch.float16])
    d = pick(gen, [64, 64, 128, 128, 96])
    hkv = pick(gen, [1, 2, 2, 4, 8])
    group = pick(gen, [1, 2, 4, 7, 8, 16])
    bs = pick(gen, [16, 16, 32, 64, 8])
    batch = int(torch.randint(1, 13, (1,), generator=gen))
    lens = torch.randint(1, 3001, (batch,), generator=gen).tolist()
    ts = pick(gen, [0, 0, 16, 48, 64, 128, 256, 272, 320, 384, 512])
    lens[0] = pick(gen, [1, bs, bs + 1, max(ts, 1), ts + 1, 3000])
    fused = bool(torch.randint(2, (1,), generator=gen))
    return dict(dtype=dtype, d=d, hkv=hkv, hq=hkv * group, bs=bs, lens=lens, ts=ts,
                fused=fused)


@pytest.mark.parametrize("seed", range(64))
def test_random_decode_matches_oracle(device, seed):
    c = decode_case(seed)
    what = (f"seed {seed}: {str(c['dtype'])[6:]} d{c['d']} {c['hq']}x{c['hkv']} bs{c['bs']} "
            f"ts{c['ts']} fused={c['fused']} lens={c['lens']}")
    dtype, d, hq, hkv, bs, lens, ts = (c[k] for k in ("dtype", "d", "hq", "hkv", "bs", "lens",
                                                      "ts"))
    q, kc, vc, bt, sl, tables = random_paged(lens, hq, hkv, d, bs, dtype=dtype, seed=seed,
                                             fill=0.0 if c["fused"] else float("nan"))
    q, bt, sl = (t.to(device) for t in (q, bt, sl))
    if not c["fused"]:
        got = kpa.paged_decode_launch(q, kc.to(device), vc.to(device), bt, sl,
                                      tokens_per_split=ts)
        want = opa.decode_batch_loop(q.cpu(), kc, vc, tables, lens, bs)
        assert torch.isfinite(got).all(), what
        assert max_abs(got, want) <= TOL[dtype], what
        return
    gen = torch.Generator().manual_seed(seed + 1)
    new_k = torch.randn(len(lens), hkv, d, generator=gen).to(dtype).to(device)
    new_v = torch.randn(len(lens), hkv, d, generator=gen).to(dtype).to(device)
    slots = torch.tensor([tables[b][(n - 1) // bs] * bs + (n - 1) % bs
                          for b, n in enumerate(lens)], device=device)
    k1, v1 = kc.to(device), vc.to(device)
    k2, v2 = kc.to(device), vc.to(device)
    fused = kpa.paged_decode_launch(q, k1, v1, bt, sl, new_k=new_k, new_v=new_v,
                                    slot_mapping=slots, tokens_per_split=ts)
    k2.view(-1, hkv, d).index_copy_(0, slots, new_k)
    v2.view(-1, hkv, d).index_copy_(0, slots, new_v)
    plain = kpa.paged_decode_launch(q, k2, v2, bt, sl, tokens_per_split=ts)
    assert torch.equal(k1, k2) and torch.equal(v1, v2), what
    assert torch.equal(fused, plain), what
    want = opa.decode_batch_loop(q.cpu(), k2.cpu(), v2.cpu(), tables, lens, bs)
    assert torch.isfinite(plain).all(), what
    assert max_abs(plain, want) <= TOL[dtype], what


def exact_prefill(q, k, v, prefix):
    """Float64 causal attention of q [C, Hq, D] over the logical rows k, v
    [prefix + C, Hkv, D] (query i sees keys 0 .. prefix + i)."""
    chunk, hq, d = q.shape
    group = hq // k.shape[1]
    kd = k.double().repeat_interleave(group, dim=1)
    vd = v.double().repeat_interleave(group, dim=1)
    scores = torch.einsum("chd,khd->hck", q.double(), kd) / d ** 0.5
    hidden = torch.arange(k.shape[0])[None, :] > (prefix + torch.arange(chunk))[:, None]
    scores.masked_fill_(hidden, float("-inf"))
    return torch.einsum("hck,khd->chd", torch.softmax(scores, dim=-1), vd)


def prefill_case(seed):
    gen = torch.Generator().manual_seed(9000 + seed)
    dtype = pick(gen, [torch.bfloat16, torch.bfloat16, torch.bfloat16, torch.float32])
    d = pick(gen, [64, 64, 128, 40])
    hkv = pick(gen, [1, 2, 4])
    group = pick(gen, [1, 2, 7, 8])
    bs = pick(gen, [16, 32, 64, 5])
    nseq = int(torch.randint(1, 7, (1,), generator=gen))
    qlens = torch.randint(1, 401, (nseq,), generator=gen).tolist()
    prefixes = torch.randint(0, 2001, (nseq,), generator=gen).tolist()
    prefixes[0] = pick(gen, [0, 1, 63, 64, 65, prefixes[0]])
    tile = pick(gen, [16, 64, 128])
    return dict(dtype=dtype, d=d, hkv=hkv, hq=hkv * group, bs=bs, qlens=qlens,
                prefixes=prefixes, tile=tile)


@pytest.mark.parametrize("seed", range(32))
def test_random_varlen_prefill_matches_oracle(device, seed):
    _check_random_prefill(device, seed, prefill_case(seed))


@pytest.mark.parametrize("seed", range(12))
def test_random_varlen_prefill_fp16_matches_oracle(device, seed):
    """The same draws in fp16: the matrix-core kernel with fp16 operands, or
    the generic kernel where the shape sends it there."""
    c = prefill_case(100 + seed)
    c["dtype"] = torch.float16
    _check_random_prefill(device, seed, c)


# Half a unit and one unit in the last place of each 16-bit type, relative.
HALF_ULP = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}


def _check_random_prefill(device, seed, c):
    dtype, d, hq, hkv, bs = (c[k] for k in ("dtype", "d", "hq", "hkv", "bs"))
    qlens, prefixes, tile = c["qlens"], c["prefixes"], c["tile"]
    what = (f"seed {seed}: {str(dtype)[6:]} d{d} {hq}x{hkv} bs{bs} tile{tile} "
            f"qlens={qlens} prefixes={prefixes}")
    gen = torch.Generator().manual_seed(seed)
    ctxs = [p + n for p, n in zip(prefixes, qlens)]
    nblk = [-(-x // bs) for x in ctxs]
    total_blocks = sum(nblk) + 2
    perm = torch.randperm(total_blocks, generator=gen).tolist()
    tables, at = [], 0
    for n in nblk:
        tables.append(perm[at:at + n])
        at += n
    kc = torch.full((total_blocks, bs, hkv, d), float("nan"), dtype=dtype)
    vc = torch.full_like(kc, float("nan"))
    qs, rows = [], []
    for s, ctx in enumerate(ctxs):
        pos = torch.arange(ctx)
        blocks = torch.tensor(tables[s])[pos // bs]
        k = torch.randn(ctx, hkv, d, generator=gen).to(dtype)
        v = torch.randn(ctx, hkv, d, generator=gen).to(dtype)
        kc[blocks, pos % bs] = k
        vc[blocks, pos % bs] = v
        rows.append((k, v))
        qs.append(torch.randn(qlens[s], hq, d, generator=gen).to(dtype))
    q = torch.cat(qs)
    width = max(nblk)
    bt = torch.tensor([t + [-1] * (width - len(t)) for t in tables], dtype=torch.long)
    qsl = torch.tensor([0] + list(itertools.accumulate(qlens)), dtype=torch.long)
    got = kpa.paged_attention_prefill_varlen(
        q.to(device), kc.to(device), vc.to(device), bt.to(device), qsl.to(device),
        torch.tensor(ctxs, dtype=torch.long).to(device), bs, tile).cpu()
    assert torch.isfinite(got).all(), what
    for s in range(len(qlens)):
        lo, hi = int(qsl[s]), int(qsl[s + 1])
        want = opa.prefill_chunk_tiled(q[lo:hi], kc, vc, tables[s], prefixes[s], ctxs[s], bs,
                                       tile)
        mine = got[lo:hi].double()
        if dtype == torch.float32:
            assert max_abs(mine, want) <= TOL[dtype], f"{what}: sequence {s}"
            continue
        exact = exact_prefill(q[lo:hi], *rows[s], prefixes[s])
        want = want.double()
        half = HALF_ULP[dtype]
        err_exact = ((mine - exact).abs() - (2e-2 + half * exact.abs())).max().item()
        err_oracle = ((mine - want).abs() - (2e-2 + 2 * half * want.abs())).max().item()
        assert err_exact <= 0, f"{what}: sequence {s} exceeds the bar against float64 " \
                               f"by {err_exact:.3g}"
        assert err_oracle <= 0, f"{what}: sequence {s} exceeds the bar against the oracle " \
                                f"by {err_oracle:.3g}"
