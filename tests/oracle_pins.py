"""Checks that pin the oracle's attention restatements to independent answers.

Each ``check_*`` takes an oracle module (``oracle.paged_attention`` or a
mutant of it) and raises AssertionError when the module disagrees with:
- the reference's stored masked-SDPA known answer (tests/golden), or
- the float64 textbook attention of ``oracle.textbook`` on paged layouts.
tests/test_oracle_pins.py runs them on the oracle; tests/test_oracle_mutants.py
plants mistakes in copies of the oracle and requires every mistake to fail.
"""

from __future__ import annotations

import os
import types

import numpy as np
import torch

from oracle import textbook

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_kat():
    with np.load(os.path.join(GOLDEN, "sdpa_known_answer.npz"), allow_pickle=False) as z:
        return {name: np.array(z[name]) for name in z.files}


def build_pool(logical_k, logical_v, block_table, block_size, num_blocks, fill=float("nan")):
    """Scatter logical [S, Hkv, D] rows into a NaN-filled [NB, BS, Hkv, D] pool."""
    shape = (num_blocks, block_size) + tuple(logical_k.shape[1:])
    k_cache = torch.full(shape, fill, dtype=logical_k.dtype)
    v_cache = torch.full(shape, fill, dtype=logical_v.dtype)
    for pos in range(logical_k.shape[0]):
        blk = block_table[pos // block_size]
        k_cache[blk, pos % block_size] = logical_k[pos]
        v_cache[blk, pos % block_size] = logical_v[pos]
    return k_cache, v_cache


def kat_rows():
    """(q [1,64], visible K [n,1,64], visible V [n,1,64], expected [64]) per KAT row."""
    kat = load_kat()
    rows = []
    for b in range(kat["q"].shape[0]):
        for i in range(kat["q"].shape[1]):
            cols = np.nonzero(kat["mask"][b, i])[0]
            rows.append((torch.from_numpy(kat["q"][b, i][None, :]),
                         torch.from_numpy(kat["k"][b, cols][:, None, :]),
                         torch.from_numpy(kat["v"][b, cols][:, None, :]),
                         kat["expected"][b, i]))
    return rows


def _table(n_blocks, num_blocks, gen):
    return torch.randperm(num_blocks, generator=gen)[:n_blocks].tolist()


def check_decode_vs_kat(mod):
    gen = torch.Generator().manual_seed(7)
    block_size, num_blocks = 4, 8
    qs, tables, lens, pools_k, pools_v, expected = [], [], [], [], [], []
    for q, k, v, exp in kat_rows():
        table = _table((k.shape[0] + block_size - 1) // block_size, num_blocks, gen)
        kc, vc = build_pool(k, v, table, block_size, num_blocks)
        out = mod.decode_single(q, kc, vc, table, k.shape[0], block_size)
        np.testing.assert_allclose(out[0].numpy(), exp, rtol=1e-4, atol=1e-5)
        # The tensorized path gathers block 0 for padded positions and
        # multiplies them by zero probability (reference :230-253), so its
        # pools hold finite filler instead of NaN.
        kc, vc = build_pool(k, v, table, block_size, num_blocks, fill=1e3)
        qs.append(q)
        tables.append(table)
        lens.append(k.shape[0])
        pools_k.append(kc)
        pools_v.append(vc)
        expected.append(exp)
    # The same rows as one ragged batch over one shared pool.
    offsets, shared_k, shared_v, shifted = 0, [], [], []
    for table, kc, vc in zip(tables, pools_k, pools_v):
        shared_k.append(kc)
        shared_v.append(vc)
        shifted.append([b + offsets for b in table])
        offsets += num_blocks
    width = max(len(t) for t in shifted)
    bt = torch.tensor([t + [-1] * (width - len(t)) for t in shifted])
    out = mod.decode_batch_parallel(torch.stack([q for q in qs]), torch.cat(shared_k),
                                    torch.cat(shared_v), bt, torch.tensor(lens), block_size)
    np.testing.assert_allclose(out[:, 0].numpy(), np.stack(expected), rtol=1e-4, atol=1e-5)


def check_prefill_vs_kat(mod):
    """A one-token chunk whose context is the row's visible keys is that row."""
    gen = torch.Generator().manual_seed(11)
    block_size, num_blocks = 4, 8
    for q, k, v, exp in kat_rows()[::3]:
        n = k.shape[0]
        table = _table((n + block_size - 1) // block_size, num_blocks, gen)
        kc, vc = build_pool(k, v, table, block_size, num_blocks)
        for fn, tile in ((mod.prefill_chunk_tiled, 3), (mod.prefill_chunk_dense, 1)):
            out = fn(q[None], kc, vc, table, n - 1, n, block_size, tile)
            np.testing.assert_allclose(out[0, 0].numpy(), exp, rtol=1e-4, atol=1e-5)


def random_paged(seq_lens, hq, hkv, d, block_size, dtype=torch.float32, seed=0,
                 spare_blocks=3, fill=float("nan")):
    """Random q and filler-padded pools with shuffled, -1-padded block tables."""
    gen = torch.Generator().manual_seed(seed)
    need = [(s + block_size - 1) // block_size for s in seq_lens]
    num_blocks = sum(need) + spare_blocks
    perm = torch.randperm(num_blocks, generator=gen).tolist()
    k_cache = torch.full((num_blocks, block_size, hkv, d), fill, dtype=dtype)
    v_cache = torch.full_like(k_cache, fill)
    tables, cursor = [], 0
    for s, n in zip(seq_lens, need):
        table = perm[cursor:cursor + n]
        cursor += n
        tables.append(table)
        k = torch.randn(s, hkv, d, generator=gen).to(dtype)
        v = torch.randn(s, hkv, d, generator=gen).to(dtype)
        pos = torch.arange(s)
        blocks = torch.tensor(table, dtype=torch.long)[pos // block_size]
        k_cache[blocks, pos % block_size] = k
        v_cache[blocks, pos % block_size] = v
    width = max(need)
    bt = torch.tensor([t + [-1] * (width - len(t)) for t in tables], dtype=torch.long)
    q = torch.randn(len(seq_lens), hq, d, generator=gen).to(dtype)
    return q, k_cache, v_cache, bt, torch.tensor(seq_lens, dtype=torch.long), tables


def check_decode_vs_textbook(mod):
    for hq, hkv, lens, d, bs in (
        (14, 2, [17, 64, 130, 255], 64, 16),   # FP32 decode workload, GQA 7:1
        (4, 4, [3, 9], 8, 4),                  # MHA
        (4, 1, [5, 1], 8, 2),                  # MQA, one-token context
        (6, 2, [33], 16, 8),
    ):
        q, kc, vc, bt, sl, tables = random_paged(lens, hq, hkv, d, bs, seed=hq * 100 + d,
                                                 fill=1e3)
        want = textbook.paged_decode(q.numpy(), kc.numpy(), vc.numpy(), tables, lens)
        got = mod.decode_batch_parallel(q, kc, vc, bt, sl, bs)
        np.testing.assert_allclose(got.numpy(), want, rtol=1e-5, atol=1e-5)
        for b in range(len(lens)):
            single = mod.decode_single(q[b], kc, vc, tables[b], lens[b], bs)
            np.testing.assert_allclose(single.numpy(), want[b], rtol=1e-5, atol=1e-5)


def check_prefill_vs_textbook(mod):
    # The reference test grid (tests/kernels/test_paged_attention.py:249-351),
    # plus a multi-block GQA 7:1 case.
    cases = []
    for hq, hkv in ((2, 2), (4, 2), (4, 1)):
        for prefix in (0, 5):
            for tile in (1, 4, 16):
                cases.append((hq, hkv, prefix, 4, 8, 3, tile))
    cases.append((14, 2, 37, 21, 64, 16, 16))
    for hq, hkv, prefix, chunk, d, bs, tile in cases:
        gen = torch.Generator().manual_seed(prefix * 31 + tile + hq)
        context = prefix + chunk
        n_blocks = (context + bs - 1) // bs
        table = torch.randperm(n_blocks + 2, generator=gen)[:n_blocks].tolist()
        k = torch.randn(context, hkv, d, generator=gen)
        v = torch.randn(context, hkv, d, generator=gen)
        q = torch.randn(chunk, hq, d, generator=gen)
        kc, vc = build_pool(k, v, table, bs, n_blocks + 2)
        want = textbook.paged_prefill(q.numpy(), kc.numpy(), vc.numpy(), table, prefix)
        for fn in (mod.prefill_chunk_tiled, mod.prefill_chunk_dense):
            got = fn(q, kc, vc, table, prefix, context, bs, tile)
            np.testing.assert_allclose(got.numpy(), want, rtol=1e-5, atol=1e-5)
        # BF16 inputs: within the reference test's BF16 tolerance of the
        # textbook answer on the same (rounded) values.
        qb, kcb, vcb = q.bfloat16(), kc.bfloat16(), vc.bfloat16()
        want_b = textbook.paged_prefill(qb.float().numpy(), kcb.float().numpy(),
                                        vcb.float().numpy(), table, prefix)
        got_b = mod.prefill_chunk_tiled(qb, kcb, vcb, table, prefix, context, bs, tile)
        np.testing.assert_allclose(got_b.float().numpy(), want_b, rtol=1e-2, atol=2e-2)


ALL_CHECKS = (check_decode_vs_kat, check_prefill_vs_kat, check_decode_vs_textbook,
              check_prefill_vs_textbook)


# ---------------------------------------------------------------------------
# Qwen2 attention callers (oracle/qwen2_attention.py) against float64 math
# written out by hand: y = W h + b; RoPE as the rotation of each pair
# (x_i, x_{i+D/2}) by angle position * theta^(-2i/D); textbook attention;
# out = W_o . attention.
# ---------------------------------------------------------------------------
QWEN2_CFG = (4, 2, 8, 10000.0)  # Hq, Hkv, D, rope theta


def qwen2_weights(seed=0, dtype=torch.float64):
    hq, hkv, d, _ = QWEN2_CFG
    hidden = hq * d
    gen = torch.Generator().manual_seed(seed)
    rnd = lambda *s: (torch.randn(*s, generator=gen) * 0.3).to(dtype)
    return {"q_w": rnd(hq * d, hidden), "q_b": rnd(hq * d), "k_w": rnd(hkv * d, hidden),
            "k_b": rnd(hkv * d), "v_w": rnd(hkv * d, hidden), "v_b": rnd(hkv * d),
            "o_w": rnd(hidden, hidden)}


def _np_rope(x, pos, theta):
    """x [heads, D] at integer position pos, pair rotation."""
    d = x.shape[-1]
    half = d // 2
    out = np.empty_like(x)
    for i in range(half):
        ang = pos * theta ** (-2.0 * i / d)
        c, s = np.cos(ang), np.sin(ang)
        out[:, i] = x[:, i] * c - x[:, i + half] * s
        out[:, i + half] = x[:, i + half] * c + x[:, i] * s
    return out


def _np_qkv(h, w, pos):
    hq, hkv, d, theta = QWEN2_CFG
    wn = {k: v.numpy() for k, v in w.items()}
    q = (wn["q_w"] @ h + wn["q_b"]).reshape(hq, d)
    k = (wn["k_w"] @ h + wn["k_b"]).reshape(hkv, d)
    v = (wn["v_w"] @ h + wn["v_b"]).reshape(hkv, d)
    return _np_rope(q, pos, theta), _np_rope(k, pos, theta), v


def _np_attend(q, keys, values, nvis):
    """q [Hq, D] over the first nvis keys [N, Hkv, D] -> [Hq*D]."""
    hq, hkv, d, _ = QWEN2_CFG
    group = hq // hkv
    rows = []
    for h in range(hq):
        rows.append(textbook.attend(q[h][None], keys[:nvis, h // group], values[:nvis, h // group],
                                    np.ones((1, nvis), bool))[0])
    return np.concatenate(rows)


def check_qwen2_callers_vs_textbook(mod):
    # Tolerance 1e-6: the reference builds the RoPE cos/sin tables in FP32
    # (model/qwen2.py:160-170) even for FP64 activations, the textbook here
    # in FP64.
    hq, hkv, d, theta = QWEN2_CFG
    from oracle.paged_kv_cache import OracleKVCache
    w = qwen2_weights()
    wo = w["o_w"].numpy()
    gen = torch.Generator().manual_seed(7)
    bs, nblocks = 4, 24
    perm = torch.randperm(nblocks, generator=gen).tolist()
    # Logical K/V history of three sequences (positions before their new token).
    lens = [5, 11, 2]
    tables = [perm[0:2], perm[2:5], perm[5:6]]
    hist_k = [torch.randn(n, hkv, d, generator=gen, dtype=torch.float64) for n in lens]
    hist_v = [torch.randn(n, hkv, d, generator=gen, dtype=torch.float64) for n in lens]

    def fresh_cache():
        cache = OracleKVCache(1, nblocks, bs, hkv, d, dtype=torch.float64)
        cache.k_cache.fill_(1e3)
        cache.v_cache.fill_(1e3)
        for s, n in enumerate(lens):
            for p in range(n):
                cache.k_cache[0, tables[s][p // bs], p % bs] = hist_k[s][p]
                cache.v_cache[0, tables[s][p // bs], p % bs] = hist_v[s][p]
        return cache

    # Batched decode: the new token sits at position len (context len + 1).
    hidden = torch.randn(3, 1, hq * d, generator=gen, dtype=torch.float64)
    ctx = torch.tensor([n + 1 for n in lens])
    pos = (ctx - 1).unsqueeze(1)
    width = max(len(t) for t in tables)
    bt = torch.tensor([t + [-1] * (width - len(t)) for t in tables])
    slots = torch.tensor([tables[s][n // bs] * bs + n % bs for s, n in enumerate(lens)])
    cache = fresh_cache()
    got = mod.decode_batch(hidden, pos, cache, 0, slots, bt, ctx, w, QWEN2_CFG)
    for s, n in enumerate(lens):
        q, k, v = _np_qkv(hidden[s, 0].numpy(), w, n)
        keys = np.concatenate([hist_k[s].numpy(), k[None]])
        vals = np.concatenate([hist_v[s].numpy(), v[None]])
        want = wo @ _np_attend(q, keys, vals, n + 1)
        np.testing.assert_allclose(got[s, 0].numpy(), want, rtol=1e-6, atol=1e-6)
        single_cache = fresh_cache()
        one = mod.decode_single(hidden[s:s + 1], pos[s:s + 1], single_cache, 0, slots[s:s + 1],
                                tables[s], n + 1, w, QWEN2_CFG)
        np.testing.assert_allclose(one[0, 0].numpy(), want, rtol=1e-6, atol=1e-6)

    # Chunk prefill of sequence 1: three new tokens after its 11-token prefix.
    prefix, chunk = lens[1], 3
    table = perm[2:6]  # room for 14 positions
    hidden = torch.randn(1, chunk, hq * d, generator=gen, dtype=torch.float64)
    positions = torch.arange(prefix, prefix + chunk).unsqueeze(0)
    cslots = torch.tensor([table[p // bs] * bs + p % bs for p in range(prefix, prefix + chunk)])
    cache = fresh_cache()
    got = mod.prefill_chunk(hidden, positions, cache, 0, cslots, table, prefix, prefix + chunk,
                            2, w, QWEN2_CFG)
    new = [_np_qkv(hidden[0, i].numpy(), w, prefix + i) for i in range(chunk)]
    keys = np.concatenate([hist_k[1].numpy(), np.stack([n[1] for n in new])])
    vals = np.concatenate([hist_v[1].numpy(), np.stack([n[2] for n in new])])
    for i in range(chunk):
        want = wo @ _np_attend(new[i][0], keys, vals, prefix + i + 1)
        np.testing.assert_allclose(got[0, i].numpy(), want, rtol=1e-6, atol=1e-6)

    # Whole-prompt prefill: five tokens at positions 0..4, causal.
    hidden = torch.randn(1, 5, hq * d, generator=gen, dtype=torch.float64)
    positions = torch.arange(5).unsqueeze(0)
    pslots = torch.tensor([perm[10] * bs + p if p < bs else perm[11] * bs + p - bs
                           for p in range(5)])
    cache = fresh_cache()
    got = mod.prefill_whole(hidden, positions, cache, 0, pslots, w, QWEN2_CFG)
    new = [_np_qkv(hidden[0, i].numpy(), w, i) for i in range(5)]
    keys = np.stack([n[1] for n in new])
    vals = np.stack([n[2] for n in new])
    for i in range(5):
        want = wo @ _np_attend(new[i][0], keys, vals, i + 1)
        np.testing.assert_allclose(got[0, i].numpy(), want, rtol=1e-6, atol=1e-6)
    # The prompt's rows landed in their slots.
    for p in range(5):
        slot = int(pslots[p])
        np.testing.assert_allclose(cache.k_cache[0, slot // bs, slot % bs].numpy(), new[p][1],
                                   rtol=1e-6, atol=1e-6)


QWEN2_CHECKS = (check_qwen2_callers_vs_textbook,)


# ---------------------------------------------------------------------------
# Whole model (oracle/qwen2_model.py) against a float64 textbook: RMSNorm as
# x / sqrt(mean(x^2) + eps) * w (eps large enough to matter), SwiGLU with
# silu(x) = x / (1 + e^-x), pre-norm residual layers, the attention of the
# callers' textbook above, final norm and lm_head.
# ---------------------------------------------------------------------------
MODEL_CFG = types.SimpleNamespace(
    vocab_size=23, hidden_size=32, intermediate_size=40, num_hidden_layers=2,
    num_attention_heads=4, num_key_value_heads=2, head_dim=8, rope_theta=10000.0,
    rms_norm_eps=0.25)


def model_state(seed=0):
    cfg = MODEL_CFG
    gen = torch.Generator().manual_seed(seed)
    rnd = lambda *s: torch.randn(*s, generator=gen, dtype=torch.float64) * 0.4  # noqa: E731
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    hid, inter = cfg.hidden_size, cfg.intermediate_size
    sd = {"model.embed_tokens.weight": rnd(cfg.vocab_size, hid),
          "model.norm.weight": 1 + rnd(hid), "lm_head.weight": rnd(cfg.vocab_size, hid)}
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        a = p + "self_attn."
        sd.update({p + "input_layernorm.weight": 1 + rnd(hid),
                   p + "post_attention_layernorm.weight": 1 + rnd(hid),
                   a + "qkv_proj.q_proj.weight": rnd(hq * d, hid), a + "qkv_proj.q_proj.bias": rnd(hq * d),
                   a + "qkv_proj.k_proj.weight": rnd(hkv * d, hid), a + "qkv_proj.k_proj.bias": rnd(hkv * d),
                   a + "qkv_proj.v_proj.weight": rnd(hkv * d, hid), a + "qkv_proj.v_proj.bias": rnd(hkv * d),
                   a + "o_proj.weight": rnd(hid, hid),
                   p + "mlp.gate_proj.weight": rnd(inter, hid),
                   p + "mlp.up_proj.weight": rnd(inter, hid),
                   p + "mlp.down_proj.weight": rnd(hid, inter)})
    return sd


def _np_rms(x, w, eps):
    return x / np.sqrt(np.mean(x * x) + eps) * w


def np_model_logits(sd, tokens):
    """Logits [S, vocab] of the sequence, position by position."""
    cfg = MODEL_CFG
    n = {k: v.numpy() for k, v in sd.items()}
    hs = [n["model.embed_tokens.weight"][t].copy() for t in tokens]
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        a = p + "self_attn.qkv_proj."
        w = {"q_w": sd[a + "q_proj.weight"], "q_b": sd[a + "q_proj.bias"],
             "k_w": sd[a + "k_proj.weight"], "k_b": sd[a + "k_proj.bias"],
             "v_w": sd[a + "v_proj.weight"], "v_b": sd[a + "v_proj.bias"]}
        qkv = [_np_qkv(_np_rms(h, n[p + "input_layernorm.weight"], cfg.rms_norm_eps), w, t)
               for t, h in enumerate(hs)]
        keys = np.stack([x[1] for x in qkv])
        vals = np.stack([x[2] for x in qkv])
        wo = n[p + "self_attn.o_proj.weight"]
        hs = [h + wo @ _np_attend(qkv[t][0], keys, vals, t + 1) for t, h in enumerate(hs)]
        out = []
        for h in hs:
            x = _np_rms(h, n[p + "post_attention_layernorm.weight"], cfg.rms_norm_eps)
            g = n[p + "mlp.gate_proj.weight"] @ x
            u = n[p + "mlp.up_proj.weight"] @ x
            out.append(h + n[p + "mlp.down_proj.weight"] @ (g / (1 + np.exp(-g)) * u))
        hs = out
    return np.stack([n["lm_head.weight"] @ _np_rms(h, n["model.norm.weight"], cfg.rms_norm_eps)
                     for h in hs])


def check_model_vs_textbook(mod):
    # Tolerance 1e-6: FP32 RoPE tables, as in the callers' check above.
    sd = model_state()
    oracle = mod.OracleQwen2(sd, MODEL_CFG)
    gen = torch.Generator().manual_seed(3)
    prompt = torch.randint(0, MODEL_CFG.vocab_size, (9,), generator=gen).tolist()
    np.testing.assert_allclose(oracle.forward(prompt).numpy(), np_model_logits(sd, prompt),
                               rtol=1e-6, atol=1e-6)
    # Greedy decoding, both ways, against the textbook's argmax and margins.
    margins: list = []
    cached = oracle.cached_greedy(prompt, 6, margins)
    assert oracle.dense_greedy(prompt, 6) == cached
    seq = list(prompt)
    for step in range(6):
        row = np_model_logits(sd, seq)[-1]
        order = np.argsort(row)[::-1]
        assert cached[step] == int(order[0])
        assert abs(margins[step][0] - (row[order[0]] - row[order[1]])) < 1e-6
        seq.append(cached[step])
    # Teacher forcing: tokens the model would not pick, fed one per step.
    forced = torch.randint(0, MODEL_CFG.vocab_size, (5,), generator=gen).tolist()
    rows = oracle.teacher_forced_logits(prompt, forced).numpy()
    np.testing.assert_allclose(rows, np_model_logits(sd, prompt + forced)[len(prompt) - 1:],
                               rtol=1e-6, atol=1e-6)


MODEL_CHECKS = (check_model_vs_textbook,)
