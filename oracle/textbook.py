"""Float64 textbook attention (oracle; tests only).

The definition of scaled dot-product attention, written with explicit loops
over (query, key) pairs and an explicit visibility predicate; it follows no
reference code. Used to pin the restatements in oracle.paged_attention:

    out[i] = sum_j softmax_j(scale * q_i . k_j | visible(i, j)) v_j

with the softmax taken over visible keys only.
"""

from __future__ import annotations

import math

import numpy as np


def attend(q, keys, values, visible, scale=None):
    """q [M, D], keys/values [N, D], visible [M, N] bool -> [M, D] float64."""
    q = np.asarray(q, dtype=np.float64)
    keys = np.asarray(keys, dtype=np.float64)
    values = np.asarray(values, dtype=np.float64)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    out = np.zeros((q.shape[0], values.shape[1]), dtype=np.float64)
    for i in range(q.shape[0]):
        cols = [j for j in range(keys.shape[0]) if visible[i][j]]
        if not cols:
            out[i] = np.nan
            continue
        logits = np.array([scale * float(np.dot(q[i], keys[j])) for j in cols])
        weights = np.exp(logits - logits.max())
        weights /= weights.sum()
        out[i] = sum(w * values[j] for w, j in zip(weights, cols))
    return out


def logical_kv(k_cache, v_cache, block_table, length, kv_head):
    """Rows [length, D] of one KV head, read position by position from a pool."""
    block_size = k_cache.shape[1]
    k = np.stack([np.asarray(k_cache[block_table[p // block_size], p % block_size, kv_head],
                             dtype=np.float64) for p in range(length)])
    v = np.stack([np.asarray(v_cache[block_table[p // block_size], p % block_size, kv_head],
                             dtype=np.float64) for p in range(length)])
    return k, v


def paged_decode(q, k_cache, v_cache, block_tables, seq_lens):
    """q [B, Hq, D] over pools [NB, BS, Hkv, D] (numpy) -> [B, Hq, D] float64."""
    batch, heads, _ = q.shape
    group = heads // k_cache.shape[2]
    out = np.zeros(q.shape, dtype=np.float64)
    for b in range(batch):
        for h in range(heads):
            k, v = logical_kv(k_cache, v_cache, block_tables[b], seq_lens[b], h // group)
            out[b, h] = attend(q[b, h][None, :], k, v, np.ones((1, seq_lens[b]), bool))[0]
    return out


def paged_prefill(q, k_cache, v_cache, block_table, prefix_len):
    """q [C, Hq, D], causal by absolute position prefix_len + i -> [C, Hq, D]."""
    chunk, heads, _ = q.shape
    group = heads // k_cache.shape[2]
    context = prefix_len + chunk
    visible = np.array([[j <= prefix_len + i for j in range(context)] for i in range(chunk)])
    out = np.zeros(q.shape, dtype=np.float64)
    for h in range(heads):
        k, v = logical_kv(k_cache, v_cache, block_table, context, h // group)
        out[:, h] = attend(q[:, h], k, v, visible)
    return out
