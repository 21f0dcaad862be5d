"""CPU restatement of the reference's paged attention math (oracle; tests only).

Every function here repeats the reference's tensor operations in the same
order (same dtypes, same rounding points) so that, on the same torch build,
it reproduces the reference's results; the validation messages are the
reference's too. The restated code is this project's own; where the steps
must match the reference, they do, and the citation says which lines.

Reference file: src/mini_llm_runtime/kernels/reference/paged_attention.py
"""

from __future__ import annotations

import math

import torch


def _check_layout(k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    if k_cache.ndim != 4 or v_cache.ndim != 4:
        raise ValueError(
            "k_cache and v_cache must have shape [num_blocks, block_size, Hkv, D]")
    if k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must have the same shape")


def _check_heads(num_q_heads: int, head_dim: int, k_cache: torch.Tensor) -> int:
    if head_dim != k_cache.shape[-1]:
        raise ValueError("q and KV cache must have the same head_dim")
    if num_q_heads % k_cache.shape[2] != 0:
        raise ValueError("num_query_heads must be divisible by num_kv_heads")
    return num_q_heads // k_cache.shape[2]


def decode_single(q, k_cache, v_cache, block_table, seq_len, block_size):
    """One request's paged decode, q [Hq, D] -> [Hq, D].

    Follows paged_attention.py:6-105: a Python loop gathers each position's
    K/V row from (block_table[pos // bs], pos % bs) (:70-80), rows are stacked
    and moved to [Hkv, S, D] (:82-86), repeated per GQA group (:89-91), then
    scores = q @ k^T * (1/sqrt(D)) in the input dtype (:95), FP32 softmax cast
    back to the value dtype (:97-101) and probs @ v (:103).
    """
    if q.ndim != 2:
        raise ValueError("q must have shape [Hq, D]")
    _check_layout(k_cache, v_cache)
    group = _check_heads(q.shape[0], q.shape[-1], k_cache)
    if seq_len <= 0:
        raise ValueError("seq_len must be greater than 0")
    if len(block_table) < (seq_len + block_size - 1) // block_size:
        raise ValueError("block_table does not contain enough blocks for seq_len")
    if block_size != k_cache.shape[1]:
        raise ValueError("block_size does not match KV cache layout")
    scale = 1.0 / math.sqrt(q.shape[-1])
    keys, values = [], []
    for pos in range(seq_len):
        block = block_table[pos // block_size]
        keys.append(k_cache[block][pos % block_size])
        values.append(v_cache[block][pos % block_size])
    k = torch.stack(keys, dim=0).permute(1, 0, 2)    # [Hkv, S, D]
    v = torch.stack(values, dim=0).permute(1, 0, 2)
    if group > 1:
        k = k.repeat_interleave(group, dim=0)
        v = v.repeat_interleave(group, dim=0)
    scores = q.unsqueeze(1) @ k.transpose(-2, -1) * scale          # [Hq, 1, S]
    probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(v.dtype)
    return (probs @ v).squeeze(1)


def decode_batch_loop(q, k_cache, v_cache, block_tables, seq_lens, block_size):
    """Per-request loop over decode_single (paged_attention.py:109-176)."""
    if q.ndim != 3:
        raise ValueError("q must have shape [B, Hq, D]")
    _check_layout(k_cache, v_cache)
    _check_heads(q.shape[1], q.shape[-1], k_cache)
    if len(block_tables) != q.shape[0]:
        raise ValueError("block_tables length must match batch size of q")
    if len(seq_lens) != q.shape[0]:
        raise ValueError("seq_lens length must match batch size of q")
    for i in range(q.shape[0]):
        if len(block_tables[i]) < (seq_lens[i] + block_size - 1) // block_size:
            raise ValueError(
                f"block_table for batch {i} does not contain enough blocks "
                f"for seq_len {seq_lens[i]}")
    return torch.stack([
        decode_single(q[i], k_cache, v_cache, block_tables[i], seq_lens[i], block_size)
        for i in range(q.shape[0])
    ], dim=0)


def decode_batch_parallel(q, k_cache, v_cache, block_tables, seq_lens, block_size):
    """Tensorized batched paged decode, q [B, Hq, D] -> [B, Hq, D].

    Follows paged_attention.py:178-254, the reference's tensorized PyTorch
    paged path: physical ids block_tables[b, pos // bs] for every position up
    to max(seq_lens) (:222-229), invalid positions pointed at block 0 (:230-232),
    a [B, maxS, Hkv, D] gather (:234-235), [B, Hq, maxS, D] after transpose and
    repeat_interleave (:238-240), scores = q @ k^T * scale in the input dtype
    (:245-247), -inf past each seq_len (:249), FP32 softmax cast to the value
    dtype (:251) and probs @ v (:253).
    """
    if q.ndim != 3:
        raise ValueError("q must have shape [B, Hq, D]")
    _check_layout(k_cache, v_cache)
    group = _check_heads(q.shape[1], q.shape[-1], k_cache)
    if len(block_tables) != q.shape[0]:
        raise ValueError("block_tables length must match batch size of q")
    if len(seq_lens) != q.shape[0]:
        raise ValueError("seq_lens length must match batch size of q")
    max_len = int(seq_lens.max().item())
    pos = torch.arange(max_len, device=block_tables.device)
    rows = torch.arange(q.shape[0], device=q.device).unsqueeze(1)
    physical = block_tables[rows, pos // block_size]                  # [B, maxS]
    live = pos.unsqueeze(0) < seq_lens.unsqueeze(1)
    physical = physical.masked_fill(~live, 0)
    offsets = (pos % block_size).unsqueeze(0)
    k = k_cache[physical, offsets].transpose(1, 2).repeat_interleave(group, dim=1)
    v = v_cache[physical, offsets].transpose(1, 2).repeat_interleave(group, dim=1)
    scale = 1.0 / math.sqrt(q.shape[-1])
    scores = torch.matmul(q.unsqueeze(2), k.transpose(-2, -1)) * scale
    scores = scores.masked_fill(~live[:, None, None, :], float("-inf"))
    probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(v.dtype)
    return torch.matmul(probs, v).squeeze(2)


def _slots(block_table, positions, block_size, device):
    table = torch.as_tensor(block_table, dtype=torch.long, device=device)
    return table[positions // block_size] * block_size + positions % block_size


def prefill_chunk_dense(q, k_cache, v_cache, block_table, prefix_len, context_len,
                        block_size, tile_size=None):
    """Dense chunk-prefill reference, q [C, Hq, D] -> [C, Hq, D].

    Follows paged_attention.py:282-343: every context key gathered by flat
    slot (:307-321), GQA repeat (:322-323), scores = (q @ k^T) / sqrt(D) in the
    input dtype (:325-328), causal mask key_pos <= prefix_len + i (:329-337),
    FP32 softmax cast to the value dtype (:338-342), then probs @ v.
    """
    del tile_size
    if context_len != prefix_len + q.shape[0]:
        raise ValueError("context_len must equal prefix_len + q.shape[0]")
    if q.shape[1] % k_cache.shape[2] != 0:
        raise ValueError("q_num_heads must be divisible by kv_num_heads")
    group = q.shape[1] // k_cache.shape[2]
    positions = torch.arange(context_len, device=q.device)
    slots = _slots(block_table, positions, block_size, q.device)
    keys = k_cache.flatten(0, 1)[slots].permute(1, 0, 2).repeat_interleave(group, dim=0)
    values = v_cache.flatten(0, 1)[slots].permute(1, 0, 2).repeat_interleave(group, dim=0)
    scores = (q.permute(1, 0, 2) @ keys.transpose(-2, -1)) / math.sqrt(q.shape[-1])
    query_pos = prefix_len + torch.arange(q.shape[0], device=q.device)
    visible = positions.unsqueeze(0) <= query_pos.unsqueeze(1)
    scores = scores.masked_fill(~visible.unsqueeze(0), float("-inf"))
    probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(values.dtype)
    return (probs @ values).permute(1, 0, 2)


def prefill_chunk_tiled(q, k_cache, v_cache, block_table, prefix_len, context_len,
                        block_size, tile_size):
    """Tiled online-softmax chunk prefill, q [C, Hq, D] -> [C, Hq, D].

    Follows paged_attention.py:346-434: FP32 running max/sum/acc per
    (head, query) (:372-384); for each key tile of tile_size positions
    (:398-409): scores = (q @ k^T) / sqrt(D) in the input dtype (:411-413),
    cast to FP32 and causally masked (:414-418), then the online update with
    FP32 values (:419-431); output acc / sum cast to the query dtype (:433-434).
    """
    if tile_size <= 0:
        raise ValueError("tile_size must be greater than 0")
    if context_len != prefix_len + q.shape[0]:
        raise ValueError("context_len must equal prefix_len + q.shape[0]")
    if q.shape[1] % k_cache.shape[2] != 0:
        raise ValueError("q_num_heads must be divisible by kv_num_heads")
    group = q.shape[1] // k_cache.shape[2]
    heads, chunk, head_dim = q.shape[1], q.shape[0], q.shape[-1]
    acc = torch.zeros((heads, chunk, head_dim), dtype=torch.float32, device=q.device)
    run_max = torch.full((heads, chunk, 1), float("-inf"), dtype=torch.float32,
                         device=q.device)
    run_sum = torch.zeros_like(run_max)
    query = q.permute(1, 0, 2)
    flat_k, flat_v = k_cache.flatten(0, 1), v_cache.flatten(0, 1)
    query_pos = prefix_len + torch.arange(chunk, device=q.device)
    for start in range(0, context_len, tile_size):
        positions = torch.arange(start, min(start + tile_size, context_len),
                                 device=q.device)
        slots = _slots(block_table, positions, block_size, q.device)
        keys = flat_k[slots].permute(1, 0, 2).repeat_interleave(group, dim=0)
        values = flat_v[slots].permute(1, 0, 2).repeat_interleave(group, dim=0)
        scores = (query @ keys.transpose(-2, -1)) / math.sqrt(head_dim)
        visible = positions.unsqueeze(0) <= query_pos.unsqueeze(1)
        scores = scores.to(torch.float32).masked_fill(~visible.unsqueeze(0),
                                                      float("-inf"))
        new_max = torch.maximum(run_max, scores.max(dim=-1, keepdim=True).values)
        rescale = torch.exp(run_max - new_max)
        weights = torch.exp(scores - new_max)
        run_sum = run_sum * rescale + weights.sum(dim=-1, keepdim=True)
        acc = acc * rescale + weights @ values.to(torch.float32)
        run_max = new_max
    return (acc / run_sum).to(q.dtype).permute(1, 0, 2)
