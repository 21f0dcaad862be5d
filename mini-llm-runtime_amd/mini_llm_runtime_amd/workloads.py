"""Seeded synthetic workloads of the paged attention path.

Each builder draws everything from one ``torch.Generator('cpu')`` seeded with
0, creates tensors on the CPU and returns them there; callers move what they
need to the GPU. The shapes are the named benchmark workloads:

- fp32_decode_b4:  FP32 single-token decode, batch 4, 14 q / 2 KV heads,
  head_dim 64, block 16, contexts {17, 64, 130, 255}, 64-block pool.
- bf16_decode_qwen05b_b64: BF16 batched decode at Qwen2.5-0.5B attention
  shape, batch 64, contexts U[128, 4096], 24576-block pool, plus the batched
  write of the 64 new tokens.
- bf16_prefill_chunk512_x8: BF16 chunk prefill, 8 sequences x 512-token chunk
  on prefixes U[0, 3584].
- bf16_decode_qwen7b_32k: BF16 decode at Qwen2.5-7B attention shape, batch 8,
  28 q / 4 KV heads, head_dim 128, context 32768.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch


@dataclass
class DecodeWorkload:
    name: str
    q: torch.Tensor               # [B, Hq, D]
    k_cache: torch.Tensor         # [NB, BS, Hkv, D] (one layer)
    v_cache: torch.Tensor
    block_tables: torch.Tensor    # [B, W] int64, -1 padded
    context_lens: torch.Tensor    # [B] int64, includes the new token
    slot_mapping: torch.Tensor    # [B] int64, slot of position ctx-1
    new_k: torch.Tensor           # [B, Hkv, D]
    new_v: torch.Tensor
    block_size: int
    tables: list = field(default_factory=list)

    @property
    def dtype(self):
        return self.q.dtype

    def algorithmic_bytes(self) -> int:
        """K+V rows read, q in, out, block ids and context lengths read."""
        esz = self.q.element_size()
        _, hq, d = self.q.shape
        hkv = self.k_cache.shape[2]
        ctx = self.context_lens
        blocks = (ctx + self.block_size - 1) // self.block_size
        return int(ctx.sum()) * hkv * d * 2 * esz + 2 * self.q.shape[0] * hq * d * esz \
            + int(blocks.sum()) * 8 + self.q.shape[0] * 8

    def write_bytes(self) -> int:
        """KV write: read new K/V, write K/V rows, read slots."""
        t, hkv, d = self.new_k.shape
        esz = self.new_k.element_size()
        return 2 * t * hkv * d * (esz + self.k_cache.element_size()) + t * 8


def _tables_from_perm(perm, need, width):
    tables, cursor = [], 0
    for n in need:
        tables.append(perm[cursor:cursor + n])
        cursor += n
    padded = [t + [-1] * (width - len(t)) for t in tables]
    return tables, torch.tensor(padded, dtype=torch.long)


def _slot_of_last(tables, ctx, block_size):
    return torch.tensor([tables[b][(c - 1) // block_size] * block_size + (c - 1) % block_size
                         for b, c in enumerate(ctx)], dtype=torch.long)


def fp32_decode_b4() -> DecodeWorkload:
    gen = torch.Generator().manual_seed(0)
    bs, nb, hkv, d = 16, 64, 2, 64
    q = torch.randn(4, 14, d, generator=gen)
    k = torch.randn(nb, bs, hkv, d, generator=gen)
    v = torch.randn(nb, bs, hkv, d, generator=gen)
    perm = torch.randperm(nb, generator=gen).tolist()
    ctx = [17, 64, 130, 255]
    need = [math.ceil(c / bs) for c in ctx]
    tables, bt = _tables_from_perm(perm, need, 16)
    new_k = torch.randn(4, hkv, d, generator=gen)
    new_v = torch.randn(4, hkv, d, generator=gen)
    return DecodeWorkload("fp32_decode_b4", q, k, v, bt, torch.tensor(ctx),
                          _slot_of_last(tables, ctx, bs), new_k, new_v, bs, tables)


def bf16_decode_qwen05b_b64(batch: int = 64, num_blocks: int = 24576,
                            max_ctx: int = 4096) -> DecodeWorkload:
    gen = torch.Generator().manual_seed(0)
    bs, hkv, d = 16, 2, 64
    ctx = torch.randint(128, max_ctx + 1, (batch,), generator=gen)
    k = (torch.randn(num_blocks, bs, hkv, d, generator=gen) * 0.5).bfloat16()
    v = (torch.randn(num_blocks, bs, hkv, d, generator=gen) * 0.5).bfloat16()
    perm = torch.randperm(num_blocks, generator=gen).tolist()
    need = [math.ceil(c / bs) for c in ctx.tolist()]
    tables, bt = _tables_from_perm(perm, need, math.ceil(max_ctx / bs))
    q = torch.randn(batch, 14, d, generator=gen).bfloat16()
    new_k = (torch.randn(batch, hkv, d, generator=gen) * 0.5).bfloat16()
    new_v = (torch.randn(batch, hkv, d, generator=gen) * 0.5).bfloat16()
    return DecodeWorkload("bf16_decode_qwen05b_b64", q, k, v, bt, ctx,
                          _slot_of_last(tables, ctx.tolist(), bs), new_k, new_v, bs, tables)


def bf16_decode_qwen7b_32k(batch: int = 8, context: int = 32768) -> DecodeWorkload:
    gen = torch.Generator().manual_seed(0)
    bs, hkv, d, hq = 16, 4, 128, 28
    need = math.ceil(context / bs)
    num_blocks = batch * need + 64
    k = torch.randn(num_blocks, bs, hkv, d, generator=gen).bfloat16()
    v = torch.randn(num_blocks, bs, hkv, d, generator=gen).bfloat16()
    perm = torch.randperm(num_blocks, generator=gen).tolist()
    tables, bt = _tables_from_perm(perm, [need] * batch, need)
    q = torch.randn(batch, hq, d, generator=gen).bfloat16()
    ctx = [context] * batch
    new_k = torch.randn(batch, hkv, d, generator=gen).bfloat16()
    new_v = torch.randn(batch, hkv, d, generator=gen).bfloat16()
    return DecodeWorkload("bf16_decode_qwen7b_32k", q, k, v, bt, torch.tensor(ctx),
                          _slot_of_last(tables, ctx, bs), new_k, new_v, bs, tables)


@dataclass
class PrefillWorkload:
    name: str
    q: torch.Tensor                # [total_q, Hq, D] packed
    chunk_k: torch.Tensor          # [total_q, Hkv, D] keys of the chunks
    chunk_v: torch.Tensor
    k_cache: torch.Tensor          # [NB, BS, Hkv, D], prefixes already written
    v_cache: torch.Tensor
    block_tables: torch.Tensor     # [S, W] int64, -1 padded
    query_start_loc: torch.Tensor  # [S + 1] int64
    context_lens: torch.Tensor     # [S] int64
    slot_mapping: torch.Tensor     # [total_q] int64, slots of the chunk tokens
    prefix_lens: list
    tables: list
    block_size: int

    def causal_flops(self) -> int:
        """4 * D * Hq * sum over sequences of (C * P + C (C + 1) / 2)."""
        _, hq, d = self.q.shape
        total = 0
        for s, p in enumerate(self.prefix_lens):
            c = int(self.query_start_loc[s + 1] - self.query_start_loc[s])
            total += c * p + c * (c + 1) // 2
        return 4 * d * hq * total


def bf16_prefill_chunk512_x8(num_seqs: int = 8, chunk: int = 512, max_prefix: int = 3584,
                             hq: int = 14, hkv: int = 2, d: int = 64,
                             dtype=torch.bfloat16) -> PrefillWorkload:
    gen = torch.Generator().manual_seed(0)
    bs = 16
    prefix = torch.randint(0, max_prefix + 1, (num_seqs,), generator=gen).tolist()
    need = [math.ceil((p + chunk) / bs) for p in prefix]
    num_blocks = sum(need) + 16
    perm = torch.randperm(num_blocks, generator=gen).tolist()
    width = max(need)
    tables, bt = _tables_from_perm(perm, need, width)
    k_cache = torch.zeros(num_blocks, bs, hkv, d, dtype=dtype)
    v_cache = torch.zeros_like(k_cache)
    qs, cks, cvs, slots = [], [], [], []
    for s, p in enumerate(prefix):
        k = torch.randn(p + chunk, hkv, d, generator=gen).to(dtype)
        v = torch.randn(p + chunk, hkv, d, generator=gen).to(dtype)
        table = torch.tensor(tables[s])
        pos = torch.arange(p + chunk)
        flat = table[pos // bs] * bs + pos % bs
        k_cache.view(-1, hkv, d)[flat[:p]] = k[:p]
        v_cache.view(-1, hkv, d)[flat[:p]] = v[:p]
        cks.append(k[p:])
        cvs.append(v[p:])
        slots.append(flat[p:])
        qs.append(torch.randn(chunk, hq, d, generator=gen).to(dtype))
    qsl = torch.tensor([0] + [chunk * (s + 1) for s in range(num_seqs)], dtype=torch.long)
    ctx = torch.tensor([p + chunk for p in prefix], dtype=torch.long)
    return PrefillWorkload("bf16_prefill_chunk512_x8", torch.cat(qs), torch.cat(cks),
                           torch.cat(cvs), k_cache, v_cache, bt, qsl, ctx, torch.cat(slots),
                           prefix, tables, bs)
