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


# ---------------------------------------------------------------------------
# End-to-end continuous batching at Qwen2.5-0.5B shape
# ---------------------------------------------------------------------------
QWEN05B_CONFIG = dict(vocab_size=151936, hidden_size=896, intermediate_size=4864,
                      num_hidden_layers=24, num_attention_heads=14, num_key_value_heads=2,
                      max_position_embeddings=32768, rope_theta=1_000_000.0,
                      rms_norm_eps=1e-6, tie_word_embeddings=False)


@dataclass
class ServingWorkload:
    """A random-init model, the requests of a serving run and its scheduler
    limits. ``initial`` requests (prompt, max_new_tokens) arrive first,
    ``arrivals`` queue behind them; once every initial prompt is admitted
    (the warm-up), ``steps`` scheduler steps are the measured run."""

    name: str
    config: dict
    model_seed: int
    block_size: int
    num_blocks: int
    max_num_batched_tokens: int
    max_num_seqs: int
    initial: list = field(default_factory=list)
    arrivals: list = field(default_factory=list)
    steps: int = 128


def qwen05b_serving(num_initial: int = 48, prefills_per_step: int = 2,
                    prefill_len: int = 1024, num_arrivals: int = 320,
                    steps: int = 128) -> ServingWorkload:
    """Mixed serving steps at Qwen2.5-0.5B shape (24 layers, hidden 896,
    intermediate 4864, 14 / 2 heads, head_dim 64, vocab 151936, RoPE theta 1e6;
    the lm_head is its own matrix so that a random model's tokens depend on
    the context). 48 requests with prompts U[64, 2048] decode while prompts of
    1024 random token ids arrive; the scheduler's budget (48 decode tokens +
    2 x 1024) and 50 seats give about 48 decodes and 2 prefills per step.
    Lifetimes of U[1, 49] and U[10, 40] new tokens (25 on average) retire
    about two requests per step, so admission, exit and block reuse go on for
    the whole run."""
    gen = torch.Generator().manual_seed(0)
    vocab = QWEN05B_CONFIG["vocab_size"]

    def prompt(n):
        return torch.randint(0, vocab, (n,), generator=gen).tolist()

    initial = [(prompt(int(n)), int(m)) for n, m in zip(
        torch.randint(64, 2049, (num_initial,), generator=gen),
        torch.randint(1, 50, (num_initial,), generator=gen))]
    arrivals = [(prompt(prefill_len), int(m))
                for m in torch.randint(10, 41, (num_arrivals,), generator=gen)]
    budget = num_initial + prefills_per_step * prefill_len
    # Pool: every seat at its longest context (2048 + 49 tokens), plus slack.
    block_size = 16
    num_blocks = (num_initial + prefills_per_step) * math.ceil((2048 + 64) / block_size) + 256
    return ServingWorkload(name="qwen05b_serving_48dec_2x1024pre", config=dict(QWEN05B_CONFIG),
                           model_seed=0, block_size=block_size, num_blocks=num_blocks,
                           max_num_batched_tokens=budget,
                           max_num_seqs=num_initial + prefills_per_step,
                           initial=initial, arrivals=arrivals, steps=steps)


def build_serving(w: ServingWorkload, device, dtype):
    """The model (seeded init on the CPU, then moved), its KV pool and a
    scheduler holding every request of ``w`` (initial ones first)."""
    from .model.qwen2 import TinyQwen2Config, TinyQwen2ForCausalLM
    from .runtime.paged_kv_cache import PagedKVCache
    from .runtime.request import Request
    from .runtime.scheduler import Scheduler

    cfg = TinyQwen2Config(**w.config)
    torch.manual_seed(w.model_seed)
    model = TinyQwen2ForCausalLM(cfg).to(device=device, dtype=dtype).eval()
    cache = PagedKVCache(cfg.num_hidden_layers, w.num_blocks, w.block_size,
                         cfg.num_key_value_heads, cfg.head_dim, dtype=dtype, device=device)
    scheduler = Scheduler(w.max_num_batched_tokens, w.max_num_seqs, kv_cache=cache)
    requests = [Request(f"init{i}", p, m, 0.0) for i, (p, m) in enumerate(w.initial)]
    requests += [Request(f"arr{i}", p, m, 1.0 + i) for i, (p, m) in enumerate(w.arrivals)]
    for request in requests:
        scheduler.add_request(request)
    return cfg, model, cache, scheduler, requests


def serving_warm_up(model, scheduler, num_initial: int, max_steps: int = 1000,
                    decode_graphs=None, prefill_graphs=None) -> int:
    """Run steps until every initial request has been admitted; returns the
    number of steps run."""
    from .runtime.model_runner import run_generation_step

    steps = 0
    while any(r.request_id.startswith("init") for r in scheduler.waiting):
        run_generation_step(model, scheduler, decode_graphs=decode_graphs,
                            prefill_graphs=prefill_graphs)
        steps += 1
        if steps > max_steps:
            raise RuntimeError("warm-up did not admit the initial requests")
    return steps
