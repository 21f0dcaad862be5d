"""The batched decode step and repeated packed prefills replayed from HIP
graphs (runtime/step_graphs.py) against the same calls run eagerly.

An eager step given the block table padded to the runner's width launches the
same kernels with the same grids as the replay, so the two must agree bit for
bit: logits and every K/V row written. Between replays the program runs eager
work of its own and synchronises, and every replay is compared, so a recorded
node that only works on a graph's first replay (a memset, for instance) fails
here. The eager step itself is checked against the oracle elsewhere
(test_gpu_runtime.py, test_gpu_model_logits.py).
"""

from __future__ import annotations

import pytest
import torch

from mini_llm_runtime_amd.model.qwen2 import TinyQwen2Config, TinyQwen2ForCausalLM
from mini_llm_runtime_amd.runtime.step_graphs import DecodeGraphs, PrefillGraphs
from mini_llm_runtime_amd.runtime.model_runner import run_greedy_generation
from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache
from mini_llm_runtime_amd.runtime.request import Request
from mini_llm_runtime_amd.runtime.scheduler import Scheduler

pytestmark = pytest.mark.gpu

# Qwen2.5-0.5B attention and MLP shapes, two layers, a small vocabulary.
QWEN_2L = dict(vocab_size=1000, hidden_size=896, intermediate_size=4864, num_hidden_layers=2,
               num_attention_heads=14, num_key_value_heads=2, max_position_embeddings=32768,
               rope_theta=1_000_000.0, rms_norm_eps=1e-6, tie_word_embeddings=False)
BS = 16
NBLOCKS = 256
WIDTH = 48  # 768 tokens


def _model(device, dtype, seed=0):
    torch.manual_seed(seed)
    return TinyQwen2ForCausalLM(TinyQwen2Config(**QWEN_2L)).to(device=device, dtype=dtype).eval()


def _cache(device, dtype, seed=1):
    cache = PagedKVCache(2, NBLOCKS, BS, 2, 64, dtype=dtype, device=device)
    gen = torch.Generator().manual_seed(seed)
    cache.k_cache.copy_(torch.randn(cache.k_cache.shape, generator=gen).to(dtype))
    cache.v_cache.copy_(torch.randn(cache.v_cache.shape, generator=gen).to(dtype))
    return cache


def _step(device, lens, gen, width=None):
    """One decode step of len(lens) requests on distinct random blocks; the
    new token of request i sits at position lens[i] - 1."""
    perm = torch.randperm(NBLOCKS, generator=gen).tolist()
    tables, used = [], 0
    for n in lens:
        nb = -(-n // BS)
        tables.append(perm[used:used + nb])
        used += nb
    w = width or max(map(len, tables))
    step = dict(
        input_ids=torch.randint(0, QWEN_2L["vocab_size"], (len(lens), 1), generator=gen),
        position_ids=torch.tensor(lens)[:, None] - 1,
        slot_mapping=torch.tensor([t[(n - 1) // BS] * BS + (n - 1) % BS
                                   for t, n in zip(tables, lens)]),
        block_tables=torch.tensor([t + [-1] * (w - len(t)) for t in tables]),
        context_lens=torch.tensor(lens))
    return {k: v.to(device) for k, v in step.items()}


def _padded(step, width):
    bt = step["block_tables"]
    pad = torch.full((bt.shape[0], width - bt.shape[1]), -1, dtype=bt.dtype, device=bt.device)
    return dict(step, block_tables=torch.cat([bt, pad], dim=1))


STEPS = [[5, 300, 17, 640, 33], [1, 64, 2], [6, 301, 18, 641, 34], [600, 2, 3], [7, 302, 19, 700, 35]]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_replays_equal_the_eager_step(device, dtype):
    """Five steps over two batch sizes (two recordings, five replays): each
    replay's logits and K/V cache equal the eager step's bit for bit."""
    model = _model(device, dtype)
    cache_g, cache_e = _cache(device, dtype), _cache(device, dtype)
    graphs = DecodeGraphs(model, cache_g, max_blocks_per_seq=WIDTH)
    gen = torch.Generator().manual_seed(7)
    with torch.no_grad():
        for i, lens in enumerate(STEPS):
            step = _step(device, lens, gen)
            want = model.forward_decode_batch_with_cache(kv_cache=cache_e,
                                                         **_padded(step, WIDTH))
            torch.cuda.synchronize()
            other = torch.randn(1 << 20, device=device).square().sum()  # eager work between
            got = graphs(**step).clone()
            torch.cuda.synchronize()
            assert torch.isfinite(other)
            what = f"step {i}, contexts {lens}"
            assert torch.equal(got, want), what
            assert torch.equal(cache_g.k_cache, cache_e.k_cache), what
            assert torch.equal(cache_g.v_cache, cache_e.v_cache), what
    assert (graphs.captures, graphs.replays, graphs.eager_calls) == (2, 5, 0)


def test_replay_of_an_unchanged_step_is_idempotent(device):
    """Replaying the same step three times gives the same logits and cache;
    the step's K/V rows are rewritten with the same values."""
    model, cache = _model(device, torch.bfloat16), _cache(device, torch.bfloat16)
    graphs = DecodeGraphs(model, cache, max_blocks_per_seq=WIDTH)
    step = _step(device, [9, 130, 513], torch.Generator().manual_seed(3))
    with torch.no_grad():
        first = graphs(**step).clone()
        k1 = cache.k_cache.clone()
        for _ in range(2):
            torch.cuda.synchronize()
            assert torch.equal(graphs(**step), first)
            assert torch.equal(cache.k_cache, k1)


@pytest.mark.parametrize("recorded_first", [False, True])
def test_bad_metadata_is_refused_before_anything_is_written(device, recorded_first):
    """A slot that does not match the block table raises the model's own
    message before the graph is recorded or replayed: the cache is unchanged."""
    model, cache = _model(device, torch.bfloat16), _cache(device, torch.bfloat16)
    graphs = DecodeGraphs(model, cache, max_blocks_per_seq=WIDTH)
    gen = torch.Generator().manual_seed(5)
    with torch.no_grad():
        if recorded_first:
            graphs(**_step(device, [40, 41, 42], gen))
        step = _step(device, [40, 41, 42], gen)
        step["slot_mapping"] = step["slot_mapping"].clone()
        step["slot_mapping"][1] += 1
        k0, v0 = cache.k_cache.clone(), cache.v_cache.clone()
        replays = graphs.replays
        with pytest.raises(ValueError, match="slot_mapping must match block_tables"):
            graphs(**step)
        torch.cuda.synchronize()
    assert graphs.replays == replays
    assert torch.equal(cache.k_cache, k0) and torch.equal(cache.v_cache, v0)


def test_shape_errors(device):
    model, cache = _model(device, torch.bfloat16), _cache(device, torch.bfloat16)
    graphs = DecodeGraphs(model, cache, max_blocks_per_seq=WIDTH)
    step = _step(device, [10, 20], torch.Generator().manual_seed(2))
    with pytest.raises(ValueError, match=r"input_ids must have shape \[B, 1\]"):
        graphs(**dict(step, input_ids=step["input_ids"][:, 0]))
    with pytest.raises(ValueError, match="block_tables must use torch.long"):
        graphs(**dict(step, block_tables=step["block_tables"].int()))
    with pytest.raises(ValueError, match="KV cache dtype must match"):
        DecodeGraphs(model, _cache(device, torch.float32), max_blocks_per_seq=WIDTH)


def test_wider_table_than_recorded_runs_eagerly(device):
    """A block table wider than max_blocks_per_seq runs the step eagerly, with
    the same result as the model's own call."""
    model = _model(device, torch.bfloat16)
    cache_g, cache_e = _cache(device, torch.bfloat16), _cache(device, torch.bfloat16)
    graphs = DecodeGraphs(model, cache_g, max_blocks_per_seq=4)
    step = _step(device, [100, 7], torch.Generator().manual_seed(4))
    with torch.no_grad():
        got = graphs(**step)
        want = model.forward_decode_batch_with_cache(kv_cache=cache_e, **step)
    assert graphs.eager_calls == 1 and graphs.captures == 0
    assert torch.equal(got, want)
    assert torch.equal(cache_g.k_cache, cache_e.k_cache)


def _serve(device, dtype, with_graphs, record_ahead=False, prefill=False, prompt_len=None):
    model = _model(device, dtype, seed=11)
    cache = PagedKVCache(2, NBLOCKS, BS, 2, 64, dtype=dtype, device=device)
    scheduler = Scheduler(max_num_batched_tokens=512, max_num_seqs=8, kv_cache=cache)
    gen = torch.Generator().manual_seed(12)
    requests = []
    for i in range(10):
        n = prompt_len or int(torch.randint(3, 200, (1,), generator=gen))
        prompt = torch.randint(0, QWEN_2L["vocab_size"], (n,), generator=gen).tolist()
        requests.append(Request(f"r{i}", prompt, int(torch.randint(4, 24, (1,), generator=gen)),
                                float(i)))
    for r in requests:
        scheduler.add_request(r)
    graphs = DecodeGraphs(model, cache, max_blocks_per_seq=WIDTH) if with_graphs else None
    pgraphs = PrefillGraphs(model, cache, record_at=2) if prefill else None
    with torch.no_grad():
        if record_ahead:
            graphs.record(range(1, 9))
        run_greedy_generation(model, scheduler, decode_graphs=graphs, prefill_graphs=pgraphs)
    if prefill:
        return {r.request_id: r.output_token_ids for r in requests}, pgraphs
    return {r.request_id: r.output_token_ids for r in requests}, graphs


def test_serving_with_decode_graphs_gives_the_eager_tokens(device):
    """Continuous batching in FP32 (ten requests, admissions and exits, so the
    decode batch size changes from step to step): the greedy tokens with the
    decode step replayed from graphs equal those of the eager run."""
    eager, _ = _serve(device, torch.float32, with_graphs=False)
    replayed, graphs = _serve(device, torch.float32, with_graphs=True)
    assert replayed == eager
    assert graphs.captures >= 2 and graphs.replays > graphs.captures


def test_recorded_ahead_serving_records_nothing_more(device):
    """Graphs of batch sizes 1..8 recorded before serving on the runner's own
    block (one block of 16 rows): the serving run records no more, gives the
    eager tokens, and release() returns the block to the allocator."""
    eager, _ = _serve(device, torch.float32, with_graphs=False)
    replayed, graphs = _serve(device, torch.float32, with_graphs=True, record_ahead=True)
    assert replayed == eager
    assert graphs.captures == 8 and graphs.replays > 0
    cache = graphs.kv_cache
    held = len(cache.block_tables[graphs._scratch_key])
    assert held == 1
    free = len(cache.free_blocks)
    graphs.release()
    assert len(cache.free_blocks) == free + held


def _prefill_step(device, qlens, prefixes, gen):
    """One packed prefill of len(qlens) requests on distinct random blocks:
    request r's chunk is positions prefixes[r] .. prefixes[r] + qlens[r] - 1."""
    ctxs = [p + n for p, n in zip(prefixes, qlens)]
    perm = torch.randperm(NBLOCKS, generator=gen).tolist()
    tables, used = [], 0
    for c in ctxs:
        nb = -(-c // BS)
        tables.append(perm[used:used + nb])
        used += nb
    width = max(map(len, tables))
    pos = torch.cat([torch.arange(p, p + n) for p, n in zip(prefixes, qlens)])
    owner = torch.cat([torch.full((n,), r) for r, n in enumerate(qlens)])
    slots = torch.tensor([tables[r][int(t) // BS] * BS + int(t) % BS
                          for r, t in zip(owner.tolist(), pos.tolist())])
    qsl = torch.tensor([0] + torch.tensor(qlens).cumsum(0).tolist())
    step = dict(input_ids=torch.randint(0, QWEN_2L["vocab_size"], (len(pos),), generator=gen),
                position_ids=pos, slot_mapping=slots,
                block_tables=torch.tensor([t + [-1] * (width - len(t)) for t in tables]),
                query_start_loc=qsl, context_lens=torch.tensor(ctxs))
    return {k: v.to(device) for k, v in step.items()}, max(qlens)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("prefixes", [[0, 0], [100, 7]], ids=["prompts", "chunks"])
def test_prefill_replays_equal_the_eager_forward(device, dtype, prefixes):
    """Four packed prefills of one shape (two requests of 64 and 130 tokens),
    recorded on the second: the first runs eagerly, all four equal the eager
    forward bit for bit (logits and K/V), with eager work between calls."""
    model = _model(device, dtype)
    cache_g, cache_e = _cache(device, dtype), _cache(device, dtype)
    graphs = PrefillGraphs(model, cache_g, record_at=2)
    gen = torch.Generator().manual_seed(21)
    with torch.no_grad():
        for i in range(4):
            step, max_q = _prefill_step(device, [64, 130], prefixes, gen)
            want = model.forward_prefill_packed_with_cache(
                step["input_ids"], step["position_ids"], cache_e, step["slot_mapping"],
                step["block_tables"], step["query_start_loc"], step["context_lens"], max_q)
            torch.cuda.synchronize()
            other = torch.randn(1 << 20, device=device).square().sum()
            got = graphs(**step, max_query_len=max_q).clone()
            torch.cuda.synchronize()
            assert torch.isfinite(other)
            assert torch.equal(got, want), f"call {i}"
            assert torch.equal(cache_g.k_cache, cache_e.k_cache), f"call {i}"
            assert torch.equal(cache_g.v_cache, cache_e.v_cache), f"call {i}"
    assert (graphs.eager_calls, graphs.captures, graphs.replays) == (1, 1, 3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_logits_written_into_out_rows(device, dtype):
    """With out= (a row range of a larger buffer, as the runner passes its
    packed logits) both graph kinds and model.logits write exactly the logits
    they return without it: at a 256-byte-aligned row offset (written by the
    GEMM in place) and at an unaligned one (computed, then copied); the rows
    around the range stay untouched."""
    model = _model(device, dtype)
    cache_g, cache_e = _cache(device, dtype), _cache(device, dtype)
    dgraphs = DecodeGraphs(model, cache_g, max_blocks_per_seq=WIDTH)
    pgraphs = PrefillGraphs(model, cache_g, record_at=1)
    vocab = QWEN_2L["vocab_size"]
    row_bytes = vocab * torch.tensor([], dtype=dtype).element_size()
    aligned = next(r for r in range(1, 257) if (r * row_bytes) % 256 == 0)
    gen = torch.Generator().manual_seed(24)
    with torch.no_grad():
        for offset in (aligned, 3):
            step = _step(device, [5, 300, 17], gen)
            want = model.forward_decode_batch_with_cache(kv_cache=cache_e,
                                                         **_padded(step, WIDTH))[:, 0]
            buf = torch.full((offset + 3 + 2, vocab), 7.0, dtype=dtype, device=device)
            got = dgraphs(**step, out=buf[offset:offset + 3])
            assert got.data_ptr() == buf[offset].data_ptr()
            assert torch.equal(buf[offset:offset + 3], want), f"decode, offset {offset}"
            assert (buf[:offset] == 7).all() and (buf[offset + 3:] == 7).all()

            pstep, max_q = _prefill_step(device, [40, 21], [0, 0], gen)
            want = model.forward_prefill_packed_with_cache(
                pstep["input_ids"], pstep["position_ids"], cache_e, pstep["slot_mapping"],
                pstep["block_tables"], pstep["query_start_loc"], pstep["context_lens"], max_q)
            buf = torch.full((offset + 61 + 2, vocab), 7.0, dtype=dtype, device=device)
            pgraphs(**pstep, max_query_len=max_q, out=buf[offset:offset + 61])
            assert torch.equal(buf[offset:offset + 61], want), f"prefill, offset {offset}"
            assert (buf[:offset] == 7).all() and (buf[offset + 61:] == 7).all()
            assert torch.equal(cache_g.k_cache, cache_e.k_cache)
            assert torch.equal(cache_g.v_cache, cache_e.v_cache)

            hidden = torch.randn(9, QWEN_2L["hidden_size"], device=device).to(dtype)
            buf = torch.zeros(offset + 9, vocab, dtype=dtype, device=device)
            model.logits(hidden, buf[offset:])
            assert torch.equal(buf[offset:], model.lm_head(hidden))
    with pytest.raises(ValueError, match="contiguous"):
        model.logits(hidden, buf[:, :vocab - 1])


def test_prefill_graphs_keep_the_most_recent_shapes(device):
    """With max_graphs=1 two alternating shapes keep replacing each other's
    recording; results stay equal to the eager forward."""
    model = _model(device, torch.bfloat16)
    cache_g, cache_e = _cache(device, torch.bfloat16), _cache(device, torch.bfloat16)
    graphs = PrefillGraphs(model, cache_g, max_graphs=1, record_at=2)
    gen = torch.Generator().manual_seed(22)
    with torch.no_grad():
        for i in range(6):
            qlens = [32, 50] if i % 2 == 0 else [17]
            step, max_q = _prefill_step(device, qlens, [0] * len(qlens), gen)
            want = model.forward_prefill_packed_with_cache(
                step["input_ids"], step["position_ids"], cache_e, step["slot_mapping"],
                step["block_tables"], step["query_start_loc"], step["context_lens"], max_q)
            assert torch.equal(graphs(**step, max_query_len=max_q), want), f"call {i}"
    assert len(graphs._recorded) == 1
    assert graphs.eager_calls == 2 and graphs.captures == 4


def test_prefill_bad_metadata_is_refused_before_anything_is_written(device):
    model, cache = _model(device, torch.bfloat16), _cache(device, torch.bfloat16)
    graphs = PrefillGraphs(model, cache, record_at=1)
    gen = torch.Generator().manual_seed(23)
    with torch.no_grad():
        for _ in range(2):  # recorded
            step, max_q = _prefill_step(device, [40, 41], [0, 0], gen)
            graphs(**step, max_query_len=max_q)
        step, max_q = _prefill_step(device, [40, 41], [0, 0], gen)
        step["slot_mapping"] = step["slot_mapping"].clone()
        step["slot_mapping"][3] += 1
        k0, v0 = cache.k_cache.clone(), cache.v_cache.clone()
        replays = graphs.replays
        with pytest.raises(ValueError, match="slot"):
            graphs(**step, max_query_len=max_q)
        torch.cuda.synchronize()
    assert graphs.replays == replays
    assert torch.equal(cache.k_cache, k0) and torch.equal(cache.v_cache, v0)


def test_serving_with_prefill_and_decode_graphs_gives_the_eager_tokens(device):
    """FP32 continuous batching with prompts of one length (so packed prefill
    shapes repeat) and both kinds of graphs: the eager run's tokens."""
    eager, _ = _serve(device, torch.float32, with_graphs=False, prompt_len=48)
    replayed, pgraphs = _serve(device, torch.float32, with_graphs=True, prefill=True,
                               prompt_len=48)
    assert replayed == eager
    assert pgraphs.replays > 0
