"""Host-side runtime on the CPU: Request, Scheduler, build_model_batch,
execute_model_batch's argument checks and greedy_sample.

The cases follow the reference's own tests (tests/runtime/test_request.py,
test_scheduler.py, test_model_runner.py); the expected values are the closed
forms of the reference's policy (runtime/scheduler.py:81-153, FIFO admission
under a token budget and a seat limit, decodes first; runtime/paged_kv_cache.py
:37-53,92-101, LIFO block reuse; runtime/model_runner.py:54-64, slot =
table[pos // B] * B + pos % B). No kernel runs here.
"""

from __future__ import annotations

import pytest
import torch

from mini_llm_runtime_amd.model.qwen2 import TinyQwen2Config, TinyQwen2ForCausalLM
from mini_llm_runtime_amd.runtime.model_runner import (
    ModelBatch,
    build_model_batch,
    execute_model_batch,
    greedy_sample,
    run_generation_step,
)
from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache
from mini_llm_runtime_amd.runtime.request import FinishReason, Request, RequestStatus
from mini_llm_runtime_amd.runtime.scheduler import Scheduler, SchedulerOutput


def req(rid, prompt, max_new=4):
    return Request(rid, list(prompt), max_new, 0.0)


def sched(budget=8, seats=2, blocks=16, block_size=4):
    cache = PagedKVCache(1, blocks, block_size, 1, 4, device="cpu")
    return Scheduler(max_num_batched_tokens=budget, max_num_seqs=seats, kv_cache=cache)


# ----------------------------------------------------------------------------
# Request (reference tests/runtime/test_request.py)
# ----------------------------------------------------------------------------
def test_request_lifecycle_and_finish_reasons():
    r = req("A", [1, 2, 3], max_new=2)
    assert (r.prompt_len, r.num_output_tokens, r.num_all_tokens) == (3, 0, 3)
    assert r.pending_token_id is None and not r.is_finished
    with pytest.raises(RuntimeError):
        r.update_after_model(num_new_computed_tokens=3, sampled_token_id=9)
    r.start_prefill()
    with pytest.raises(RuntimeError):
        r.start_prefill()
    r.update_after_model(num_new_computed_tokens=3, sampled_token_id=9)
    assert r.status is RequestStatus.DECODING and r.pending_token_id == 9
    assert r.num_computed_tokens == 3 and r.num_all_tokens == 4
    r.update_after_model(num_new_computed_tokens=1, sampled_token_id=7)
    assert r.is_finished and r.finish_reason is FinishReason.LENGTH
    e = req("E", [1], max_new=5)
    e.start_prefill()
    e.update_after_model(num_new_computed_tokens=1, sampled_token_id=0, reached_eos=True)
    assert e.finish_reason is FinishReason.EOS and e.output_token_ids == [0]


# ----------------------------------------------------------------------------
# SchedulerOutput and Scheduler (reference tests/runtime/test_scheduler.py)
# ----------------------------------------------------------------------------
def test_scheduler_output_properties_and_checks():
    empty = SchedulerOutput()
    assert empty.is_empty and empty.total_num_scheduled_tokens == 0
    a, b = req("A", [1, 2, 3]), req("B", [4, 5])
    out = SchedulerOutput([a], [b], {"A": 3, "B": 1})
    assert out.scheduled_requests == [a, b] and out.total_num_scheduled_tokens == 4
    for bad in (dict(prefill_requests=[a], decode_requests=[a], num_scheduled_tokens={"A": 1}),
                dict(prefill_requests=[a], num_scheduled_tokens={}),
                dict(num_scheduled_tokens={"A": 1}),
                dict(prefill_requests=[a], num_scheduled_tokens={"A": 0})):
        with pytest.raises(ValueError):
            SchedulerOutput(**bad)


def test_add_request_aliases_the_cache_table_and_rejects_duplicates():
    s = sched()
    a = req("A", [1, 2])
    s.add_request(a)
    assert a.block_table is s.kv_cache.block_tables["A"] and list(s.waiting) == [a]
    with pytest.raises(ValueError, match="already in the scheduler"):
        s.add_request(req("A", [3]))
    b = req("B", [1])
    b.start_prefill()
    with pytest.raises(ValueError, match="WAITING"):
        s.add_request(b)


def test_fifo_admission_under_budget_and_seats():
    s = sched(budget=8, seats=2)
    a, b, c = req("A", [1, 2, 3]), req("B", [4, 5, 6, 7]), req("C", [8])
    for r in (a, b, c):
        s.add_request(r)
    out = s.schedule()
    # A (3) and B (4) fit the budget of 8; C would fit the budget but not the seats.
    assert out.prefill_requests == [a, b] and out.num_scheduled_tokens == {"A": 3, "B": 4}
    assert (a.block_table, b.block_table) == ([0], [1])  # pop() hands out 0, 1, ...
    assert list(s.waiting) == [c] and s.running == [a, b]


def test_head_of_line_blocks_admission():
    s = sched(budget=8, seats=4)
    big, small = req("big", list(range(9))), req("small", [1])
    s.add_request(big)
    s.add_request(small)
    assert s.schedule().is_empty  # 9 > 8: FIFO stops, small does not skip ahead


def test_decodes_first_then_admission_and_kv_waits():
    s = sched(budget=8, seats=2, blocks=2, block_size=4)
    b = req("B", [20, 21], max_new=2)
    s.add_request(b)
    out = s.schedule()
    s.update_after_model(out, {"B": 5})
    a = req("A", [10, 11, 12, 13, 14], max_new=1)  # needs 2 blocks; 1 is free
    s.add_request(a)
    out = s.schedule()
    assert out.decode_requests == [b] and out.prefill_requests == []
    finished = s.update_after_model(out, {"B": 6})
    assert finished == [b] and b.finish_reason is FinishReason.LENGTH
    assert "B" not in s.kv_cache.block_tables and len(s.kv_cache.free_blocks) == 2
    out = s.schedule()
    assert out.prefill_requests == [a]
    assert a.block_table == [0, 1]  # B's block 0 freed last, popped first


def test_decode_skipped_when_the_pool_is_full():
    s = sched(budget=16, seats=2, blocks=1, block_size=4)
    a = req("A", [1, 2, 3, 4], max_new=3)
    s.add_request(a)
    s.update_after_model(s.schedule(), {"A": 9})
    out = s.schedule()  # position 4 needs a second block: none free
    assert out.is_empty and s.running == [a]


# ----------------------------------------------------------------------------
# build_model_batch (reference tests/runtime/test_model_runner.py:105-237)
# ----------------------------------------------------------------------------
def test_build_model_batch_packs_prefill_then_decode():
    s = sched(budget=16, seats=4, blocks=8, block_size=4)
    d = req("D", [1, 2, 3, 4, 5], max_new=3)
    s.add_request(d)
    s.update_after_model(s.schedule(), {"D": 77})  # D: 5 computed, pending 77
    p = req("P", [9, 8, 7, 6, 5, 4])
    s.add_request(p)
    out = s.schedule()
    batch = build_model_batch(out, block_size=4)
    assert batch.request_ids == ["P", "D"]
    assert batch.request_phases == [RequestStatus.PREFILLING, RequestStatus.DECODING]
    assert batch.input_token_ids.tolist() == [9, 8, 7, 6, 5, 4, 77]
    assert batch.positions.tolist() == [0, 1, 2, 3, 4, 5, 5]
    assert batch.query_start_loc.tolist() == [0, 6, 7]
    assert batch.context_lens.tolist() == [6, 6]
    tp, td = p.block_table, d.block_table
    assert batch.block_tables.tolist() == [tp + [-1] * (2 - len(tp)), td + [-1] * (2 - len(td))]
    want = [tp[q // 4] * 4 + q % 4 for q in range(6)] + [td[1] * 4 + 1]
    assert batch.slot_mapping.tolist() == want
    assert all(t.dtype is torch.long for t in (batch.input_token_ids, batch.positions,
                                                batch.query_start_loc, batch.context_lens,
                                                batch.block_tables, batch.slot_mapping))


def test_build_model_batch_errors():
    assert build_model_batch(SchedulerOutput(), block_size=4).block_tables.shape == (0, 0)
    with pytest.raises(ValueError, match="block_size must be greater than 0"):
        build_model_batch(SchedulerOutput(), block_size=0)
    r = req("A", [1, 2])
    r.status = RequestStatus.DECODING
    with pytest.raises(ValueError, match="has no pending token"):
        build_model_batch(SchedulerOutput(decode_requests=[r], num_scheduled_tokens={"A": 1}), 4)
    fresh = req("A", [1, 2])
    with pytest.raises(ValueError, match="Request A has no KV cache block for position 0"):
        build_model_batch(SchedulerOutput(prefill_requests=[fresh],
                                          num_scheduled_tokens={"A": 2}), 4)
    half = req("H", list(range(6)))
    half.block_table = [3]
    with pytest.raises(ValueError, match="Request H has no KV cache block for position 4"):
        build_model_batch(SchedulerOutput(prefill_requests=[half],
                                          num_scheduled_tokens={"H": 6}), 4)


# ----------------------------------------------------------------------------
# execute_model_batch checks (reference test_model_runner.py:280-565); every
# case raises before any kernel launch
# ----------------------------------------------------------------------------
@pytest.fixture(scope="module")
def tiny_cpu():
    cfg = TinyQwen2Config(vocab_size=31, hidden_size=16, intermediate_size=24,
                          num_hidden_layers=1, num_attention_heads=2, num_key_value_heads=1)
    torch.manual_seed(0)
    model = TinyQwen2ForCausalLM(cfg).float()
    cache = PagedKVCache(1, 8, 4, 1, cfg.head_dim, dtype=torch.float32, device="cpu")
    return model, cache


def good_batch(**changes):
    t = lambda v: torch.tensor(v, dtype=torch.long)  # noqa: E731
    fields = dict(request_ids=["A", "B"], input_token_ids=t([1, 2, 3]), positions=t([0, 1, 4]),
                  query_start_loc=t([0, 2, 3]),
                  request_phases=[RequestStatus.PREFILLING, RequestStatus.DECODING],
                  context_lens=t([2, 5]), block_tables=t([[0, -1], [1, 2]]),
                  slot_mapping=t([0, 1, 8]))
    fields.update(changes)
    return ModelBatch(**fields)


@pytest.mark.parametrize("changes,message", [
    (dict(request_ids=[], request_phases=[]), "empty ModelBatch"),
    (dict(request_phases=[RequestStatus.PREFILLING]),
     "request_phases length must match request_ids"),
    (dict(positions=torch.tensor([0, 1])), "positions length must match input_token_ids"),
    (dict(slot_mapping=torch.tensor([0, 1])), "slot_mapping length must match input_token_ids"),
    (dict(context_lens=torch.tensor([2])), "context_lens length must match request_ids"),
    (dict(block_tables=torch.tensor([[0, -1]])), "block_tables rows must match request_ids"),
    (dict(positions=torch.tensor([0, 1, 4], dtype=torch.int32)),
     "positions must use torch.long dtype"),
    (dict(query_start_loc=torch.tensor([1, 2, 3])), "query_start_loc must start at 0"),
    (dict(query_start_loc=torch.tensor([0, 2, 2])), "query_start_loc must be strictly increasing"),
    (dict(query_start_loc=torch.tensor([0, 1, 2])),
     "query_start_loc must end at the packed token count"),
    (dict(context_lens=torch.tensor([0, 5])), "Request A context_len must be greater than 0"),
    (dict(context_lens=torch.tensor([2, 9])), "Request B block_table has insufficient blocks"),
    (dict(block_tables=torch.tensor([[0, -1], [1, 8]])),
     "Request B block_table contains an invalid physical block"),
    (dict(query_start_loc=torch.tensor([0, 1, 3]), positions=torch.tensor([0, 3, 4]),
          context_lens=torch.tensor([1, 5])),
     "Decode requires exactly one token per request"),
    (dict(request_phases=[RequestStatus.PREFILLING, RequestStatus.WAITING]),
     "Unsupported request phase"),
    # The packed prefill's and the batched decode's metadata checks, run in
    # the same pass (model/qwen2.py check_prefill_packed_inputs,
    # qwen2_attention.py _check_decode_metadata).
    (dict(context_lens=torch.tensor([1, 5])), "context_lens must cover each request's tokens"),
    (dict(positions=torch.tensor([0, 2, 4])), "position_ids must run from context_len"),
    (dict(slot_mapping=torch.tensor([0, 2, 8])),
     "slot_mapping must match block_tables and positions"),
    (dict(positions=torch.tensor([0, 1, 3])), "decode positions must equal context_lens - 1"),
    (dict(slot_mapping=torch.tensor([0, 1, 9])),
     "slot_mapping must match block_tables and positions"),
    (dict(request_phases=[RequestStatus.PREFILLING, RequestStatus.PREFILLING],
          input_token_ids=torch.tensor([1, 2]), positions=torch.tensor([0, 0]),
          query_start_loc=torch.tensor([0, 1, 2]), context_lens=torch.tensor([1, 1]),
          block_tables=torch.tensor([[0], [0]]), slot_mapping=torch.tensor([0, 0])),
     "packed tokens must use distinct write slots"),
    (dict(request_phases=[RequestStatus.DECODING, RequestStatus.DECODING],
          input_token_ids=torch.tensor([1, 2]), positions=torch.tensor([0, 0]),
          query_start_loc=torch.tensor([0, 1, 2]), context_lens=torch.tensor([1, 1]),
          block_tables=torch.tensor([[0], [0]]), slot_mapping=torch.tensor([0, 0])),
     "decode requests must use distinct write slots"),
])
def test_execute_model_batch_rejects(tiny_cpu, changes, message):
    model, cache = tiny_cpu
    with pytest.raises(ValueError, match=message):
        execute_model_batch(model, good_batch(**changes), cache)


def test_execute_model_batch_rejects_dtype_mismatch(tiny_cpu):
    model, _ = tiny_cpu
    cache16 = PagedKVCache(1, 8, 4, 1, 8, dtype=torch.float16, device="cpu")
    with pytest.raises(ValueError, match="KV cache dtype must match model dtype"):
        execute_model_batch(model, good_batch(), cache16)


def test_run_generation_step_errors(tiny_cpu):
    model, cache = tiny_cpu
    with pytest.raises(ValueError, match="no requests"):
        run_generation_step(model, Scheduler(8, 2, kv_cache=cache))
    s = Scheduler(4, 2, kv_cache=PagedKVCache(1, 8, 4, 1, 8, dtype=torch.float32, device="cpu"))
    s.add_request(req("long", list(range(5))))
    with pytest.raises(RuntimeError, match="made no progress"):
        run_generation_step(model, s)


# ----------------------------------------------------------------------------
# greedy_sample (reference test_model_runner.py:627-656)
# ----------------------------------------------------------------------------
def test_greedy_sample_uses_each_requests_last_token():
    batch = good_batch()
    logits = torch.zeros(3, 5)
    logits[0, 4] = 9.0   # A's first token: ignored
    logits[1, 2] = 1.0   # A's last token
    logits[2, 3] = 1.0   # B
    assert greedy_sample(logits, batch) == {"A": 2, "B": 3}
    with pytest.raises(ValueError, match="token dimension"):
        greedy_sample(torch.zeros(2, 5), batch)
    with pytest.raises(ValueError, match=r"\[total_tokens, vocab_size\]"):
        greedy_sample(torch.zeros(3), batch)


# ----------------------------------------------------------------------------
# Block tables of the Qwen2.5-0.5B-shape serving run (workloads.qwen05b_serving)
# against the oracle allocator (oracle/paged_kv_cache.py, the reference's LIFO
# free list). The schedule does not depend on token values (no EOS), so a
# bookkeeping-only run with dummy samples visits the same states.
# ----------------------------------------------------------------------------
def test_serving_schedule_block_tables_match_oracle_allocator():
    from mini_llm_runtime_amd import workloads
    from oracle.paged_kv_cache import OracleKVCache

    w = workloads.qwen05b_serving()
    runs = []
    for cache in (PagedKVCache(1, w.num_blocks, w.block_size, 1, 1, dtype=torch.float32),
                  OracleKVCache(1, w.num_blocks, w.block_size, 1, 1, dtype=torch.float32)):
        s = Scheduler(w.max_num_batched_tokens, w.max_num_seqs, kv_cache=cache)
        reqs = [Request(f"init{i}", p, m, 0.0) for i, (p, m) in enumerate(w.initial)]
        reqs += [Request(f"arr{i}", p, m, 1.0) for i, (p, m) in enumerate(w.arrivals)]
        for r in reqs:
            s.add_request(r)
        trace = []
        for _ in range(160):
            out = s.schedule()
            batch = build_model_batch(out, w.block_size)
            trace.append((batch.request_ids, batch.block_tables.tolist(),
                          batch.slot_mapping.tolist()))
            s.update_after_model(out, {r.request_id: 0 for r in out.scheduled_requests})
        runs.append(trace)
    assert runs[0] == runs[1]
    # The run exercised admission, exit and reuse.
    steps_with_prefill = sum(any(rid.startswith("arr") for rid in ids[:2]) for ids, _, _ in runs[0])
    assert steps_with_prefill > 50


def test_step_graphs_need_a_hip_cache(tiny_cpu):
    """The HIP-graph decode and prefill refuse a cache not on a HIP device."""
    from mini_llm_runtime_amd.runtime.step_graphs import DecodeGraphs, PrefillGraphs

    model, cache = tiny_cpu
    with pytest.raises(ValueError, match="need the KV cache on a HIP device"):
        DecodeGraphs(model, cache, max_blocks_per_seq=4)
    with pytest.raises(ValueError, match="need the KV cache on a HIP device"):
        PrefillGraphs(model, cache)


def test_execute_model_batch_refuses_foreign_step_graphs(tiny_cpu):
    """Step graphs of another model or cache are refused before any launch."""

    class Foreign:
        model = None
        kv_cache = None

    model, cache = tiny_cpu
    with pytest.raises(ValueError, match="decode_graphs must belong to this model"):
        execute_model_batch(model, good_batch(), cache, decode_graphs=Foreign())
    with pytest.raises(ValueError, match="prefill_graphs must belong to this model"):
        execute_model_batch(model, good_batch(), cache, prefill_graphs=Foreign())
