"""Host-side checks of the drop-in API (CPU; no kernel is launched).

The product functions raise the reference's errors for bad arguments, check
everything before touching the cache, and refuse CPU tensors instead of
falling back to PyTorch math.
"""

from __future__ import annotations

import pytest
import torch

from mini_llm_runtime_amd.kernels import paged_attention as kpa
from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache


def test_write_slots_valid_call_on_cpu_refuses_to_fall_back():
    cache = PagedKVCache(2, 3, 4, 2, 8, dtype=torch.float32)
    with pytest.raises(RuntimeError, match="only on HIP devices"):
        cache.write_slots(torch.tensor([1, 2]), torch.randn(2, 2, 8), torch.randn(2, 2, 8),
                          layer_idx=1)


@pytest.mark.parametrize("slots,error,message", [
    ([0, 0], ValueError, "distinct"),
    ([0, -1], IndexError, "out-of-range"),
    ([0, 12], IndexError, "out-of-range"),
    ([0.0, 1.0], TypeError, "integer"),
])
def test_invalid_slot_write_does_not_modify_cache(slots, error, message):
    # tests/runtime/test_write_slots_batch.py:39-55 of the reference.
    cache = PagedKVCache(2, 3, 4, 2, 8, dtype=torch.float32)
    cache.k_cache.fill_(17)
    cache.v_cache.fill_(23)
    with pytest.raises(error, match=message):
        cache.write_slots(torch.tensor(slots), torch.randn(2, 2, 8), torch.randn(2, 2, 8),
                          layer_idx=1)
    assert torch.all(cache.k_cache == 17) and torch.all(cache.v_cache == 23)


@pytest.mark.parametrize("layer_idx", [-1, 2])
def test_write_slots_rejects_layer(layer_idx):
    cache = PagedKVCache(2, 2, 4, 2, 8, dtype=torch.float32)
    with pytest.raises(IndexError, match="layer_idx"):
        cache.write_slots(torch.tensor([1]), torch.randn(1, 2, 8), torch.randn(1, 2, 8),
                          layer_idx=layer_idx)


def test_write_slots_rejects_non_3d():
    cache = PagedKVCache(2, 2, 4, 2, 8, dtype=torch.float32)
    with pytest.raises(ValueError, match="Expected K/V shape"):
        cache.write_slots(torch.tensor([0, 1]), torch.randn(2, 8), torch.randn(2, 8), 0)


def test_empty_write_is_allowed_on_any_device():
    cache = PagedKVCache(1, 2, 4, 2, 8, dtype=torch.float32)
    cache.write_slots(torch.tensor([], dtype=torch.long), torch.randn(0, 2, 8),
                      torch.randn(0, 2, 8))


def test_allocator_matches_reference_behaviour():
    cache = PagedKVCache(1, 3, 2, 1, 4)
    cache.add_sequence("A")
    assert cache.reserve_tokens("A", 3) is True and cache.block_tables["A"] == [0, 1]
    assert cache.reserve_tokens("A", 4) is True and len(cache.free_blocks) == 1
    cache.add_sequence("B")
    assert cache.reserve_tokens("B", 3) is False and cache.block_tables["B"] == []
    cache.free_sequence("A")
    assert cache.reserve_tokens("B", 3) is True and cache.block_tables["B"] == [1, 0]
    with pytest.raises(KeyError):
        cache.add_sequence("B")
    with pytest.raises(ValueError, match="negative"):
        cache.reserve_tokens("B", -1)


def test_cpu_append_helpers_keep_reference_semantics():
    cache = PagedKVCache(1, 8, 4, 2, 8, dtype=torch.float32)
    cache.add_sequence(0)
    prompt_k, prompt_v = torch.randn(8, 2, 8), torch.randn(8, 2, 8)
    cache.append_tokens(0, prompt_k, prompt_v)
    cache.append(0, torch.randn(2, 8), torch.randn(2, 8))
    assert cache.seq_lens[0] == 9 and len(cache.block_tables[0]) == 3
    got_k, _ = cache.get_sequence(0)
    torch.testing.assert_close(got_k[:8], prompt_k)
    small = PagedKVCache(1, 2, 4, 2, 8, dtype=torch.float32)
    small.add_sequence(0)
    with pytest.raises(RuntimeError):
        small.append_tokens(0, torch.randn(10, 2, 8), torch.randn(10, 2, 8))
    assert small.block_tables[0] == [] and len(small.free_blocks) == 2


def _decode_args():
    q = torch.randn(2, 4, 8)
    k = torch.randn(5, 2, 2, 8)
    return q, k, torch.randn_like(k), torch.tensor([[2, 0, -1], [1, 3, 4]]), torch.tensor([3, 5])


@pytest.mark.parametrize("mutate,error,message", [
    (lambda a: (a[0][0],) + a[1:], ValueError, r"q must have shape \[B, Hq, D\]"),
    (lambda a: (a[0], a[1][0]) + a[2:], ValueError, "k_cache and v_cache must have shape"),
    (lambda a: (a[0], a[1], a[2][:4]) + a[3:], ValueError, "same shape"),
    (lambda a: (a[0][..., :4],) + a[1:], ValueError, "same head_dim"),
    (lambda a: (torch.randn(2, 3, 8),) + a[1:], ValueError, "divisible"),
    (lambda a: a[:3] + (a[3][:1],) + a[4:], ValueError, "block_tables length"),
    (lambda a: a[:4] + (a[4][:1],), ValueError, "seq_lens length"),
])
def test_batch_decode_validation_messages(mutate, error, message):
    args = mutate(_decode_args())
    with pytest.raises(error, match=message):
        kpa.paged_attention_decode_batch_parallel(*args, block_size=2)


def test_batch_decode_on_cpu_refuses_to_fall_back():
    with pytest.raises(RuntimeError, match="only on HIP devices"):
        kpa.paged_attention_decode_batch_parallel(*_decode_args(), block_size=2)


def test_single_decode_validation_messages():
    q, k, v = torch.randn(4, 8), torch.randn(2, 4, 2, 8), torch.randn(2, 4, 2, 8)
    with pytest.raises(ValueError, match="greater than 0"):
        kpa.paged_attention_decode(q, k, v, [0], 0, 4)
    with pytest.raises(ValueError, match="enough blocks"):
        kpa.paged_attention_decode(q, k, v, [0], 5, 4)
    with pytest.raises(ValueError, match="block_size does not match"):
        kpa.paged_attention_decode(q, k, v, [0, 1, 0], 5, 2)
    with pytest.raises(ValueError, match="divisible"):
        kpa.paged_attention_decode(torch.randn(3, 8), k, v, [0], 3, 4)
    with pytest.raises(RuntimeError, match="only on HIP devices"):
        kpa.paged_attention_decode(q, k, v, [1, 0], 5, 4)


def test_chunk_prefill_validation_messages():
    q = torch.randn(4, 4, 8)
    k = torch.randn(4, 3, 2, 8)
    v = torch.randn_like(k)
    with pytest.raises(ValueError, match="tile_size must be greater than 0"):
        kpa.paged_attention_prefill_chunk_tiled(q, k, v, [2, 0, 3], 5, 9, 3, 0)
    with pytest.raises(ValueError, match="context_len must equal"):
        kpa.paged_attention_prefill_chunk_tiled(q, k, v, [2, 0, 3], 5, 8, 3, 4)
    with pytest.raises(ValueError, match="divisible"):
        kpa.paged_attention_prefill_chunk_tiled(torch.randn(4, 3, 8), k, v, [2, 0, 3], 5,
                                                9, 3, 4)
    with pytest.raises(RuntimeError, match="only on HIP devices"):
        kpa.paged_attention_prefill_chunk_tiled(q, k, v, [2, 0, 3], 5, 9, 3, 4)


def _tiny_attention():
    import types

    from mini_llm_runtime_amd.model.qwen2_attention import Qwen2Attention
    cfg = types.SimpleNamespace(hidden_size=32, num_attention_heads=4, num_key_value_heads=2,
                                head_dim=8, rope_theta=10_000.0)
    torch.manual_seed(0)
    return Qwen2Attention(cfg), cfg


@pytest.mark.parametrize("mutate,message", [
    (lambda a: a.update(context_lens=torch.tensor([0, 6])), "context_lens must be greater than 0"),
    (lambda a: a.update(position_ids=torch.tensor([[3], [5]])),
     "decode positions must equal context_lens - 1"),
    (lambda a: a.update(block_tables=torch.tensor([[1], [2]]), context_lens=torch.tensor([5, 6]),
                        position_ids=torch.tensor([[4], [5]])),
     "block_tables have insufficient blocks for context_lens"),
    (lambda a: a.update(block_tables=torch.tensor([[1, 99], [2, 3]])),
     "block_tables contain an invalid physical block"),
    (lambda a: a.update(slot_mapping=torch.tensor([4 * 1 + 1, 3 * 4 + 1])),
     "slot_mapping must match block_tables and positions"),
    (lambda a: a.update(slot_mapping=torch.tensor([5, 5]), block_tables=torch.tensor([[1, 1], [1, 1]]),
                        position_ids=torch.tensor([[5], [5]]), context_lens=torch.tensor([6, 6])),
     "decode requests must use distinct write slots"),
])
def test_qwen2_decode_batch_validation_messages(mutate, message):
    """Reference model/qwen2.py:578-602: each check raises its message before
    anything is written (one host sync evaluates them all)."""
    from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache
    attn, cfg = _tiny_attention()
    cache = PagedKVCache(1, 8, 4, 2, 8, dtype=torch.float32)
    cache.k_cache.zero_()
    before = cache.k_cache.clone()
    args = dict(position_ids=torch.tensor([[4], [5]]), slot_mapping=torch.tensor([4 * 2 + 0, 4 * 3 + 1]),
                block_tables=torch.tensor([[1, 2], [2, 3]]), context_lens=torch.tensor([5, 6]))
    mutate(args)
    with pytest.raises(ValueError, match=message):
        attn.forward_decode_batch_with_cache(torch.zeros(2, 1, cfg.hidden_size), args["position_ids"],
                                             cache, 0, args["slot_mapping"], args["block_tables"],
                                             args["context_lens"])
    assert torch.equal(cache.k_cache, before)


def test_qwen2_decode_batch_valid_call_refuses_cpu():
    from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache
    attn, cfg = _tiny_attention()
    cache = PagedKVCache(1, 8, 4, 2, 8, dtype=torch.float32)
    with pytest.raises(RuntimeError, match="HIP"):
        attn.forward_decode_batch_with_cache(
            torch.zeros(2, 1, cfg.hidden_size), torch.tensor([[4], [5]]), cache, 0,
            torch.tensor([4 * 2 + 0, 4 * 3 + 1]), torch.tensor([[1, 2], [2, 3]]),
            torch.tensor([5, 6]))


@pytest.mark.parametrize("kwargs,message", [
    (dict(prefix_len=-1, context_len=2), "prefix_len cannot be negative"),
    (dict(prefix_len=0, context_len=5), "context_len must equal prefix_len"),
    (dict(prefix_len=0, context_len=3, tile_size=0), "tile_size must be greater than 0"),
    (dict(prefix_len=0, context_len=3, positions=[[1, 2, 3]]), "contiguous global positions"),
    (dict(prefix_len=0, context_len=3, table=[]), "enough blocks"),
    (dict(prefix_len=0, context_len=3, table=[42]), "out-of-range physical block"),
    (dict(prefix_len=0, context_len=3, slots=[5, 6, 7]), "slot_mapping does not match"),
])
def test_qwen2_chunk_prefill_validation_messages(kwargs, message):
    from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache
    attn, cfg = _tiny_attention()
    cache = PagedKVCache(1, 8, 4, 2, 8, dtype=torch.float32)
    table = kwargs.get("table", [3])
    positions = torch.tensor(kwargs.get("positions", [[0, 1, 2]]))
    slots = torch.tensor(kwargs.get("slots", [12, 13, 14]))
    with pytest.raises(ValueError, match=message):
        attn.forward_prefill_chunk_with_cache(
            torch.zeros(1, 3, cfg.hidden_size), positions, cache, 0, slots, table,
            kwargs["prefix_len"], kwargs["context_len"], kwargs.get("tile_size", 4))


def test_qwen2_chunk_prefill_rejects_repeated_block_before_writing():
    """A table that repeats a block inside the chunk's range passes the
    table/slot checks (every slot follows the table) but maps two positions to
    one slot; write_slots rejects that (reference paged_kv_cache.py:238-239,
    reached from model/qwen2.py:741-746) before anything is written."""
    from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache
    attn, cfg = _tiny_attention()
    cache = PagedKVCache(1, 8, 4, 2, 8, dtype=torch.float32)
    cache.k_cache.fill_(3)
    before = cache.k_cache.clone()
    slots = torch.tensor([12, 13, 14, 15, 12, 13, 14, 15])
    with pytest.raises(ValueError, match="slot_mapping must contain distinct slots"):
        attn.forward_prefill_chunk_with_cache(
            torch.zeros(1, 8, cfg.hidden_size), torch.arange(8).unsqueeze(0), cache, 0,
            slots, [3, 3], 0, 8, 4)
    assert torch.equal(cache.k_cache, before)


def _tiny_model():
    from mini_llm_runtime_amd.model.qwen2 import TinyQwen2Config, TinyQwen2Model
    cfg = TinyQwen2Config(vocab_size=32, hidden_size=32, intermediate_size=64,
                          num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=2)
    torch.manual_seed(0)
    return TinyQwen2Model(cfg), cfg


@pytest.mark.parametrize("qsl,message", [
    ([1, 3], "query_start_loc must start at 0"),
    ([0, 2], "query_start_loc must end at the packed token count"),
    ([0, 4], "query_start_loc must end at the packed token count"),
    ([0, 0, 3], "query_start_loc must be strictly increasing"),
    ([0, 3, 2], "query_start_loc must be strictly increasing"),
])
def test_packed_prefill_rejects_bad_query_start_loc(qsl, message):
    """Each malformed query_start_loc raises its own message (no size error
    from building the token-to-request map first), and nothing is written."""
    from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache
    model, cfg = _tiny_model()
    cache = PagedKVCache(1, 8, 4, 2, 8, dtype=torch.float32)
    cache.k_cache.fill_(9)
    before = cache.k_cache.clone()
    requests = len(qsl) - 1
    ids = torch.tensor([1, 2, 3])
    positions = torch.tensor([0, 1, 2])
    slots = torch.tensor([4, 5, 6])
    tables = torch.tensor([[1, 2]] * requests)
    ctx = torch.tensor([3] * requests)
    with pytest.raises(ValueError, match=message):
        model.forward_prefill_packed_with_cache(ids, positions, cache, slots, tables,
                                                torch.tensor(qsl), ctx, 3)
    assert torch.equal(cache.k_cache, before)


def test_qwen2_attention_matches_reference_state_dict_names():
    attn, _ = _tiny_attention()
    assert list(attn.state_dict()) == [
        "qkv_proj.q_proj.weight", "qkv_proj.q_proj.bias", "qkv_proj.v_proj.weight",
        "qkv_proj.v_proj.bias", "qkv_proj.k_proj.weight", "qkv_proj.k_proj.bias",
        "o_proj.weight"]


def _pre_attention_args(**over):
    from mini_llm_runtime_amd.model.qwen2_attention import Qwen2RotaryEmbedding
    cache = PagedKVCache(1, 4, 16, 2, 8, dtype=torch.float32)
    args = dict(qkv=torch.randn(3, (4 + 4) * 8), positions=torch.arange(3),
                inv_freq=Qwen2RotaryEmbedding(8).inv_freq, kv_cache=cache, layer_idx=0,
                slot_mapping=torch.tensor([0, 5, 9]), num_q_heads=4)
    args.update(over)
    return args


@pytest.mark.parametrize("over,error,message", [
    (dict(layer_idx=1), IndexError, "layer_idx"),
    (dict(num_q_heads=3), ValueError, "multiple"),
    (dict(qkv=torch.randn(3, 60)), ValueError, "qkv must have shape"),
    (dict(positions=torch.arange(3, dtype=torch.int32)), ValueError, "positions"),
    (dict(slot_mapping=torch.tensor([0, 1])), ValueError, "slot_mapping must have shape"),
    (dict(slot_mapping=torch.tensor([0.0, 1.0, 2.0])), TypeError, "integer"),
    (dict(inv_freq=torch.ones(3)), ValueError, "inv_freq"),
    (dict(qkv=torch.randn(3, 64).double()), TypeError, "not supported"),
    (dict(qkv=torch.randn(3, 64).half()), TypeError, "KV cache dtype"),
])
def test_qkv_rope_write_rejects_bad_arguments(over, error, message):
    from mini_llm_runtime_amd.kernels.pre_attention import qkv_rope_write
    with pytest.raises(error, match=message):
        qkv_rope_write(**_pre_attention_args(**over))


def test_qkv_rope_write_refuses_cpu_tensors():
    from mini_llm_runtime_amd.kernels.pre_attention import qkv_rope_write
    args = _pre_attention_args()
    args["kv_cache"].k_cache.fill_(5)
    with pytest.raises(RuntimeError, match="only on HIP devices"):
        qkv_rope_write(**args)
    assert torch.all(args["kv_cache"].k_cache == 5)


def test_qkv_rope_decode_checks_shape_then_device():
    from mini_llm_runtime_amd.kernels.pre_attention import (qkv_rope_decode,
                                                            qkv_rope_decode_fusable)
    from mini_llm_runtime_amd.model.qwen2_attention import Qwen2RotaryEmbedding
    ctx = torch.tensor([3, 20])
    tables = torch.tensor([[0, -1], [1, 2]])
    slots = torch.tensor([2, 35])
    fp32 = PagedKVCache(1, 4, 16, 2, 64, dtype=torch.float32)
    assert not qkv_rope_decode_fusable(torch.float32, fp32, 14)
    with pytest.raises(ValueError, match="needs bf16"):
        qkv_rope_decode(torch.randn(2, 18 * 64), Qwen2RotaryEmbedding(64).inv_freq, fp32, 0,
                        slots, tables, ctx, 14)
    cache = PagedKVCache(1, 4, 16, 2, 64, dtype=torch.bfloat16)
    assert qkv_rope_decode_fusable(torch.bfloat16, cache, 14)
    assert not qkv_rope_decode_fusable(torch.bfloat16, cache, 34)  # 17 heads per KV head
    cache.k_cache.fill_(5)
    qkv = torch.randn(2, 18 * 64).bfloat16()
    with pytest.raises(ValueError, match="qkv must have shape"):
        qkv_rope_decode(qkv[:, :-8], Qwen2RotaryEmbedding(64).inv_freq, cache, 0, slots,
                        tables, ctx, 14)
    with pytest.raises(RuntimeError, match="only on HIP devices"):
        qkv_rope_decode(qkv, Qwen2RotaryEmbedding(64).inv_freq, cache, 0, slots, tables,
                        ctx, 14)
    assert torch.all(cache.k_cache == 5)


@pytest.mark.parametrize("p,v,error,message", [
    (torch.randn(2, 64), torch.randn(2, 64, 256), ValueError, "CUDA tensors"),
])
def test_accumulator_rejects_cpu_tensors(p, v, error, message):
    # kernels/cuda/accumulator.py:25-36 of the reference: the same checks.
    from mini_llm_runtime_amd.kernels.accumulator import paged_attention_accumulator_cuda
    with pytest.raises(error, match=message):
        paged_attention_accumulator_cuda(p, v)


def test_rotary_freq_cache_follows_in_place_changes():
    # The FP32 copy of a bf16 inv_freq buffer is reused while the buffer is
    # unchanged and rebuilt after an in-place change.
    from mini_llm_runtime_amd.kernels import pre_attention as kpre

    f = torch.tensor([1.0, 0.5, 0.25, 0.125], dtype=torch.bfloat16)
    a = kpre._freq_fp32(f)
    assert a.dtype == torch.float32 and torch.equal(a, f.float())
    assert kpre._freq_fp32(f) is a
    f.mul_(2)
    b = kpre._freq_fp32(f)
    assert b is not a and torch.equal(b, f.float())
    g = torch.tensor([1.0, 0.5], dtype=torch.float32)
    assert kpre._freq_fp32(g) is g
