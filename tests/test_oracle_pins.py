"""Pin the oracle (CPU) before trusting it as the reference for the HIP kernels."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle.paged_attention as pa
from oracle.paged_kv_cache import OracleKVCache, write_slots_closed_form
from oracle.slots import pad_block_tables, slots_for_positions

import oracle_pins


@pytest.mark.parametrize("check", oracle_pins.QWEN2_CHECKS, ids=lambda c: c.__name__)
def test_oracle_qwen2_callers_are_pinned(check):
    import oracle.qwen2_attention as qa
    check(qa)


@pytest.mark.parametrize("check", oracle_pins.ALL_CHECKS, ids=lambda c: c.__name__)
def test_oracle_attention_is_pinned(check):
    check(pa)


@pytest.mark.parametrize(
    "hq,hkv,seq_lens,tables",
    [
        (4, 2, [3, 5], [[2, 0, -1], [1, 3, 4]]),
        (2, 2, [3, 5], [[2, 0, -1], [1, 3, 4]]),
        (4, 1, [3, 5], [[2, 0, -1], [1, 3, 4]]),
        (4, 2, [3, 4], [[2, 0], [1, 3]]),
    ],
    ids=["gqa-ragged", "mha-ragged", "mqa-ragged", "seq-length-equals-heads"],
)
def test_batch_parallel_matches_request_loop(hq, hkv, seq_lens, tables):
    # The reference's own cross-check (tests/kernels/test_paged_attention_batch.py:10-43).
    torch.manual_seed(42)
    q = torch.randn(len(seq_lens), hq, 8)
    k_cache = torch.randn(5, 2, hkv, 8)
    v_cache = torch.randn_like(k_cache)
    want = pa.decode_batch_loop(q, k_cache, v_cache, tables, seq_lens, 2)
    got = pa.decode_batch_parallel(q, k_cache, v_cache, torch.tensor(tables),
                                   torch.tensor(seq_lens), 2)
    torch.testing.assert_close(got, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("slots", [[], [11], [11, 0, 7, 4, 2]])
def test_oracle_write_slots_is_the_closed_form(dtype, slots):
    torch.manual_seed(42)
    cache = OracleKVCache(2, 3, 4, 2, 8, dtype=dtype)
    cache.k_cache.normal_()
    cache.v_cache.normal_()
    want_k, want_v = cache.k_cache.clone(), cache.v_cache.clone()
    idx = torch.tensor(slots, dtype=torch.int32)
    k = torch.randn(len(slots), 8, 2).transpose(1, 2)   # non-contiguous FP32 source
    v = torch.randn_like(k)
    write_slots_closed_form(want_k[1], want_v[1], idx, k, v)
    cache.write_slots(idx, k, v, layer_idx=1)
    assert torch.equal(cache.k_cache, want_k)
    assert torch.equal(cache.v_cache, want_v)


@pytest.mark.parametrize("slots,error,message", [
    ([0, 0], ValueError, "distinct"),
    ([0, -1], IndexError, "out-of-range"),
    ([0, 12], IndexError, "out-of-range"),
    ([0.0, 1.0], TypeError, "integer"),
])
def test_oracle_write_slots_rejects_before_writing(slots, error, message):
    cache = OracleKVCache(2, 3, 4, 2, 8, dtype=torch.float32)
    cache.k_cache.fill_(17)
    cache.v_cache.fill_(23)
    with pytest.raises(error, match=message):
        cache.write_slots(torch.tensor(slots), torch.randn(2, 2, 8), torch.randn(2, 2, 8),
                          layer_idx=1)
    assert torch.all(cache.k_cache == 17) and torch.all(cache.v_cache == 23)


def test_oracle_allocator_is_lifo_and_atomic():
    # Assertions of tests/runtime/test_paged_kv_cache.py:62-104 and :285-320.
    cache = OracleKVCache(1, 3, 2, 1, 4)
    cache.add_sequence("A")
    assert cache.reserve_tokens("A", 3) and cache.block_tables["A"] == [0, 1]
    assert cache.reserve_tokens("A", 4) and cache.free_blocks == [2]
    cache.add_sequence("B")
    assert cache.reserve_tokens("B", 3) is False
    assert cache.block_tables["B"] == [] and cache.free_blocks == [2]
    cache.free_sequence("A")
    assert cache.free_blocks == [2, 0, 1]
    assert cache.reserve_tokens("B", 3) and cache.block_tables["B"] == [1, 0]


def test_slot_formula_and_padding():
    table = [7, 2, 5]
    assert slots_for_positions(table, range(0, 9, 4), 4) == [28, 8, 20]
    with pytest.raises(ValueError, match="no KV cache block"):
        slots_for_positions(table, [12], 4)
    assert pad_block_tables([[1], [2, 3, 4], []]) == [[1, -1, -1], [2, 3, 4], [-1, -1, -1]]


@pytest.mark.parametrize("check", oracle_pins.MODEL_CHECKS, ids=lambda c: c.__name__)
def test_oracle_model_is_pinned(check):
    import oracle.qwen2_model as qm
    check(qm)


def test_rope_tables_of_a_cast_module_use_rounded_frequencies():
    """A reference rotary module cast with .to(torch.bfloat16) holds its
    inv_freq buffer in bf16 (registered at model/qwen2.py:135-141), and the
    FP32 positions multiply those rounded values (:164-167). Pinned against
    float64 arithmetic on the rounded frequencies, and shown to differ from
    the FP32-frequency tables at long positions (so the test tells them apart)."""
    import oracle.qwen2_attention as oqa

    pos = torch.tensor([0, 1, 7, 100, 1000])
    cos, sin = oqa.rope_tables(pos, 64, 1e6, torch.float32, freq_dtype=torch.bfloat16)
    inv = 1.0 / (1e6 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))
    inv = inv.to(torch.bfloat16).double().numpy()
    angles = pos.double().numpy()[:, None] * inv
    angles = np.concatenate([angles, angles], axis=-1)
    # FP32 rounding of an angle of up to 1000 rad moves it by at most 3e-5.
    np.testing.assert_allclose(cos.numpy(), np.cos(angles), atol=1e-4)
    np.testing.assert_allclose(sin.numpy(), np.sin(angles), atol=1e-4)
    cos32, _ = oqa.rope_tables(pos, 64, 1e6, torch.float32)
    assert (cos32[-1] - cos[-1]).abs().max().item() > 1e-2
