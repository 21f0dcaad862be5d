"""KV-cache write on the GPU: bit-exact against the oracle's index_copy_ scatter."""

from __future__ import annotations

import pytest
import torch

from mini_llm_runtime_amd import workloads
from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache
from oracle.paged_kv_cache import OracleKVCache, write_slots_closed_form

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("slots", [[], [11], [11, 0, 7, 4, 2]])
def test_batched_slot_write_matches_copy_reference(device, dtype, slots):
    # The reference test tests/runtime/test_write_slots_batch.py:11-36 on a GPU.
    torch.manual_seed(42)
    cache = PagedKVCache(2, 3, 4, 2, 8, dtype=dtype, device=device)
    cache.k_cache.normal_()
    cache.v_cache.normal_()
    want_k, want_v = cache.k_cache.cpu(), cache.v_cache.cpu()
    idx = torch.tensor(slots, dtype=torch.int32, device=device)
    k = torch.randn(len(slots), 8, 2, device=device).transpose(1, 2)
    v = torch.randn_like(k)
    write_slots_closed_form(want_k[1], want_v[1], idx.cpu(), k.cpu(), v.cpu())
    cache.write_slots(idx, k, v, layer_idx=1)
    assert torch.equal(cache.k_cache.cpu(), want_k)
    assert torch.equal(cache.v_cache.cpu(), want_v)
    # Rewriting slots in a later call is allowed.
    write_slots_closed_form(want_k[1], want_v[1], idx.cpu(), (k + 1).cpu(), (v + 1).cpu())
    cache.write_slots(idx, k + 1, v + 1, layer_idx=1)
    assert torch.equal(cache.k_cache.cpu(), want_k)
    assert torch.equal(cache.v_cache.cpu(), want_v)


@pytest.mark.parametrize("src", [torch.float32, torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("dst", DTYPES + [torch.float64])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_conversions_round_like_tensor_to(device, src, dst, index_dtype):
    gen = torch.Generator().manual_seed(3)
    oracle = OracleKVCache(1, 6, 4, 2, 16, dtype=dst)
    oracle.k_cache.copy_(torch.randn(oracle.k_cache.shape, generator=gen))
    oracle.v_cache.copy_(torch.randn(oracle.v_cache.shape, generator=gen))
    cache = PagedKVCache(1, 6, 4, 2, 16, dtype=dst, device=device)
    cache.k_cache.copy_(oracle.k_cache)
    cache.v_cache.copy_(oracle.v_cache)
    slots = torch.tensor([23, 0, 5, 17, 9, 12, 3], dtype=index_dtype)
    # Values spanning ties, subnormals and large magnitudes.
    k = (torch.randn(7, 2, 16, generator=gen, dtype=torch.float64) *
         torch.logspace(-40, 30, 16, dtype=torch.float64)).to(src)
    v = (torch.randn(7, 2, 16, generator=gen, dtype=torch.float64) * 3.0).to(src)
    oracle.write_slots(slots, k, v)
    cache.write_slots(slots.to(device), k.to(device), v.to(device))
    assert torch.equal(cache.k_cache.cpu(), oracle.k_cache)
    assert torch.equal(cache.v_cache.cpu(), oracle.v_cache)


def test_untouched_slots_stay_bit_identical(device):
    cache = PagedKVCache(3, 10, 4, 2, 8, dtype=torch.bfloat16, device=device)
    cache.k_cache.normal_()
    cache.v_cache.normal_()
    before_k, before_v = cache.k_cache.clone(), cache.v_cache.clone()
    slots = torch.tensor([5, 39, 0, 22], device=device)
    k = torch.randn(4, 2, 8, device=device, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    cache.write_slots(slots, k, v, layer_idx=2)
    touched = torch.zeros(cache.k_cache.shape[:3], dtype=torch.bool, device=device)
    touched[2, slots // 4, slots % 4] = True
    assert torch.equal(cache.k_cache[~touched], before_k[~touched])
    assert torch.equal(cache.v_cache[~touched], before_v[~touched])
    assert torch.equal(cache.k_cache[2, slots // 4, slots % 4], k)
    assert torch.equal(cache.v_cache[2, slots // 4, slots % 4], v)


@pytest.mark.parametrize("slots,error,message", [
    ([0, 0], ValueError, "distinct"),
    ([0, -1], IndexError, "out-of-range"),
    ([0, 12], IndexError, "out-of-range"),
    ([0.0, 1.0], TypeError, "integer"),
])
def test_invalid_slot_write_does_not_modify_cache(device, slots, error, message):
    cache = PagedKVCache(2, 3, 4, 2, 8, dtype=torch.float32, device=device)
    cache.k_cache.fill_(17)
    cache.v_cache.fill_(23)
    with pytest.raises(error, match=message):
        cache.write_slots(torch.tensor(slots, device=device),
                          torch.randn(2, 2, 8, device=device),
                          torch.randn(2, 2, 8, device=device), layer_idx=1)
    assert torch.all(cache.k_cache == 17) and torch.all(cache.v_cache == 23)


def test_decode_step_write_at_qwen05b_shape(device):
    """64 new tokens into a 24576-block bf16 layer, as one decode step does."""
    wl = workloads.bf16_decode_qwen05b_b64()
    cache = PagedKVCache(1, wl.k_cache.shape[0], 16, 2, 64, dtype=torch.bfloat16,
                         device=device)
    cache.k_cache[0].copy_(wl.k_cache)
    cache.v_cache[0].copy_(wl.v_cache)
    cache.write_slots(wl.slot_mapping.to(device), wl.new_k.to(device), wl.new_v.to(device))
    slots = wl.slot_mapping
    got_k = cache.k_cache[0].view(-1, 2, 64)[slots.to(device)].cpu()
    got_v = cache.v_cache[0].view(-1, 2, 64)[slots.to(device)].cpu()
    assert torch.equal(got_k, wl.new_k) and torch.equal(got_v, wl.new_v)
    mask = torch.ones(wl.k_cache.shape[0] * 16, dtype=torch.bool)
    mask[slots] = False
    assert torch.equal(cache.k_cache[0].view(-1, 2, 64)[mask.to(device)].cpu(),
                       wl.k_cache.view(-1, 2, 64)[mask])
