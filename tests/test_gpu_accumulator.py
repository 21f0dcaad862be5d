"""The accumulator extension's contract on the GPU: the reference's own test
(tests/kernels/test_accumulator_cuda.py:10-27: batches 1, 7, 1024 against
torch.sum(p[:, :, None] * v, dim=1) at 2e-5) plus a float64 CPU sum."""

from __future__ import annotations

import pytest
import torch

from mini_llm_runtime_amd.kernels.accumulator import paged_attention_accumulator_cuda

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("batch", [1, 7, 1024])
def test_paged_attention_accumulator(device, batch):
    gen = torch.Generator(device=device)
    gen.manual_seed(0)
    p = torch.randn(batch, 64, device=device, dtype=torch.float32, generator=gen)
    v = torch.randn(batch, 64, 256, device=device, dtype=torch.float32, generator=gen)
    actual = paged_attention_accumulator_cuda(p, v)
    expected = torch.sum(p[:, :, None] * v, dim=1)
    torch.testing.assert_close(actual, expected, rtol=2e-5, atol=2e-5)
    exact = (p.double()[:, :, None] * v.double()).sum(dim=1)
    assert (actual.double() - exact).abs().max().item() <= 2e-5


def test_non_contiguous_inputs_and_empty_batch(device):
    gen = torch.Generator().manual_seed(1)
    p = torch.randn(64, 5, generator=gen).to(device).t()               # [5, 64] strided
    v = torch.randn(5, 256, 64, generator=gen).to(device).transpose(1, 2)
    got = paged_attention_accumulator_cuda(p, v)
    want = (p.double()[:, :, None] * v.double()).sum(dim=1)
    assert (got.double() - want).abs().max().item() <= 2e-5
    empty = paged_attention_accumulator_cuda(torch.empty(0, 64, device=device),
                                             torch.empty(0, 64, 256, device=device))
    assert empty.shape == (0, 256)
