"""RMSNorm (with and without the residual add) and silu(gate) * up on the HIP
library (kernels/layer_ops.py) against the PyTorch operations they replace
and against the oracle's RMSNorm (oracle/qwen2_model.py, CPU).

- silu_mul: bit-exact against F.silu(gate) * up on the same GPU (the same
  FP32 formula, expf and IEEE division, and the same two roundings).
- The residual add: bit-exact against residual + x.
- rms_norm: the row sum of squares is added in another order than torch's
  reduction, so the FP32 statistic may differ in its last bits. That can move
  T(r * inv) by one unit in the last place, and the weight product by up to
  two after its own rounding: every output is within two units in the last
  place of the dtype at its value (FP32: relative 1e-6) of the module's
  PyTorch sequence on the GPU and of the oracle. The fused and unfused forms
  give the same bits (one reduction order).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from mini_llm_runtime_amd.kernels import layer_ops as kops
from oracle.qwen2_model import rms_norm as oracle_rms_norm

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32]
ULP = {torch.bfloat16: 2.0 ** -6, torch.float16: 2.0 ** -9, torch.float32: 1e-6}  # 2 ulps
SHAPES = [(1, 896), (5, 896), (48, 896), (2048, 896), (3, 64), (7, 3584), (4, 100), (9, 7)]


def torch_rms_norm(x, weight, eps):
    """Qwen2RMSNorm's PyTorch sequence (statistics in FP32 for 16-bit)."""
    stats = torch.float32 if x.dtype in (torch.float16, torch.bfloat16) else x.dtype
    xf = x.to(stats)
    normalized = xf * torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    return weight.to(x.dtype) * normalized.to(x.dtype)


def within_ulp(got, want, dtype):
    g, w = got.double().cpu(), want.double().cpu()
    bound = ULP[dtype] * w.abs() + 1e-30
    return bool(((g - w).abs() <= bound).all()), (g - w).abs().max().item()


def _inputs(rows, hidden, dtype, device, seed):
    gen = torch.Generator().manual_seed(seed)
    x = (torch.randn(rows, hidden, generator=gen) * 3).to(dtype)
    res = torch.randn(rows, hidden, generator=gen).to(dtype)
    w = (1 + 0.2 * torch.randn(hidden, generator=gen)).to(dtype)
    return x.to(device), res.to(device), w.to(device)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d)[6:])
@pytest.mark.parametrize("rows,hidden", SHAPES)
def test_rms_norm_matches_torch_and_oracle(device, dtype, rows, hidden):
    x, _, w = _inputs(rows, hidden, dtype, device, seed=rows * 1000 + hidden)
    got = kops.rms_norm(x, w, 1e-6)
    ok, err = within_ulp(got, torch_rms_norm(x, w, 1e-6), dtype)
    assert ok, f"against torch on the GPU: max abs {err}"
    ok, err = within_ulp(got, oracle_rms_norm(x.cpu(), w.cpu(), 1e-6), dtype)
    assert ok, f"against the oracle: max abs {err}"
    exact = (got.cpu() == torch_rms_norm(x, w, 1e-6).cpu()).float().mean().item()
    print(f"{rows}x{hidden} {dtype}: {100 * exact:.2f}% of elements bit-equal to torch")


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d)[6:])
@pytest.mark.parametrize("rows,hidden", [(1, 896), (48, 896), (2048, 896), (4, 100)])
def test_fused_residual_add(device, dtype, rows, hidden):
    x, res, w = _inputs(rows, hidden, dtype, device, seed=7 + rows)
    normed, total = kops.rms_norm(x, w, 1e-6, residual=res)
    assert torch.equal(total, res + x)
    assert torch.equal(normed, kops.rms_norm(res + x, w, 1e-6))
    ok, err = within_ulp(normed, torch_rms_norm(res + x, w, 1e-6), dtype)
    assert ok, f"max abs {err}"


def test_rms_norm_strided_rows_and_3d(device):
    """A [B, 1, H] decode activation and a row-strided view."""
    x, _, w = _inputs(8, 1024, torch.bfloat16, device, seed=3)
    got3 = kops.rms_norm(x[:, :896].reshape(8, 1, 896), w[:896], 1e-6)
    want = kops.rms_norm(x[:, :896].contiguous(), w[:896], 1e-6)
    assert got3.shape == (8, 1, 896)
    assert torch.equal(got3.reshape(8, 896), want)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d)[6:])
@pytest.mark.parametrize("rows,inter", [(1, 4864), (48, 4864), (2048, 4864), (5, 7), (3, 100)])
def test_silu_mul_is_bit_exact(device, dtype, rows, inter):
    gen = torch.Generator().manual_seed(rows + inter)
    gate_up = (torch.randn(rows, 2 * inter, generator=gen) * 4).to(dtype).to(device)
    got = kops.silu_mul(gate_up)
    want = F.silu(gate_up[:, :inter]) * gate_up[:, inter:]
    assert got.shape == (rows, inter)
    assert torch.equal(got, want)


def test_special_values(device):
    """Zeros, huge and tiny rows (FP32 statistics); silu at +inf and where
    expf(-g) overflows."""
    w = torch.ones(896, dtype=torch.bfloat16, device=device)
    x = torch.zeros(3, 896, dtype=torch.bfloat16, device=device)
    x[1] = 3.0e38
    x[2] = 1e-30
    got = kops.rms_norm(x, w, 1e-6)
    assert torch.equal(got, torch_rms_norm(x, w, 1e-6))
    g = torch.tensor([[float("inf"), -100.0, 0.0, 1.0]], device=device)
    gu = torch.cat([g, torch.full_like(g, 2.0)], dim=1)
    assert torch.equal(kops.silu_mul(gu), F.silu(g) * 2.0)


def test_argument_errors(device):
    x = torch.zeros(2, 8, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="weight must have shape"):
        kops.rms_norm(x, torch.ones(7, dtype=torch.bfloat16, device=device), 1e-6)
    with pytest.raises(ValueError, match="residual must match"):
        kops.rms_norm(x, torch.ones(8, dtype=torch.bfloat16, device=device), 1e-6,
                      residual=torch.zeros(2, 8, device=device))
    with pytest.raises(ValueError, match="needs a bf16, fp16 or fp32"):
        kops.silu_mul(torch.zeros(2, 8, dtype=torch.float64, device=device))
    with pytest.raises(ValueError, match="2 \\* intermediate"):
        kops.silu_mul(torch.zeros(2, 7, dtype=torch.bfloat16, device=device))
