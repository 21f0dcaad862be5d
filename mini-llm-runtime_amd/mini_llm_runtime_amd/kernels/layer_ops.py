"""RMSNorm (with the residual add before it) and the MLP's silu(gate) * up on
the HIP library: one launch each where PyTorch issues several.

``rms_norm`` computes what ``Qwen2RMSNorm.forward`` computes (reference
model/qwen2.py:88-123) and ``silu_mul`` what ``F.silu(gate) * up`` in
``Qwen2MLP.forward`` (:768-792) computes, with the same roundings (see
csrc/layer_ops.hip); the decoder layer's residual add before its
post-attention norm rides on ``rms_norm(..., residual=...)``. bf16, fp16 and
FP32 on a HIP device; there is no PyTorch fallback.
"""

from __future__ import annotations

import torch

from .. import _lib

DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def supported(x: torch.Tensor) -> bool:
    """Whether these kernels take `x` (a HIP tensor of a supported dtype)."""
    return x.is_cuda and x.dtype in DTYPES


def _rows(t: torch.Tensor, name: str) -> torch.Tensor:
    """`t` as [rows, last] with unit stride along the last dimension."""
    if t.stride(-1) != 1:
        t = t.contiguous()
    rows = t.reshape(-1, t.shape[-1])
    if rows.numel() and rows.stride(-1) != 1:
        raise ValueError(f"{name} must be unit-stride along its last dimension")
    return rows


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float,
             residual: torch.Tensor | None = None):
    """weight * x / sqrt(mean(x^2) + eps) over the last dimension.

    With `residual`: r = residual + x (rounded to the dtype) is normalised
    instead, and (normalised, r) is returned; r is a new tensor."""
    if not supported(x):
        raise ValueError("rms_norm needs a bf16, fp16 or fp32 tensor on a HIP device")
    hidden = x.shape[-1]
    if weight.shape != (hidden,) or weight.dtype != x.dtype or weight.device != x.device:
        raise ValueError("weight must have shape [hidden] and x's dtype and device")
    if residual is not None and (residual.shape != x.shape or residual.dtype != x.dtype
                                 or residual.device != x.device):
        raise ValueError("residual must match x in shape, dtype and device")
    xr = _rows(x, "x")
    weight = weight.contiguous()
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    res_out = None
    if residual is not None:
        rr = _rows(residual, "residual")
        res_out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    rows = xr.shape[0]
    lib = _lib.load()
    with torch.cuda.device(x.device):
        status = lib.mlr_rms_norm(
            xr.data_ptr(), xr.stride(0) if rows else hidden,
            rr.data_ptr() if residual is not None else None,
            rr.stride(0) if residual is not None and rows else hidden,
            res_out.data_ptr() if residual is not None else None, hidden,
            weight.data_ptr(), out.data_ptr(), hidden, rows, hidden, float(eps),
            _lib.dtype_code(x.dtype, "rms_norm"), _lib.stream_handle(x.device))
    _lib.check(status, "mlr_rms_norm")
    return out if residual is None else (out, res_out)


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up for gate_up = [..., 2 * intermediate] (the gate in the
    first half of the last dimension, up in the second)."""
    if not supported(gate_up):
        raise ValueError("silu_mul needs a bf16, fp16 or fp32 tensor on a HIP device")
    if gate_up.shape[-1] % 2:
        raise ValueError("gate_up's last dimension must be 2 * intermediate")
    inter = gate_up.shape[-1] // 2
    g = _rows(gate_up, "gate_up")
    out = torch.empty(*gate_up.shape[:-1], inter, dtype=gate_up.dtype, device=gate_up.device)
    rows = g.shape[0]
    lib = _lib.load()
    with torch.cuda.device(gate_up.device):
        status = lib.mlr_silu_mul(g.data_ptr(), g.stride(0) if rows else 2 * inter,
                                  out.data_ptr(), inter, rows, inter,
                                  _lib.dtype_code(gate_up.dtype, "silu_mul"),
                                  _lib.stream_handle(gate_up.device))
    _lib.check(status, "mlr_silu_mul")
    return out
