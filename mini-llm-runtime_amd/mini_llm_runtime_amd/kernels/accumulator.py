"""Batched weighted row sum on the HIP library: the drop-in for the
reference's CUDA accumulator extension (kernels/cuda/accumulator.py:21-37,
kernels/cuda/paged_attention_accumulator.cu).

``paged_attention_accumulator_cuda(p, v)`` keeps the reference's name,
argument checks and messages (ROCm torch reports HIP tensors as CUDA
tensors) and computes ``sum_n p[:, n, None] * v[:, n, :]`` for N=64, D=256
with ``mlr_pa_accumulate``; there is no PyTorch fallback.
"""

from __future__ import annotations

import torch

from .. import _lib


def paged_attention_accumulator_cuda(p: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Compute batched ``sum_n p[n] * v[n, d]`` for N=64 and D=256."""
    if not p.is_cuda or not v.is_cuda:
        raise ValueError("p and v must be CUDA tensors")
    if p.dtype != torch.float32 or v.dtype != torch.float32:
        raise TypeError("p and v must have dtype torch.float32")
    if p.ndim != 2 or p.shape[1] != 64:
        raise ValueError("p must have shape [batch, 64]")
    if v.ndim != 3 or v.shape[1:] != (64, 256):
        raise ValueError("v must have shape [batch, 64, 256]")
    if p.shape[0] != v.shape[0]:
        raise ValueError("p and v must have the same batch dimension")
    if p.device != v.device:
        raise ValueError("p and v must be on the same device")
    p, v = p.contiguous(), v.contiguous()
    out = torch.empty((p.shape[0], 256), dtype=torch.float32, device=p.device)
    if p.shape[0] == 0:
        return out
    lib = _lib.load()
    with torch.cuda.device(p.device):
        status = lib.mlr_pa_accumulate(p.data_ptr(), v.data_ptr(), out.data_ptr(), p.shape[0],
                                       _lib.stream_handle(p.device))
    _lib.check(status, "mlr_pa_accumulate")
    return out


paged_attention_accumulator = paged_attention_accumulator_cuda
