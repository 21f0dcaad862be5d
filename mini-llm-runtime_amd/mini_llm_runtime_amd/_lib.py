"""Loader for libmlr_attn.so, the C-ABI library of hand-written HIP kernels.

Every kernel call in this package goes through here. There is no fallback:
if the library has not been built, or a tensor is not on a HIP device, the
call raises. ``import torch`` happens first so that the library binds to the
HIP runtime torch already loaded (both carry the soname libamdhip64.so.7),
which keeps torch's streams valid inside the library.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_NAME = "libmlr_attn.so"
# MLR_ATTN_LIB names another build of the same library (e.g. to compare two
# builds on one machine); by default the in-tree build next to this file.
LIB_PATH = os.environ.get(
    "MLR_ATTN_LIB", os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME))

# enum mlr_dtype / mlr_index_dtype in include/mlr_attn.h
DTYPE_CODES = {
    torch.float32: 0,
    torch.float16: 1,
    torch.bfloat16: 2,
    torch.float64: 3,
}
INDEX_CODES = {torch.int32: 0, torch.int64: 1}

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_ptr = ctypes.c_void_p
_c_f64 = ctypes.c_double
_c_size = ctypes.c_size_t

# name -> (restype, argtypes); must match include/mlr_attn.h
_PROTOTYPES = {
    "mlr_last_error": (ctypes.c_char_p, []),
    "mlr_version": (_c_int, []),
    "mlr_kv_write": (
        _c_int,
        [_c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int, _c_i64,
         _c_i64, _c_i64, _c_ptr],
    ),
    "mlr_paged_decode_workspace_size": (
        _c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int]),
    "mlr_paged_decode": (
        _c_int,
        [_c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_f64,
         _c_int, _c_i64, _c_ptr, _c_size, _c_ptr, _c_i64, _c_i64, _c_ptr],
    ),
    "mlr_paged_decode_append": (
        _c_int,
        [_c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_f64,
         _c_int, _c_i64, _c_ptr, _c_size, _c_ptr, _c_ptr, _c_i64, _c_i64,
         _c_ptr, _c_ptr, _c_i64, _c_i64, _c_ptr],
    ),
    "mlr_paged_decode_qkv": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_f64,
         _c_int, _c_i64, _c_ptr, _c_size, _c_ptr, _c_i64, _c_i64, _c_ptr],
    ),
    "mlr_paged_decode_append_static": (
        _c_int,
        [_c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_f64,
         _c_int, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr,
         _c_i64, _c_i64, _c_ptr],
    ),
    "mlr_paged_decode_workspace_check": (_c_int, [_c_ptr, _c_size, _c_ptr]),
    "mlr_paged_decode_static_check": (_c_int, [_c_ptr]),
    "mlr_paged_prefill": (
        _c_int,
        [_c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64,
         _c_i64, _c_f64, _c_int, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr],
    ),
    "mlr_paged_prefill_chunk": (
        _c_int,
        [_c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_f64, _c_int,
         _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr],
    ),
    "mlr_qkv_rope_write": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr,
         _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_int, _c_ptr],
    ),
    "mlr_pa_accumulate": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_i64, _c_ptr]),
    "mlr_build_step_metadata": (
        _c_int,
        [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr,
         _c_ptr, _c_ptr, _c_ptr],
    ),
    "mlr_rms_norm": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64,
         _c_i64, _c_f64, _c_int, _c_ptr],
    ),
    "mlr_silu_mul": (
        _c_int, [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr]),
    "mlr_paged_kv_read_floor_outputs": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "mlr_paged_kv_read_floor": (
        _c_int,
        [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr,
         _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr],
    ),
}

EXPORTED_SYMBOLS = tuple(_PROTOTYPES)


class NativeLibraryError(RuntimeError):
    """libmlr_attn.so is missing or does not export the expected symbols."""


class KernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


# enum mlr_status in include/mlr_attn.h
MLR_ERR_MERGE = 5


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Return the loaded library, loading it on first use."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NativeLibraryError(
                    f"{LIB_PATH} is not built; run __graft_entry__.build() "
                    "(hipcc --offload-arch=gfx950) first")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (restype, argtypes) in _PROTOTYPES.items():
                try:
                    fn = getattr(handle, name)
                except AttributeError as exc:
                    raise NativeLibraryError(
                        f"{LIB_PATH} does not export {name}") from exc
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        message = load().mlr_last_error().decode(errors="replace")
        raise KernelError(f"{what} failed (status {status}): {message}")


def require_hip(*tensors: torch.Tensor, what: str) -> torch.device:
    """Every kernel operand must live on one HIP device; no CPU fallback."""
    device = tensors[0].device
    for tensor in tensors:
        if tensor.device.type != "cuda":
            raise RuntimeError(
                f"{what} runs only on HIP devices (gfx950); got a tensor on "
                f"{tensor.device}")
        if tensor.device != device:
            raise RuntimeError(f"{what}: operands are on different devices")
    return device


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype: torch.dtype, what: str) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"{what}: unsupported dtype {dtype}") from None
