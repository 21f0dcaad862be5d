"""The C-ABI library loads and exports every function include/mlr_attn.h declares.

Runs without a GPU: loading the library and calling its argument checks never
reaches the HIP runtime (every call below fails validation before a launch).
"""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from mini_llm_runtime_amd import _lib

from conftest import REPO

HEADER = os.path.join(REPO, "include", "mlr_attn.h")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mlr_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for name in ("mlr_kv_write", "mlr_paged_decode", "mlr_paged_prefill",
                 "mlr_paged_prefill_chunk", "mlr_paged_decode_workspace_size",
                 "mlr_last_error", "mlr_version"):
        assert name in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in mlr_attn.h but not exported"
    # The Python prototypes cover the header exactly.
    assert sorted(_lib.EXPORTED_SYMBOLS) == declared_functions()


def test_loader_binds_prototypes():
    lib = _lib.load()
    assert lib.mlr_version() >= 100
    assert lib.mlr_last_error() == b""


def test_workspace_size_is_host_arithmetic():
    lib = _lib.load()
    # D=64, 4096 tokens: 256-token splits. A 256-byte flag region, then
    # 64 x 14 heads x 16 split rows of (m, l), then acc; each part
    # 256-aligned, split rows per head a multiple of 16.
    size = lib.mlr_paged_decode_workspace_size(64, 14, 64, 4096, 0, 2)
    rows = 64 * 14 * 16
    flags = 256
    ml = (rows * 8 + 255) // 256 * 256
    assert size == flags + ml + rows * 64 * 4
    # Short contexts: the generic kernel's default split is an eighth of the
    # context (32 tokens here, 8 splits, padded to 16 rows), the smallest
    # default, so the size covers it whichever kernel the call takes.
    size = lib.mlr_paged_decode_workspace_size(4, 14, 64, 256, 0, 0)
    rows = 4 * 14 * 16
    assert size == flags + (rows * 8 + 255) // 256 * 256 + rows * 64 * 4
    # 13 splits (320-token splits over 4096 tokens) also take 16 rows.
    assert (lib.mlr_paged_decode_workspace_size(64, 14, 64, 4096, 320, 2)
            == lib.mlr_paged_decode_workspace_size(64, 14, 64, 4096, 256, 2))
    assert lib.mlr_paged_decode_workspace_size(0, 14, 64, 4096, 0, 2) == 0


@pytest.mark.parametrize("call,needle", [
    (lambda lib: lib.mlr_kv_write(None, None, 0, -1, 0, 0, 0, 0, 0, 0, None, 1,
                                  None, None, 0, 16, 2, 64, None), b"num_tokens"),
    (lambda lib: lib.mlr_kv_write(None, None, 9, 1, 0, 0, 0, 0, 0, 0, None, 1,
                                  None, None, 0, 16, 2, 64, None), b"source dtype"),
    (lambda lib: lib.mlr_paged_decode(None, 0, 0, None, None, 8, 16, 3, 64, None, 4, 4,
                                      None, 2, 14, 0.125, 2, 0, None, 0, None, 0, 0,
                                      None), b"divisible"),
    (lambda lib: lib.mlr_paged_prefill(None, 0, 0, None, None, 8, 16, 2, 300, None, 4, 4,
                                       None, None, 1, 4, 14, 0.125, 2, 64, None, 0, 0,
                                       None), b"head_dim"),
    (lambda lib: lib.mlr_paged_decode_qkv(None, 1152, None, None, None, 8, 16, 2, 64,
                                          None, 4, 4, None, None, 2, 14, 0.125, 2, 0, None,
                                          0, None, 0, 0, None), b"null qkv or inv_freq"),
    # FP32 has no fused rotary path: refused on the host, before any launch
    # (the device pointers are never dereferenced).
    (lambda lib: lib.mlr_paged_decode_qkv(1 << 12, 1152, 1 << 13, 1 << 20, 1 << 21, 8,
                                          16, 2, 64, 1 << 22, 4, 4, 1 << 23, 1 << 24, 2, 14,
                                          0.125, 0, 0, 1 << 25, 1 << 30, 1 << 26, 896, 64,
                                          None), b"needs bf16"),
    # The workspace check validates its arguments before touching the stream.
    (lambda lib: lib.mlr_paged_decode_workspace_check(None, 4096, None), b"flag region"),
    (lambda lib: lib.mlr_paged_decode_workspace_check(1 << 20, 128, None), b"flag region"),
    (lambda lib: lib.mlr_paged_decode_workspace_check((1 << 20) + 64, 4096, None),
     b"256-byte aligned"),
])
def test_argument_errors_return_before_any_launch(call, needle):
    lib = _lib.load()
    assert call(lib) == 1  # MLR_ERR_INVALID
    assert needle in lib.mlr_last_error()


def test_empty_kv_write_is_a_no_op():
    lib = _lib.load()
    assert lib.mlr_kv_write(None, None, 2, 0, 0, 0, 0, 0, 0, 0, None, 1, None, None,
                            2, 16, 2, 64, None) == 0
