"""mini_llm_runtime_amd: the paged attention path of mini-llm-runtime on MI355X.

Hand-written gfx950 HIP kernels (libmlr_attn.so, C ABI in include/mlr_attn.h)
behind the reference's Python interface:

- ``runtime.paged_kv_cache.PagedKVCache`` - block pool, allocator, write_slots
- ``kernels.paged_attention`` - batched/single paged decode, chunk prefill
"""

from . import _lib  # noqa: F401

__all__ = ["_lib"]
