"""Paged KV cache: block pool, LIFO block allocator and the slot-mapping write.

Same interface and semantics as the reference's ``PagedKVCache``
(runtime/paged_kv_cache.py): one pool tensor per K and V of shape
[num_layers, num_blocks, block_size, num_kv_heads, head_dim]; a free list that
starts as [num_blocks-1, ..., 0] so ``pop()`` hands out 0, 1, 2, ... and freed
blocks are reused last-freed-first; all-or-nothing ``reserve_tokens``; and
``write_slots``, which validates everything before touching the pool and then
scatters K/V rows with the HIP kernel ``mlr_kv_write``.

Storage layout matters for the kernels: a layer is one contiguous
[num_blocks, block_size, Hkv, D] array, so a slot (block * block_size + offset)
is a contiguous run of Hkv * D elements and a block is one contiguous
block_size * Hkv * D run.
"""

from __future__ import annotations

import torch

from .. import _lib


class PagedKVCache:
    def __init__(
        self,
        num_layers: int,
        num_blocks: int,
        block_size: int,
        num_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype = torch.float16,
        device: torch.device | str = "cpu",
    ):
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = torch.device(device)
        shape = (num_layers, num_blocks, block_size, num_kv_heads, head_dim)
        self.k_cache = torch.empty(shape, dtype=dtype, device=device)
        self.v_cache = torch.empty_like(self.k_cache)
        # Reference runtime/paged_kv_cache.py:37 - pop() yields 0, 1, 2, ...
        self.free_blocks: list[int] = list(range(num_blocks - 1, -1, -1))
        self.block_tables: dict[int, list[int]] = {}
        self.seq_lens: dict[int, int] = {}

    # ------------------------------------------------------------------
    # Allocator (reference :42-53, :92-101, :104-119, :178-192)
    # ------------------------------------------------------------------
    def add_sequence(self, seq_id) -> None:
        if seq_id in self.block_tables:
            raise KeyError(f"Sequence {seq_id} is already exists")
        self.block_tables[seq_id] = []
        self.seq_lens[seq_id] = 0

    def _allocate_block(self) -> int:
        if not self.free_blocks:
            raise RuntimeError("KV cache out of physical blocks")
        return self.free_blocks.pop()

    def free_sequence(self, seq_id) -> None:
        if seq_id not in self.block_tables:
            raise KeyError(f"Unknown sequence {seq_id}")
        blocks = self.block_tables[seq_id]
        # Appended in table order: the table's last block is reused first.
        self.free_blocks.extend(blocks)
        blocks.clear()
        del self.block_tables[seq_id]
        del self.seq_lens[seq_id]

    def _check_capacity(self, seq_id, num_new_tokens: int) -> bool:
        final_len = self.seq_lens[seq_id] + num_new_tokens
        needed = -(-final_len // self.block_size) - len(self.block_tables[seq_id])
        return len(self.free_blocks) >= needed

    def reserve_tokens(self, seq_id, total_num_tokens: int) -> bool:
        if total_num_tokens < 0:
            raise ValueError("total_num_tokens cannot be negative")
        needed = -(-total_num_tokens // self.block_size) - len(self.block_tables[seq_id])
        needed = max(needed, 0)
        if len(self.free_blocks) < needed:
            return False
        self.block_tables[seq_id].extend(self._allocate_block() for _ in range(needed))
        return True

    # ------------------------------------------------------------------
    # Token-at-a-time helpers of the reference (:55-176). They address layer 0
    # only, as the reference does, and are not on the serving path.
    # ------------------------------------------------------------------
    def _block_and_offset(self, seq_id, position: int):
        """Physical block and row of a sequence's token position."""
        return (self.block_tables[seq_id][position // self.block_size],
                position % self.block_size)

    def append(self, seq_id, k: torch.Tensor, v: torch.Tensor) -> None:
        if seq_id not in self.block_tables:
            raise KeyError(f"Unknow sequence {seq_id}")
        expected = (self.num_kv_heads, self.head_dim)
        if tuple(k.shape) != expected:
            raise ValueError(f"Expected k shape {expected}, got {tuple(k.shape)}")
        if tuple(v.shape) != expected:
            raise ValueError(f"Expected v shape {expected}, got {tuple(v.shape)}")
        position = self.seq_lens[seq_id]
        if position // self.block_size == len(self.block_tables[seq_id]):
            self.block_tables[seq_id].append(self._allocate_block())
        block, offset = self._block_and_offset(seq_id, position)
        self.k_cache[0, block, offset].copy_(k)
        self.v_cache[0, block, offset].copy_(v)
        self.seq_lens[seq_id] += 1

    def append_tokens(self, seq_id, k: torch.Tensor, v: torch.Tensor) -> None:
        if k.ndim != 3 or v.ndim != 3:
            raise ValueError("Expected K/V shape [T, H_kv, D]")
        if k.shape != v.shape:
            raise ValueError("K and V must have the same shape")
        if tuple(k.shape[1:]) != (self.num_kv_heads, self.head_dim):
            raise ValueError(
                f"Expected K/V shape [T, {self.num_kv_heads}, {self.head_dim}]")
        if not self._check_capacity(seq_id, k.shape[0]):
            raise RuntimeError("out of memory")
        for i in range(k.shape[0]):
            self.append(seq_id, k[i], v[i])

    def get_sequence(self, seq_id):
        seq_len = self.seq_lens[seq_id]
        k_out = torch.empty(seq_len, self.num_kv_heads, self.head_dim,
                            dtype=self.dtype, device=self.device)
        v_out = torch.empty_like(k_out)
        for position in range(seq_len):
            block, offset = self._block_and_offset(seq_id, position)
            k_out[position].copy_(self.k_cache[0, block, offset])
            v_out[position].copy_(self.v_cache[0, block, offset])
        return k_out, v_out

    # ------------------------------------------------------------------
    # Hot path: slot-mapping write (reference :194-249)
    # ------------------------------------------------------------------
    def write_slots(
        self,
        slot_mapping: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        layer_idx: int = 0,
        *,
        validate: bool = True,
    ) -> None:
        """Write [T, Hkv, D] K/V to distinct flat slots of one layer.

        Empty writes are allowed; duplicate slots are rejected; the source
        dtype is converted with round-to-nearest-even like Tensor.to. All
        checks run before the pool is touched. validate=False skips the value
        checks on slot_mapping (range, distinctness), which cost a host sync,
        for callers that validated the step's metadata already; shape, dtype
        and device checks always run, and the kernel skips out-of-range slots.
        """
        if layer_idx < 0 or layer_idx >= self.num_layers:
            raise IndexError("Unexpected layer_idx")
        expected_tail = (self.num_kv_heads, self.head_dim)
        if k.ndim != 3 or v.ndim != 3:
            raise ValueError("Expected K/V shape [T, H_kv, D]")
        if k.shape != v.shape:
            raise ValueError("K and V must have the same shape")
        if tuple(k.shape[1:]) != expected_tail:
            raise ValueError(
                f"Expected K/V shape [T, {self.num_kv_heads}, {self.head_dim}]")
        if slot_mapping.ndim != 1:
            raise ValueError("Expected slot_mapping shape [T]")
        if slot_mapping.shape[0] != k.shape[0]:
            raise ValueError("slot_mapping length must match the number of K/V tokens")
        if slot_mapping.dtype not in (torch.int32, torch.int64):
            raise TypeError("slot_mapping must use an integer index dtype")
        cache_device = self.k_cache.device
        if (slot_mapping.device != cache_device or k.device != cache_device
                or v.device != cache_device):
            raise ValueError("slot_mapping and K/V must be on the KV cache device")
        if k.dtype != v.dtype:
            raise TypeError("K and V must share one dtype")
        if validate:
            self.check_slots(slot_mapping)
        if k.shape[0] == 0:
            return
        self._launch_write(slot_mapping, k, v, layer_idx)

    def check_slots(self, slot_mapping: torch.Tensor) -> None:
        """The value checks of write_slots (reference :235-239): every slot in
        range, no slot twice. Both run in one device pass and one host sync;
        the range check wins when both fail, as in the reference."""
        if slot_mapping.numel() == 0:
            return
        num_slots = self.num_blocks * self.block_size
        ordered = slot_mapping.sort().values
        flags = torch.stack([
            ((ordered[0] < 0) | (ordered[-1] >= num_slots)),
            (ordered[1:] == ordered[:-1]).any(),
        ]).cpu()
        if bool(flags[0]):
            raise IndexError("slot_mapping contains an out-of-range slot")
        if bool(flags[1]):
            raise ValueError("slot_mapping must contain distinct slots")

    def _launch_write(self, slot_mapping: torch.Tensor, k: torch.Tensor,
                      v: torch.Tensor, layer_idx: int) -> None:
        device = _lib.require_hip(self.k_cache, slot_mapping, k, v,
                                  what="PagedKVCache.write_slots")
        lib = _lib.load()
        layer_k = self.k_cache[layer_idx]
        layer_v = self.v_cache[layer_idx]
        if not (layer_k.is_contiguous() and layer_v.is_contiguous()):
            raise ValueError("KV cache layers must be contiguous")
        with torch.cuda.device(device):
            status = lib.mlr_kv_write(
                k.data_ptr(), v.data_ptr(), _lib.dtype_code(k.dtype, "write_slots"),
                k.shape[0], k.stride(0), k.stride(1), k.stride(2),
                v.stride(0), v.stride(1), v.stride(2),
                slot_mapping.data_ptr(), _lib.INDEX_CODES[slot_mapping.dtype],
                layer_k.data_ptr(), layer_v.data_ptr(),
                _lib.dtype_code(self.dtype, "write_slots"),
                self.num_blocks * self.block_size, self.num_kv_heads,
                self.head_dim, _lib.stream_handle(device))
        _lib.check(status, "mlr_kv_write")

    def get_layer_cache(self, layer_idx: int = 0):
        if layer_idx < 0 or layer_idx >= self.num_layers:
            raise IndexError("Unexpect layer_idx")
        return self.k_cache[layer_idx], self.v_cache[layer_idx]
