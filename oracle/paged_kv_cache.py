"""CPU restatement of the reference's KV block pool (oracle; tests only).

Follows src/mini_llm_runtime/runtime/paged_kv_cache.py: the free list
[NB-1, ..., 0] with pop() from the end (:37, :49-53), all-or-nothing
reserve_tokens (:178-192), free_sequence appending the table back in order
(:92-101) and write_slots (:194-249): validate everything, then
``flat = cache[layer].flatten(0, 1)``; ``flat.index_copy_(0, slots, k.to(dtype))``.
"""

from __future__ import annotations

import torch


class OracleKVCache:
    def __init__(self, num_layers, num_blocks, block_size, num_kv_heads, head_dim,
                 dtype=torch.float16, device="cpu"):
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
        self.free_blocks = list(range(num_blocks - 1, -1, -1))
        self.block_tables: dict = {}
        self.seq_lens: dict = {}

    def add_sequence(self, seq_id):
        if seq_id in self.block_tables:
            raise KeyError(f"Sequence {seq_id} is already exists")
        self.block_tables[seq_id] = []
        self.seq_lens[seq_id] = 0

    def allocate_block(self):
        if not self.free_blocks:
            raise RuntimeError("KV cache out of physical blocks")
        return self.free_blocks.pop()

    def reserve_tokens(self, seq_id, total_num_tokens):
        if total_num_tokens < 0:
            raise ValueError("total_num_tokens cannot be negative")
        have = len(self.block_tables[seq_id])
        need = max((total_num_tokens + self.block_size - 1) // self.block_size - have, 0)
        if len(self.free_blocks) < need:
            return False
        for _ in range(need):
            self.block_tables[seq_id].append(self.allocate_block())
        return True

    def free_sequence(self, seq_id):
        if seq_id not in self.block_tables:
            raise KeyError(f"Unknown sequence {seq_id}")
        self.free_blocks.extend(self.block_tables.pop(seq_id))
        del self.seq_lens[seq_id]

    def write_slots(self, slot_mapping, k, v, layer_idx=0):
        if layer_idx < 0 or layer_idx >= self.num_layers:
            raise IndexError("Unexpected layer_idx")
        if k.ndim != 3 or v.ndim != 3:
            raise ValueError("Expected K/V shape [T, H_kv, D]")
        if k.shape != v.shape:
            raise ValueError("K and V must have the same shape")
        if tuple(k.shape[1:]) != (self.num_kv_heads, self.head_dim):
            raise ValueError(
                f"Expected K/V shape [T, {self.num_kv_heads}, {self.head_dim}]")
        if slot_mapping.ndim != 1:
            raise ValueError("Expected slot_mapping shape [T]")
        if slot_mapping.shape[0] != k.shape[0]:
            raise ValueError("slot_mapping length must match the number of K/V tokens")
        if slot_mapping.dtype not in (torch.int32, torch.int64):
            raise TypeError("slot_mapping must use an integer index dtype")
        num_slots = self.num_blocks * self.block_size
        if torch.any(slot_mapping < 0) or torch.any(slot_mapping >= num_slots):
            raise IndexError("slot_mapping contains an out-of-range slot")
        if slot_mapping.unique().numel() != slot_mapping.numel():
            raise ValueError("slot_mapping must contain distinct slots")
        slots = slot_mapping.to(torch.long)
        self.k_cache[layer_idx].flatten(0, 1).index_copy_(0, slots, k.to(self.dtype))
        self.v_cache[layer_idx].flatten(0, 1).index_copy_(0, slots, v.to(self.dtype))

    def get_layer_cache(self, layer_idx=0):
        if layer_idx < 0 or layer_idx >= self.num_layers:
            raise IndexError("Unexpect layer_idx")
        return self.k_cache[layer_idx], self.v_cache[layer_idx]


def write_slots_closed_form(cache_layer_k, cache_layer_v, slots, k, v):
    """flat[slot[t]] = k[t]: the definition a scatter must meet, one row at a time."""
    block_size = cache_layer_k.shape[1]
    for t, slot in enumerate(slots.tolist()):
        cache_layer_k[slot // block_size, slot % block_size].copy_(k[t])
        cache_layer_v[slot // block_size, slot % block_size].copy_(v[t])
