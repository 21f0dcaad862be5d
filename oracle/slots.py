"""Slot and block-table construction of the ModelBatch builder (oracle; tests only).

Follows src/mini_llm_runtime/runtime/model_runner.py:54-64 (one slot per
token: table[pos // bs] * bs + pos % bs, error when the table has no block for
a position) and :110-122 (tables right-padded with -1 to the widest row).
"""

from __future__ import annotations


def slots_for_positions(block_table, positions, block_size):
    slots = []
    for pos in positions:
        logical = pos // block_size
        if logical >= len(block_table):
            raise ValueError(f"no KV cache block for position {pos}")
        slots.append(block_table[logical] * block_size + pos % block_size)
    return slots


def pad_block_tables(tables):
    width = max((len(t) for t in tables), default=0)
    return [list(t) + [-1] * (width - len(t)) for t in tables]
