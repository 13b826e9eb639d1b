"""Integer rules of the paged KV bookkeeping -- test infrastructure only.

Restates the block allocator of engine/cache.py:4-57 and the slot rule of
engine/runner.py:49-55 in plain Python so tests can check the engine's
allocator and its device-side slot computation bit-exactly.
"""
from __future__ import annotations

import numpy as np


class BlockAllocatorRef:
    """FIFO free list of physical block ids (engine/cache.py:29-46)."""

    def __init__(self, num_blocks: int, block_size: int):
        self.block_size = block_size
        self.free = list(range(num_blocks))
        self.tables: dict[int, list[int]] = {}

    def allocate_sequence(self, seq_id: int, num_tokens: int) -> None:
        need = (num_tokens + self.block_size - 1) // self.block_size  # cache.py:34
        if len(self.free) < need:
            raise RuntimeError("out of KV blocks")
        self.tables[seq_id] = [self.free.pop(0) for _ in range(need)]  # cache.py:38

    def append_token(self, seq_id: int, current_seq_len: int) -> None:
        if current_seq_len % self.block_size == 0:  # cache.py:43
            if not self.free:
                raise RuntimeError("out of KV blocks")
            self.tables[seq_id].append(self.free.pop(0))

    def block_table(self, seq_ids, max_blocks: int) -> np.ndarray:
        """Zero-padded int32 [len(seq_ids), max_blocks] (engine/cache.py:48-57)."""
        out = np.zeros((len(seq_ids), max_blocks), dtype=np.int32)
        for i, s in enumerate(seq_ids):
            blocks = self.tables[s][:max_blocks]
            out[i, : len(blocks)] = blocks
        return out


def slot_mapping_ref(tables: dict, seq_ids, context_lens, block_size: int) -> np.ndarray:
    """Slot of each sequence's newest token (engine/runner.py:49-55).

    pos = ctx - 1; slot = table[pos // BS] * BS + pos % BS.
    """
    out = np.zeros(len(seq_ids), dtype=np.int32)
    for i, s in enumerate(seq_ids):
        pos = int(context_lens[i]) - 1
        out[i] = tables[s][pos // block_size] * block_size + pos % block_size
    return out


def prefill_slots_ref(tables: dict, seq_ids, seq_len: int, block_size: int) -> np.ndarray:
    """Slots of positions 0..seq_len-1 of each sequence, flattened [B * S]
    (the per-position loop of benchmarks/benchmark_engine.py:64-73)."""
    out = np.zeros((len(seq_ids), seq_len), dtype=np.int32)
    for i, s in enumerate(seq_ids):
        for p in range(seq_len):
            out[i, p] = tables[s][p // block_size] * block_size + p % block_size
    return out.reshape(-1)
