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


def decode_advance_ref(table: np.ndarray, positions, context_lens, block_size: int):
    """One step of device-side decode preparation, restated from the slot rule
    of engine/cache.py:48-57 and engine/runner.py:49-55 (reference): every
    sequence moves one position on (context length too) and its new slot is
    table[b, p // BS] * BS + p % BS on the zero-padded [B, W] int32 table, -1
    when the new position p falls outside the W blocks.  Returns (positions,
    context_lens, slots) as new int32 arrays."""
    table = np.asarray(table, dtype=np.int64)
    pos = np.asarray(positions, dtype=np.int64).reshape(-1) + 1
    ctx = np.asarray(context_lens, dtype=np.int64).reshape(-1) + 1
    slots = np.full(pos.shape, -1, dtype=np.int64)
    for b in range(pos.size):
        blk = pos[b] // block_size
        if pos[b] >= 0 and blk < table.shape[1]:
            slots[b] = table[b, blk] * block_size + pos[b] % block_size
    return pos.astype(np.int32), ctx.astype(np.int32), slots.astype(np.int32)


def argmax_rows_ref(logits: np.ndarray) -> np.ndarray:
    """Greedy token of each row (the torch.argmax of
    benchmarks/benchmark_engine.py:265): index of the largest value, the first
    one among equals; a NaN ranks above every number (numpy's argmax)."""
    return np.argmax(np.asarray(logits, dtype=np.float32), axis=-1).astype(np.int64)
