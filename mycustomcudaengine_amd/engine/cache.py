"""Paged KV-cache block allocator (reference: engine/cache.py:4-57).

Same interface and allocation rules as the reference:
  * kv_cache is one tensor [num_layers, 2, num_blocks, block_size, num_heads,
    head_dim] (K at index 0, V at index 1), so kv_cache[l, 0] is the
    contiguous [num_blocks, block_size, Hkv, D] pool the kernels take;
  * free blocks are handed out first-in first-out (cache.py:29,38);
  * allocate_sequence takes ceil(num_tokens / block_size) blocks (:33-39);
  * append_token takes one more block when current_seq_len % block_size == 0
    (:41-46);
  * get_block_table_tensor returns a zero-padded int32 [B, max_blocks] (:48-57).
Differences: the free list is a deque (O(1) pops), block tables are built on
the host and copied to the device in one transfer (the reference does one copy
per row), free_sequence returns a sequence's blocks to the pool (the reference
never frees), and slot_mapping/prefill_slot_mapping compute the flat slot ids
the KV-store kernel takes.
"""
from __future__ import annotations

from collections import deque
from typing import Dict, List, Sequence

import numpy as np
import torch


class KVCacheManager:
    def __init__(self, num_blocks: int, block_size: int, num_layers: int, num_heads: int,
                 head_dim: int, dtype: torch.dtype = torch.float16, device: str = "cuda"):
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive")
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.num_layers = num_layers
        self.device = device
        # [num_layers, 2 (K, V), num_blocks, block_size, num_heads, head_dim]
        self.kv_cache = torch.empty((num_layers, 2, num_blocks, block_size, num_heads, head_dim),
                                    dtype=dtype, device=device)
        self.free_blocks = deque(range(num_blocks))
        self.block_tables: Dict[int, List[int]] = {}

    # --- allocation rules of the reference ---------------------------------
    def allocate_sequence(self, seq_id: int, num_tokens: int) -> None:
        needed = (num_tokens + self.block_size - 1) // self.block_size
        if len(self.free_blocks) < needed:
            raise RuntimeError("Out of GPU KV-Cache Blocks!")
        self.block_tables[seq_id] = [self.free_blocks.popleft() for _ in range(needed)]

    def append_token(self, seq_id: int, current_seq_len: int) -> None:
        """Allocates a new physical block if the sequence's last block is full."""
        if current_seq_len % self.block_size == 0:
            if not self.free_blocks:
                raise RuntimeError("Out of GPU KV-Cache Blocks during token generation!")
            self.block_tables[seq_id].append(self.free_blocks.popleft())

    def free_sequence(self, seq_id: int) -> None:
        """Returns a sequence's blocks to the end of the free list."""
        self.free_blocks.extend(self.block_tables.pop(seq_id))

    def get_block_table_tensor(self, seq_ids: Sequence[int], max_blocks_per_seq: int) -> torch.Tensor:
        """Zero-padded int32 [len(seq_ids), max_blocks_per_seq] block table."""
        return torch.from_numpy(self.block_table_array(seq_ids, max_blocks_per_seq)).to(self.device)

    # --- host-side helpers ---------------------------------------------------
    def block_table_array(self, seq_ids: Sequence[int], max_blocks_per_seq: int) -> np.ndarray:
        out = np.zeros((len(seq_ids), max_blocks_per_seq), dtype=np.int32)
        for i, s in enumerate(seq_ids):
            blocks = self.block_tables[s][:max_blocks_per_seq]
            out[i, :len(blocks)] = blocks
        return out

    def slot_of(self, seq_id: int, position: int) -> int:
        """Flat slot (block * block_size + offset) of token `position`."""
        table = self.block_tables[seq_id]
        return table[position // self.block_size] * self.block_size + position % self.block_size

    def slot_mapping(self, seq_ids: Sequence[int], context_lens: Sequence[int]) -> np.ndarray:
        """Slot of each sequence's newest token, position ctx - 1
        (the rule of engine/runner.py:49-55)."""
        return np.array([self.slot_of(s, int(c) - 1) for s, c in zip(seq_ids, context_lens)],
                        dtype=np.int32)

    def prefill_slot_mapping(self, seq_ids: Sequence[int], seq_len: int) -> np.ndarray:
        """Slots of positions 0..seq_len-1 of every sequence, flattened [B * S]."""
        bs = self.block_size
        pos = np.arange(seq_len)
        rows = []
        for s in seq_ids:
            table = np.asarray(self.block_tables[s], dtype=np.int64)
            rows.append(table[pos // bs] * bs + pos % bs)
        return np.concatenate(rows).astype(np.int32) if rows else np.zeros(0, np.int32)
