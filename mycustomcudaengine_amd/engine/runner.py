"""Graph-replayed decode runner (reference: engine/runner.py:8-178).

CUDAGraphRunner keeps the reference's interface: static input/output
buffers, _prepare_inputs(seq_ids, context_lens, max_blocks=None) ->
(slot_mapping, block_tables, max_blocks), capture_graph(input_ids,
positions, seq_ids, context_lens) and execute(...) -> logits.  On ROCm,
torch.cuda.CUDAGraph records a hipGraph, so one replay submits the whole
decode step (every layer's kernels) at once.

Differences from the reference:
  * the block-table width frozen into the graph is the sequences' allocated
    capacity (max blocks they own at capture time, or `max_blocks`), not the
    current context; the reference freezes ceil(ctx/16) at capture and then
    decodes past it (runner.py:72-75,164-166);
  * slot ids and block tables are computed on the host from the allocator's
    tables with one device->host read of context_lens per step (the
    reference calls .item() per sequence and copies the table row by row);
  * no clone of the whole KV cache around warm-up/capture: a decode step
    writes only its own slot before any attention reads it, so warm-up
    writes are overwritten by the first real step at that slot (the
    reference clones kv_cache twice, runner.py:108,128,147);
  * capture_graph(..., device_steps=n) also records the greedy token
    (ops.argmax_rows into the static input ids) and the next step's
    preparation (ops.decode_advance: positions, context lengths and slots
    from the device block table, the token appended to a log), so
    run_device_loop(k) replays k steps back to back with no host work in
    between (the reference prepares every step on the host, runner.py:39-60,
    153-178, and takes the argmax between replays, benchmark_engine.py:265).
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from ..ops import argmax_rows, decode_advance


class CUDAGraphRunner:
    def __init__(self, model, max_batch_size: int = 16):
        self.model = model
        self.max_batch_size = max_batch_size
        self.device = model.device
        self.cuda_graph: Optional[torch.cuda.CUDAGraph] = None
        self.is_captured = False
        self.max_blocks_per_seq = 0
        self.device_steps = 0
        self._ctx: List[int] = []
        self._alloc_static(max_batch_size, 1)

    def _alloc_static(self, batch: int, max_blocks: int) -> None:
        dev = self.device
        self.static_input_ids = torch.zeros((batch, 1), dtype=torch.int64, device=dev)
        self.static_positions = torch.zeros((batch, 1), dtype=torch.int32, device=dev)
        self.static_context_lens = torch.zeros((batch,), dtype=torch.int32, device=dev)
        self.static_slot_mapping = torch.zeros((batch,), dtype=torch.int32, device=dev)
        self.static_block_tables = torch.zeros((batch, max_blocks), dtype=torch.int32, device=dev)
        self.static_logits = torch.zeros((batch, self.model.config.vocab_size),
                                         dtype=torch.float16, device=dev)

    @staticmethod
    def _host_ints(t) -> List[int]:
        if isinstance(t, torch.Tensor):
            return [int(v) for v in t.reshape(-1).tolist()]
        return [int(v) for v in t]

    def _prepare_inputs(self, seq_ids: List[int], context_lens,
                        max_blocks: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor, int]:
        cache = self.model.cache_manager
        ctx = self._host_ints(context_lens)
        if max_blocks is None:
            max_blocks = (max(ctx) + cache.block_size - 1) // cache.block_size
        slots = torch.from_numpy(cache.slot_mapping(seq_ids, ctx)).to(self.device)
        tables = torch.from_numpy(cache.block_table_array(seq_ids, max_blocks)).to(self.device)
        return slots, tables, max_blocks

    def _step(self, b: int) -> torch.Tensor:
        return self.model.decode_step(self.static_input_ids[:b], self.static_positions[:b],
                                      self.static_context_lens[:b], self.static_slot_mapping[:b],
                                      self.static_block_tables[:b], self.max_blocks_per_seq)

    def capture_graph(self, input_ids: torch.Tensor, positions: torch.Tensor,
                      seq_ids: List[int], context_lens, max_blocks: Optional[int] = None,
                      warmup: int = 3, device_steps: int = 0) -> None:
        cache = self.model.cache_manager
        b = input_ids.size(0)
        ctx = self._host_ints(context_lens)
        if max_blocks is None:
            owned = max(len(cache.block_tables[s]) for s in seq_ids)
            max_blocks = max(owned, (max(ctx) + cache.block_size - 1) // cache.block_size)
        self.max_blocks_per_seq = max_blocks
        self._alloc_static(b, max_blocks)
        self._fill(input_ids, positions, seq_ids, ctx)

        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            for _ in range(warmup):
                self._step(b)
        s.synchronize()
        self.device_steps = int(device_steps)
        if self.device_steps > 0:
            self.token_log = torch.zeros((self.device_steps, b), dtype=torch.int64,
                                         device=self.device)
            self.step_counter = torch.zeros((1,), dtype=torch.int32, device=self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(graph, stream=s):
                out = self._step(b)
                self.static_logits.copy_(out)
                if self.device_steps > 0:
                    # greedy token -> next input ids; next step's positions,
                    # context lengths and slots, all on the device
                    argmax_rows(self.static_logits[:b], out=self.static_input_ids[:b])
                    decode_advance(self.static_block_tables[:b], self.static_positions[:b],
                                   self.static_context_lens[:b], self.static_slot_mapping[:b],
                                   cache.block_size, input_ids=self.static_input_ids[:b],
                                   token_log=self.token_log, step_counter=self.step_counter)
        s.synchronize()
        torch.cuda.current_stream(self.device).wait_stream(s)
        self.cuda_graph = graph
        self.is_captured = True
        self.batch_size = b

    def _fill(self, input_ids, positions, seq_ids, ctx: List[int]) -> None:
        b = len(seq_ids)
        cache = self.model.cache_manager
        self._seq_ids, self._ctx = list(seq_ids), list(ctx)
        self.static_input_ids[:b].copy_(input_ids)
        self.static_positions[:b].copy_(positions)
        self.static_context_lens[:b].copy_(torch.tensor(ctx, dtype=torch.int32))
        self.static_slot_mapping[:b].copy_(torch.from_numpy(cache.slot_mapping(seq_ids, ctx)))
        self.static_block_tables[:b].copy_(
            torch.from_numpy(cache.block_table_array(seq_ids, self.max_blocks_per_seq)))

    def execute(self, input_ids: torch.Tensor, positions: torch.Tensor, seq_ids: List[int],
                context_lens) -> torch.Tensor:
        assert self.is_captured, "CUDA Graph must be captured before execution!"
        b = input_ids.size(0)
        if b != self.batch_size:
            raise RuntimeError(f"graph captured for batch {self.batch_size}, got {b}")
        ctx = self._host_ints(context_lens)
        if max(ctx) > self.max_blocks_per_seq * self.model.cache_manager.block_size:
            raise RuntimeError("context exceeds the block-table width captured in the graph")
        self._fill(input_ids, positions, seq_ids, ctx)
        self.cuda_graph.replay()
        if self.device_steps > 0:  # the replay also prepared the next step
            self._ctx = [c + 1 for c in ctx]
        return self.static_logits[:b]

    def run_device_loop(self, steps: int) -> torch.Tensor:
        """Replays the captured step `steps` times back to back, each replay
        feeding its greedy token and its successor's slots to the next on the
        device; starts from the state of the last capture_graph / execute.
        Returns the [steps, B] int64 log of generated tokens (a view of the
        runner's buffer).  Needs capture_graph(..., device_steps >= steps) and
        every sequence's blocks allocated for the positions it reaches."""
        assert self.is_captured, "CUDA Graph must be captured before execution!"
        if steps > self.device_steps:
            raise RuntimeError(f"graph captured for {self.device_steps} device steps, got {steps}")
        cache = self.model.cache_manager
        for s, c in zip(self._seq_ids, self._ctx):
            if c + steps - 1 > self.max_blocks_per_seq * cache.block_size:
                raise RuntimeError(f"sequence {s} reaches position {c + steps - 2}, past the "
                                   "block-table width captured in the graph")
            if c + steps - 1 > len(cache.block_tables[s]) * cache.block_size:
                raise RuntimeError(f"sequence {s} has no block for position {c + steps - 2}")
        # The replays read static_block_tables, which the last capture_graph /
        # execute filled; blocks appended since (append_token) are copied in
        # here, or decode_advance would map their positions to block 0.
        b = len(self._seq_ids)
        self.static_block_tables[:b].copy_(
            torch.from_numpy(cache.block_table_array(self._seq_ids, self.max_blocks_per_seq)))
        self.step_counter.zero_()
        for _ in range(steps):
            self.cuda_graph.replay()
        self._ctx = [c + steps for c in self._ctx]
        return self.token_log[:steps]
