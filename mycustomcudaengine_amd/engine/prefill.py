"""Batched prompt prefill (reference: benchmarks/benchmark_engine.py:12-129).

prefill_step(model, input_ids [B, S], seq_ids, context_lens) -> last-token
logits [B, vocab].  Per layer: RMSNorm -> fused q/k/v projection -> RoPE in
place (positions 0..S-1) and the paged KV store of all B*S tokens in ONE launch ->
causal prefill attention on the contiguous q/k/v -> o_proj + residual ->
RMSNorm -> fused gate/up -> SwiGLU -> down + residual; then the final
RMSNorm and lm_head on the last position only (benchmark_engine.py:124-127).

Differences from the reference driver, all defects of it (not semantics):
the reference builds slot_mapping element by element and launches the KV
store once per position (benchmark_engine.py:64-73), reorders the attention
output with a stray transpose (:90-91) and computes an unused GQA expansion
(:79-87).  Here slots for every (sequence, position) come from the block
tables in one host->device copy and the attention output is used as
[B, S, Hq * D] directly.  The sequences must already own blocks for S tokens
(KVCacheManager.allocate_sequence), as in the reference.

With chunk_size < S the prompt is processed chunk_size positions at a time:
each chunk's K/V go to the page pool first and its queries attend to every
cached key so far through ops.prefill_attention_paged, so activations scale
with the chunk, not the prompt; the cache holds the same slots as after the
one-shot prefill and cache and logits agree within rounding (the library GEMM
may choose another kernel for the chunk's row count).
"""
from __future__ import annotations

from typing import List

import torch

import my_cuda_engine_cpp as ops

from ..ops import prefill_attention_paged, rope_kv_store


def prefill_step(model, input_ids: torch.Tensor, seq_ids: List[int],
                 context_lens: torch.Tensor = None, chunk_size: int = None) -> torch.Tensor:
    c = model.config
    b, s = input_ids.shape
    if chunk_size is not None and 0 < chunk_size < s:
        return _prefill_chunked(model, input_ids, seq_ids, chunk_size)
    hq, hkv, d = c.num_attention_heads, c.num_key_value_heads, c.head_dim
    dev = input_ids.device
    cache = model.cache_manager
    slots = torch.from_numpy(cache.prefill_slot_mapping(seq_ids, s)).to(dev)
    positions = torch.arange(s, dtype=torch.int32, device=dev).repeat(b, 1).contiguous()
    x = model.weights["model.embed_tokens.weight"][input_ids.reshape(-1)]  # [B*S, hidden]
    kv = cache.kv_cache
    for l in range(c.num_hidden_layers):
        p = f"model.layers.{l}"
        xn = ops.rmsnorm(x, model.weights[f"{p}.input_layernorm.weight"], c.rms_norm_eps)
        q, k, v = model._attention_block_proj(l, xn)
        q4, k4, v4 = q.view(b, s, hq, d), k.view(b, s, hkv, d), v.view(b, s, hkv, d)
        rope_kv_store(q.view(b * s, hq, d), k.view(b * s, hkv, d), v.view(b * s, hkv, d),
                      kv[l, 0], kv[l, 1], model.cos_table, model.sin_table,
                      positions.view(-1), slots)
        attn = ops.prefill_attention(q4, k4, v4, model.scale)  # [B, S, Hq, D]
        x.addmm_(attn.view(b * s, hq * d), model.weights[f"{p}.self_attn.o_proj.weight"].T)
        model._mlp(l, x)
    last = x.view(b, s, -1)[:, -1].contiguous()
    xf = ops.rmsnorm(last, model.weights["model.norm.weight"], c.rms_norm_eps)
    return torch.matmul(xf, model.lm_head.T)


def _prefill_chunked(model, input_ids: torch.Tensor, seq_ids: List[int],
                     chunk: int) -> torch.Tensor:
    c = model.config
    b, s = input_ids.shape
    hq, hkv, d = c.num_attention_heads, c.num_key_value_heads, c.head_dim
    dev = input_ids.device
    cache = model.cache_manager
    all_slots = torch.from_numpy(cache.prefill_slot_mapping(seq_ids, s)).to(dev).view(b, s)
    width = (s + cache.block_size - 1) // cache.block_size
    tables = cache.get_block_table_tensor(seq_ids, width)
    kv = cache.kv_cache
    x = None
    for c0 in range(0, s, chunk):
        c1 = min(s, c0 + chunk)
        n = c1 - c0
        slots = all_slots[:, c0:c1].contiguous().view(-1)
        positions = torch.arange(c0, c1, dtype=torch.int32, device=dev).repeat(b, 1).contiguous()
        ctx = torch.full((b,), c1, dtype=torch.int32, device=dev)
        x = model.weights["model.embed_tokens.weight"][input_ids[:, c0:c1].reshape(-1)]
        for l in range(c.num_hidden_layers):
            p = f"model.layers.{l}"
            xn = ops.rmsnorm(x, model.weights[f"{p}.input_layernorm.weight"], c.rms_norm_eps)
            q, k, v = model._attention_block_proj(l, xn)
            rope_kv_store(q.view(b * n, hq, d), k.view(b * n, hkv, d), v.view(b * n, hkv, d),
                          kv[l, 0], kv[l, 1], model.cos_table, model.sin_table,
                          positions.view(-1), slots)
            # keys split over workgroups only behind a long cached prefix
            # (measured on MI355X, 24/8 heads: from 1536 cached tokens the split
            # ties or wins, by 4-21% for chunks of 128-512 tokens at B = 1-4;
            # at 1024 it is 6% faster to 5% slower, at 512 21% slower)
            attn = prefill_attention_paged(q.view(b, n, hq, d), kv[l, 0], kv[l, 1], tables, ctx,
                                           model.scale, split_keys=c0 >= 1536)
            x.addmm_(attn.view(b * n, hq * d), model.weights[f"{p}.self_attn.o_proj.weight"].T)
            model._mlp(l, x)
    last = x.view(b, -1, x.size(-1))[:, -1].contiguous()
    xf = ops.rmsnorm(last, model.weights["model.norm.weight"], c.rms_norm_eps)
    return torch.matmul(xf, model.lm_head.T)
