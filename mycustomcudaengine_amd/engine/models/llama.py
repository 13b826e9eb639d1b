"""Llama-3.2-3B wrapper over the paged KV cache (reference:
engine/models/llama.py:10-174).

Llama3BConfig reads a Hugging Face config dict with the reference's defaults
(llama.py:10-23).  Llama3BEngineModel.decode_step runs one token for B
sequences with the same arguments and result as the reference (llama.py:
59-174): embedding -> L x [RMSNorm -> q/k/v projection -> RoPE in place ->
paged KV store -> paged decode attention -> o_proj + residual -> RMSNorm ->
gate/up projection -> SwiGLU -> down projection + residual] -> RMSNorm ->
lm_head (tied to the embedding when lm_head.weight is absent, llama.py:173).
It makes no host synchronisation and no host-visible allocation, so it can
be captured into a hipGraph.

Layout choices: the q/k/v projection weights of a layer are concatenated
into one [(Hq + 2 Hkv) D, hidden] matrix and gate/up into one [2 I, hidden]
matrix, so a layer runs 4 GEMMs instead of 7 and SwiGLU reads the gate/up
GEMM output directly (the reference concatenates gate and up activations
with torch.cat every step, llama.py:161).  The original weight names stay
in `weights` as views into the fused matrices.  q/k/v are strided views of
the fused projection output.  When the block tables hold at most 1024 tokens
(the decode attention's one-workgroup-per-sequence mode) one launch rotates
q and k, writes k/v to their pages and runs the attention
(decode_rope_attention); for longer tables one fused launch rotates q (into
a contiguous buffer) and k and writes k/v to their pages, then the decode
attention runs (the reference calls rope_inplace, paged_kv_store and
paged_attention_decode, llama.py:117-134).  The o_proj / down_proj GEMMs add
into the residual stream in place instead of a separate add.  At decode
batch sizes (at most 8 tokens, fp16, the 3B model's widths) the projections
run on the decode-sized GEMM kernels: RMSNorm fused in front of the q/k/v and
gate/up projections, SwiGLU fused behind gate/up, the residual adds fused
into o_proj / down_proj, the final RMSNorm in front of lm_head -- 4 launches
per layer besides the attention instead of 7; other shapes use torch.matmul
(hipBLASLt) with the separate RMSNorm / SwiGLU ops.
RoPE tables cover max_position_embeddings positions (capped at 131072)
instead of the reference's fixed 4096 (llama.py:42).
"""
from __future__ import annotations

import math
from typing import Dict

import torch

import my_cuda_engine_cpp as ops

from ...ops import (PER_SEQ_MAX_TOKENS, decode_gemm, decode_rope_attention, rmsnorm_decode_gemm,
                   rope_kv_store)
from ..cache import KVCacheManager

ROPE_TABLE_CAP = 131072


class Llama3BConfig:
    def __init__(self, config_dict: dict):
        self.hidden_size: int = config_dict.get("hidden_size", 3072)
        self.intermediate_size: int = config_dict.get("intermediate_size", 8192)
        self.num_hidden_layers: int = config_dict.get("num_hidden_layers", 28)
        self.num_attention_heads: int = config_dict.get("num_attention_heads", 24)
        self.num_key_value_heads: int = config_dict.get("num_key_value_heads", 8)
        self.head_dim: int = config_dict.get("head_dim", 128)
        self.vocab_size: int = config_dict.get("vocab_size", 128256)
        self.rms_norm_eps: float = config_dict.get("rms_norm_eps", 1e-5)
        self.rope_theta: float = config_dict.get("rope_theta", 500000.0)
        self.max_position_embeddings: int = config_dict.get("max_position_embeddings", 131072)


def rope_tables(max_positions: int, head_dim: int, theta: float, device):
    """cos/sin [max_positions, head_dim/2] fp32, inv_freq = theta^(-2i/D)
    (reference: engine/models/llama.py:47-57)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device)
                                / head_dim))
    t = torch.arange(max_positions, dtype=torch.float32, device=device)
    freqs = torch.outer(t, inv_freq)
    return torch.cos(freqs), torch.sin(freqs)


class Llama3BEngineModel:
    def __init__(self, config: Llama3BConfig, weights: Dict[str, torch.Tensor],
                 cache_manager: KVCacheManager, rope_positions: int | None = None):
        self.config = config
        self.weights = weights
        self.cache_manager = cache_manager
        self.scale = 1.0 / math.sqrt(config.head_dim)
        emb = weights["model.embed_tokens.weight"]
        self.device = emb.device
        self.dtype = emb.dtype
        n = rope_positions or min(config.max_position_embeddings, ROPE_TABLE_CAP)
        self.cos_table, self.sin_table = rope_tables(n, config.head_dim, config.rope_theta,
                                                     self.device)
        self._fuse_weights()

    def _fuse_weights(self) -> None:
        """Concatenate q/k/v and gate/up per layer; keep the original names as
        views into the fused matrices (no extra memory once the originals go)."""
        w = self.weights
        self.w_qkv, self.w_gate_up = [], []
        for l in range(self.config.num_hidden_layers):
            p = f"model.layers.{l}"
            names = [f"{p}.self_attn.{n}_proj.weight" for n in ("q", "k", "v")]
            qkv = torch.cat([w[n] for n in names], dim=0)
            off = 0
            for n in names:
                rows = w[n].shape[0]
                w[n] = qkv[off:off + rows]
                off += rows
            gu_names = [f"{p}.mlp.gate_proj.weight", f"{p}.mlp.up_proj.weight"]
            gu = torch.cat([w[n] for n in gu_names], dim=0)
            inter = w[gu_names[0]].shape[0]
            w[gu_names[0]], w[gu_names[1]] = gu[:inter], gu[inter:]
            self.w_qkv.append(qkv)
            self.w_gate_up.append(gu)
        self.lm_head = w.get("lm_head.weight", w["model.embed_tokens.weight"])

    # -----------------------------------------------------------------------
    def _attention_block_proj(self, l: int, x_norm: torch.Tensor):
        """q/k/v projection; returns strided views (tokens, heads, head_dim)."""
        c = self.config
        qkv = torch.matmul(x_norm, self.w_qkv[l].T)
        hq, hkv, d = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        q = qkv[:, : hq * d]
        k = qkv[:, hq * d:(hq + hkv) * d]
        v = qkv[:, (hq + hkv) * d:]
        return q, k, v

    def _mlp(self, l: int, x: torch.Tensor) -> None:
        """x += down(SwiGLU(gate_up(RMSNorm(x)))), the residual add done by the
        down-projection GEMM (addmm_ accumulates into x)."""
        p = f"model.layers.{l}"
        xn = ops.rmsnorm(x, self.weights[f"{p}.post_attention_layernorm.weight"],
                         self.config.rms_norm_eps)
        act = ops.swiglu(torch.matmul(xn, self.w_gate_up[l].T))
        x.addmm_(act, self.weights[f"{p}.mlp.down_proj.weight"].T)

    def _decode_gemms_take(self, b: int) -> bool:
        """Whether the decode-sized GEMM kernels take every projection of a
        decode step of b tokens: fp16, b <= 8 (the down projection stages its
        whole K = intermediate-size rows), K in {2048, 3072, 4096} (8192 for
        down_proj), every N a multiple of 16."""
        c = self.config
        ks = {2048, 3072, 4096}
        hq, hkv, d = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        return (self.dtype == torch.float16 and 1 <= b <= 8 and c.hidden_size in ks and
                hq * d in ks and c.intermediate_size in ks | {8192} and
                all(n % 16 == 0 for n in ((hq + 2 * hkv) * d, c.hidden_size,
                                          c.intermediate_size, self.lm_head.shape[0])))

    def decode_step(self, input_ids: torch.Tensor, positions: torch.Tensor,
                    context_lens: torch.Tensor, slot_mapping: torch.Tensor,
                    block_tables_tensor: torch.Tensor, max_blocks_per_seq: int) -> torch.Tensor:
        """One decode token for B sequences; logits [B, vocab].  No host syncs."""
        c = self.config
        b = input_ids.size(0)
        hq, hkv, d = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        x = self.weights["model.embed_tokens.weight"][input_ids.view(-1)]  # [B, hidden]
        kv = self.cache_manager.kv_cache
        # tables of at most PER_SEQ_MAX_TOKENS: RoPE + KV append fused into attention
        fused = max_blocks_per_seq * self.cache_manager.block_size <= PER_SEQ_MAX_TOKENS
        gemms = self._decode_gemms_take(b)
        eps = c.rms_norm_eps
        for l in range(c.num_hidden_layers):
            p = f"model.layers.{l}"
            ln_in = self.weights[f"{p}.input_layernorm.weight"]
            if gemms:  # RMSNorm + q/k/v projection in one launch
                qkv = rmsnorm_decode_gemm(x, ln_in, eps, self.w_qkv[l])
                q, k, v = qkv[:, : hq * d], qkv[:, hq * d:(hq + hkv) * d], qkv[:, (hq + hkv) * d:]
            else:
                q, k, v = self._attention_block_proj(l, ops.rmsnorm(x, ln_in, eps))
            q3, k3, v3 = q.view(b, hq, d), k.view(b, hkv, d), v.view(b, hkv, d)
            if fused:  # RoPE, KV append and attention in one launch
                attn = decode_rope_attention(q3, k3, v3, kv[l, 0], kv[l, 1], self.cos_table,
                                             self.sin_table, positions.view(-1), slot_mapping,
                                             block_tables_tensor, context_lens,
                                             max_blocks_per_seq, self.scale)
            else:
                q_rot = torch.empty(b, hq, d, dtype=q.dtype, device=q.device)
                rope_kv_store(q3, k3, v3, kv[l, 0], kv[l, 1], self.cos_table, self.sin_table,
                              positions.view(-1), slot_mapping, query_out=q_rot)
                attn = ops.paged_attention_decode(q_rot, kv[l, 0], kv[l, 1],
                                                  block_tables_tensor, context_lens,
                                                  max_blocks_per_seq,
                                                  self.cache_manager.block_size, self.scale)
            w_o = self.weights[f"{p}.self_attn.o_proj.weight"]
            if gemms:  # o_proj + residual; RMSNorm + gate/up + SwiGLU; down_proj + residual
                decode_gemm(attn.view(b, hq * d), w_o, out=x, epilogue="add")
                act = rmsnorm_decode_gemm(x, self.weights[f"{p}.post_attention_layernorm.weight"],
                                          eps, self.w_gate_up[l], epilogue="swiglu")
                decode_gemm(act, self.weights[f"{p}.mlp.down_proj.weight"], out=x,
                            epilogue="add")
            else:
                x.addmm_(attn.view(b, hq * d), w_o.T)
                self._mlp(l, x)
        if gemms:
            return rmsnorm_decode_gemm(x, self.weights["model.norm.weight"], eps, self.lm_head)
        xf = ops.rmsnorm(x, self.weights["model.norm.weight"], eps)
        return torch.matmul(xf, self.lm_head.T)
