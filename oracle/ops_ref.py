"""CPU restatement of the six hot-path ops -- test infrastructure only.

All floating-point functions compute in fp32 (or the dtype of `acc`) on CPU
tensors and return fp32 results; callers compare the GPU's fp16 output
against them.  Integer/index functions are exact.
"""
from __future__ import annotations

import math

import numpy as np
import torch


def rmsnorm_ref(x: torch.Tensor, w: torch.Tensor, eps: float,
                acc: torch.dtype = torch.float32) -> torch.Tensor:
    """y = x * rsqrt(mean(x^2) + eps) * w over the last dim.

    Follows csrc/kernels/rmsnorm.cu:55-107 (fp32 sum of squares, one
    rsqrt, weight multiply in fp32) and the unfused formula of
    tests/test_ops.py:14-15.
    """
    xf = x.to(acc)
    var = (xf * xf).mean(dim=-1, keepdim=True)
    return xf * torch.rsqrt(var + eps) * w.to(acc)


def swiglu_ref(gate_up: torch.Tensor, acc: torch.dtype = torch.float32) -> torch.Tensor:
    """silu(g) * u with g, u the two halves of the last dim, every row.

    Follows csrc/kernels/swiglu.cu:6,16-26 (silu(x) = x / (1 + e^-x)); the
    reference's row guard (swiglu.cu:13) is a defect and is not reproduced.
    """
    x = gate_up.to(acc)
    inter = x.shape[-1] // 2
    g, u = x[..., :inter], x[..., inter:]
    return g / (1.0 + torch.exp(-g)) * u


def rope_tables(max_positions: int, head_dim: int, theta: float,
                acc: torch.dtype = torch.float32):
    """cos/sin tables [max_positions, head_dim/2], inv_freq = theta^(-2i/D).

    Follows engine/models/llama.py:47-57 (fp32 arange/outer/cos/sin).
    """
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=acc) / head_dim))
    t = torch.arange(max_positions, dtype=acc)
    freqs = torch.outer(t, inv_freq)
    return torch.cos(freqs), torch.sin(freqs)


def rope_ref(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
             positions: torch.Tensor, acc: torch.dtype = torch.float32) -> torch.Tensor:
    """Half-split rotation of x [B, S, H, D] at positions [B, S].

    For i < D/2: (x_i, x_{i+D/2}) -> (x_i c - x_{i+D/2} s, x_i s + x_{i+D/2} c)
    with c, s = table[pos, i].  Follows csrc/kernels/rope.cu:39-46,53-60.
    Returns the rotated copy (fp32); x is not modified.
    """
    xf = x.to(acc)
    half = xf.shape[-1] // 2
    pos = positions.reshape(xf.shape[0], xf.shape[1]).long()
    c = cos.to(acc)[pos].unsqueeze(2)  # [B, S, 1, D/2]
    s = sin.to(acc)[pos].unsqueeze(2)
    x0, x1 = xf[..., :half], xf[..., half:]
    return torch.cat([x0 * c - x1 * s, x0 * s + x1 * c], dim=-1)


def kv_store_ref(key: np.ndarray, value: np.ndarray, key_cache: np.ndarray,
                 value_cache: np.ndarray, slot_mapping: np.ndarray) -> None:
    """In-place scatter of key/value [N, H, D] rows into [NB, BS, H, D] pools.

    Follows csrc/kernels/paged_kv.cu:16-42: slot s -> (s // BS, s % BS);
    s < 0 is skipped (:18).  BS is taken from the cache (the reference
    hard-codes 16 at :22).  Slots past the pool are skipped as well.
    Bit-exact (a copy of the raw 16-bit values).
    """
    nb, bs = key_cache.shape[0], key_cache.shape[1]
    slots = np.asarray(slot_mapping, dtype=np.int64)
    ok = (slots >= 0) & (slots < nb * bs)
    idx = np.nonzero(ok)[0]
    s = slots[idx]
    key_cache[s // bs, s % bs] = key[idx]
    value_cache[s // bs, s % bs] = value[idx]


def gather_kv(cache: torch.Tensor, block_table_row, ctx: int) -> torch.Tensor:
    """Logical [ctx, H, D] view of one sequence from a [NB, BS, H, D] pool.

    Token t lives at cache[block_table_row[t // BS], t % BS]
    (csrc/kernels/flash_attn_paged.cu:71-85).
    """
    bs = cache.shape[1]
    t = torch.arange(ctx)
    blocks = torch.as_tensor(block_table_row, dtype=torch.long)[t // bs]
    return cache[blocks, t % bs]


def decode_attention_ref(query: torch.Tensor, key_cache: torch.Tensor,
                         value_cache: torch.Tensor, block_tables: torch.Tensor,
                         context_lens, scale: float,
                         acc: torch.dtype = torch.float32) -> torch.Tensor:
    """Paged one-token attention with GQA; returns [B, Hq, D] in `acc`.

    out[b, h] = sum_{t < ctx_b} softmax_t(scale * q[b,h] . k_t) v_t, with k_t,
    v_t gathered through block_tables and kv head h // (Hq / Hkv).  Follows
    csrc/kernels/flash_attn_paged.cu:40-141 (the online softmax there is an
    exact rewrite of this softmax).  Rows with ctx <= 0 are zeros (the
    reference leaves them unwritten, :40-42).
    """
    b, hq, d = query.shape
    hkv = key_cache.shape[2]
    grp = hq // hkv
    out = torch.zeros(b, hq, d, dtype=acc)
    for i in range(b):
        ctx = int(context_lens[i])
        if ctx <= 0:
            continue
        k = gather_kv(key_cache, block_tables[i], ctx).to(acc)  # [ctx, Hkv, D]
        v = gather_kv(value_cache, block_tables[i], ctx).to(acc)
        k = k.repeat_interleave(grp, dim=1)  # [ctx, Hq, D]
        v = v.repeat_interleave(grp, dim=1)
        q = query[i].to(acc)  # [Hq, D]
        s = torch.einsum("hd,thd->ht", q, k) * scale
        p = torch.softmax(s, dim=-1)
        out[i] = torch.einsum("ht,thd->hd", p, v)
    return out


def prefill_attention_ref(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                          scale: float, acc: torch.dtype = torch.float32) -> torch.Tensor:
    """Causal GQA attention on contiguous [B, S, H, D] tensors; returns [B, S, Hq, D].

    out[b, s, h] = sum_{t <= s} softmax_t(scale * q . k_t) v_t, kv head
    h // (Hq / Hkv).  Follows csrc/kernels/prefill_attention.cu:26-35 (GQA map),
    :167-169 (mask k > q) and :246-268 (normalisation by the row sum).
    """
    b, s, hq, d = query.shape
    hkv = key.shape[2]
    grp = hq // hkv
    q = query.to(acc).permute(0, 2, 1, 3)  # [B, Hq, S, D]
    k = key.to(acc).repeat_interleave(grp, dim=2).permute(0, 2, 1, 3)
    v = value.to(acc).repeat_interleave(grp, dim=2).permute(0, 2, 1, 3)
    sc = torch.matmul(q, k.transpose(-1, -2)) * scale  # [B, Hq, S, S]
    mask = torch.triu(torch.ones(s, s, dtype=torch.bool), diagonal=1)
    sc = sc.masked_fill(mask, float("-inf"))
    p = torch.softmax(sc, dim=-1)
    return torch.matmul(p, v).permute(0, 2, 1, 3).contiguous()


def scale_for(head_dim: int) -> float:
    """1 / sqrt(head_dim) (engine/models/llama.py:38)."""
    return 1.0 / math.sqrt(head_dim)


def prefill_paged_ref(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                      block_table_row, ctx: int, scale: float) -> torch.Tensor:
    """Chunked causal prefill of one sequence from the page pool: query
    [S, Hq, D] holds positions ctx - S .. ctx - 1; K/V of positions 0 .. ctx-1
    are gathered through the block table (gather_kv) and row i attends to
    keys 0 .. ctx - S + i.  Returns [S, Hq, D] fp32.  Causal attention of
    the whole sequence (prefill_attention_ref) restricted to its last S rows:
    a row depends on its own query and the keys up to its position only, so
    the earlier positions' queries are zeros here."""
    s, hq, d = query.shape
    k = gather_kv(key_cache, block_table_row, ctx)
    v = gather_kv(value_cache, block_table_row, ctx)
    q = torch.zeros(ctx, hq, d, dtype=query.dtype)
    q[ctx - s:] = query
    return prefill_attention_ref(q[None], k[None], v[None], scale)[0, ctx - s:]
