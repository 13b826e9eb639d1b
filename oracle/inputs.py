"""Seeded CPU generators for the hot-path workloads -- test infrastructure only.

Every input is drawn on the CPU with torch.Generator().manual_seed(seed) and
copied to the device by the caller, so the GPU path and the oracle see the
same values.  Defaults follow the benchmark configurations:
  cfg1 decode  B=1, ctx 512, 24/8 heads, pool 64 blocks, 32 used (seed 42)
  cfg2 decode  B=32, ctx ~ U[128, 4096], pool 1.25x the blocks used (seed 43)
  cfg3 prefill B=1, S=2048, 24/8 heads, RoPE theta 5e5 (seed 44)
  cfg4 decode  B=8, ctx 32768 (seed 45)
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

HEAD_DIM = 128
BLOCK = 16


@dataclass
class DecodeCase:
    query: torch.Tensor          # [B, Hq, D] fp16
    key_cache: torch.Tensor      # [NB, BS, Hkv, D] fp16
    value_cache: torch.Tensor    # [NB, BS, Hkv, D] fp16
    block_tables: torch.Tensor   # [B, max_blocks] int32
    context_lens: torch.Tensor   # [B] int32
    block_size: int
    scale: float

    @property
    def max_blocks(self) -> int:
        return self.block_tables.shape[1]

    def algorithmic_bytes(self) -> int:
        """K+V bytes read once each, q read and out written once, plus the
        block-table entries and context lengths actually used."""
        b, hq, d = self.query.shape
        hkv = self.key_cache.shape[2]
        ctx = [int(c) for c in self.context_lens]
        kv = sum(ctx) * hkv * d * 2 * 2
        qo = 2 * b * hq * d * 2
        tables = 4 * sum((c + self.block_size - 1) // self.block_size for c in ctx)
        return kv + qo + tables + 4 * b


def make_decode_case(seed: int, batch: int, context_lens, num_heads: int = 24,
                     num_kv_heads: int = 8, head_dim: int = HEAD_DIM,
                     block_size: int = BLOCK, spare: float = 0.25,
                     max_blocks: int | None = None, nan_pool: bool = True,
                     dtype=torch.float16) -> DecodeCase:
    """Decode workload with shuffled, non-contiguous block tables.

    The pool holds ceil((1 + spare) * blocks used) blocks; each sequence's
    table is a slice of one random permutation of the pool, zero-padded to
    `max_blocks`.  Unused pool blocks are NaN (nan_pool) so that any read of
    a block outside a sequence's table poisons the result.
    """
    g = torch.Generator().manual_seed(seed)
    ctx = [int(c) for c in context_lens]
    assert len(ctx) == batch
    need = [(c + block_size - 1) // block_size for c in ctx]
    used = sum(need)
    pool = max(1, math.ceil((1.0 + spare) * used))
    if max_blocks is None:
        max_blocks = max(1, max(need))
    perm = torch.randperm(pool, generator=g)
    tables = torch.zeros(batch, max_blocks, dtype=torch.int32)
    off = 0
    for i, n in enumerate(need):
        tables[i, :n] = perm[off:off + n].to(torch.int32)
        off += n
    q = torch.randn(batch, num_heads, head_dim, generator=g).to(dtype)
    shape = (pool, block_size, num_kv_heads, head_dim)
    fill = float("nan") if nan_pool else 0.0
    kc = torch.full(shape, fill, dtype=dtype)
    vc = torch.full(shape, fill, dtype=dtype)
    used_blocks = perm[:used]
    kc[used_blocks] = torch.randn(used, block_size, num_kv_heads, head_dim, generator=g).to(dtype)
    vc[used_blocks] = torch.randn(used, block_size, num_kv_heads, head_dim, generator=g).to(dtype)
    return DecodeCase(q, kc, vc, tables, torch.tensor(ctx, dtype=torch.int32), block_size,
                      1.0 / math.sqrt(head_dim))


def cfg1_decode() -> DecodeCase:
    """B=1, ctx 512, pool of 64 blocks with 32 used (a random 32 of 64)."""
    g = torch.Generator().manual_seed(42)
    hq, hkv, d, bs, pool, ctx = 24, 8, HEAD_DIM, BLOCK, 64, 512
    q = torch.randn(1, hq, d, generator=g).to(torch.float16)
    k = torch.randn(ctx, hkv, d, generator=g).to(torch.float16)
    v = torch.randn(ctx, hkv, d, generator=g).to(torch.float16)
    bt = torch.randperm(pool, generator=g)[: ctx // bs].to(torch.int32)
    kc = torch.full((pool, bs, hkv, d), float("nan"), dtype=torch.float16)
    vc = torch.full((pool, bs, hkv, d), float("nan"), dtype=torch.float16)
    kc[bt.long()] = k.view(ctx // bs, bs, hkv, d)
    vc[bt.long()] = v.view(ctx // bs, bs, hkv, d)
    return DecodeCase(q, kc, vc, bt.view(1, -1).contiguous(),
                      torch.tensor([ctx], dtype=torch.int32), bs, 1.0 / math.sqrt(d))


def cfg2_context_lens(seed: int = 43, batch: int = 32, lo: int = 128, hi: int = 4096):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (batch,), generator=g).tolist()


def cfg2_decode(seed: int = 43, batch: int = 32, nan_pool: bool = False) -> DecodeCase:
    """B=32, ctx ~ U[128, 4096], table width 256 (4096 / 16), 25% spare pool."""
    ctx = cfg2_context_lens(seed, batch)
    return make_decode_case(seed + 1000, batch, ctx, max_blocks=4096 // BLOCK,
                            nan_pool=nan_pool)


def cfg4_decode(seed: int = 45, batch: int = 8, ctx: int = 32768,
                nan_pool: bool = False) -> DecodeCase:
    """B=8, ctx 32768 per sequence, 2048 blocks per table."""
    return make_decode_case(seed, batch, [ctx] * batch, max_blocks=ctx // BLOCK,
                            spare=0.05, nan_pool=nan_pool)


@dataclass
class PrefillCase:
    query: torch.Tensor   # [B, S, Hq, D] fp16 (before RoPE)
    key: torch.Tensor     # [B, S, Hkv, D] fp16 (before RoPE)
    value: torch.Tensor   # [B, S, Hkv, D] fp16
    scale: float

    def algorithmic_flops(self) -> int:
        """2 FLOP/MAC x (QK^T + PV) over the causal (t <= s) pairs only."""
        b, s, hq, d = self.query.shape
        return 2 * d * hq * s * (s + 1) * b


def make_prefill_case(seed: int, batch: int, seq_len: int, num_heads: int = 24,
                      num_kv_heads: int = 8, head_dim: int = HEAD_DIM,
                      dtype=torch.float16) -> PrefillCase:
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, seq_len, num_heads, head_dim, generator=g).to(dtype)
    k = torch.randn(batch, seq_len, num_kv_heads, head_dim, generator=g).to(dtype)
    v = torch.randn(batch, seq_len, num_kv_heads, head_dim, generator=g).to(dtype)
    return PrefillCase(q, k, v, 1.0 / math.sqrt(head_dim))


def cfg3_prefill() -> PrefillCase:
    return make_prefill_case(44, 1, 2048)
