"""CPU: pin the oracle against independent formulations.

Each oracle function is checked against something that does not restate its
own formula: a torch library routine (SDPA, F.rms_norm, F.silu), a different
mathematical formulation (complex rotation for RoPE), scalar brute force on
tiny inputs, or an invariant a plausible bug would break (a wrong GQA map,
a transposed gather, a dropped mask, a swapped rotation sign).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.alloc_ref import (BlockAllocatorRef, argmax_rows_ref, decode_advance_ref,
                              prefill_slots_ref, slot_mapping_ref)
from oracle.inputs import cfg1_decode, make_decode_case, make_prefill_case
from oracle.ops_ref import (decode_attention_ref, gather_kv, kv_store_ref, prefill_paged_ref,
                            prefill_attention_ref, rmsnorm_ref, rope_ref, rope_tables,
                            swiglu_ref)


def gen(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------- decode
def test_decode_matches_sdpa_gqa():
    case = make_decode_case(1, 3, [40, 1, 77], num_heads=6, num_kv_heads=2, nan_pool=True)
    ref = decode_attention_ref(case.query, case.key_cache, case.value_cache,
                               case.block_tables, case.context_lens, case.scale,
                               acc=torch.float64)
    for b in range(3):
        ctx = int(case.context_lens[b])
        k = gather_kv(case.key_cache, case.block_tables[b], ctx).double()  # [ctx, Hkv, D]
        v = gather_kv(case.value_cache, case.block_tables[b], ctx).double()
        q = case.query[b].double().unsqueeze(1)                              # [Hq, 1, D]
        out = F.scaled_dot_product_attention(q, k.transpose(0, 1), v.transpose(0, 1),
                                             scale=case.scale, enable_gqa=True)
        assert torch.allclose(ref[b], out.squeeze(1), atol=1e-10)


def test_decode_scalar_brute_force():
    case = make_decode_case(2, 2, [5, 9], num_heads=4, num_kv_heads=2, head_dim=8,
                            block_size=4)
    ref = decode_attention_ref(case.query, case.key_cache, case.value_cache,
                               case.block_tables, case.context_lens, case.scale,
                               acc=torch.float64)
    hq, d = case.query.shape[1], case.query.shape[2]
    for b in range(2):
        ctx = int(case.context_lens[b])
        for h in range(hq):
            g = h // 2  # GQA: h // (Hq / Hkv)
            scores = []
            for t in range(ctx):
                blk = int(case.block_tables[b, t // 4])
                kt = case.key_cache[blk, t % 4, g].double()
                scores.append(sum(float(case.query[b, h, i]) * float(kt[i]) for i in range(d))
                              * case.scale)
            mx = max(scores)
            w = [math.exp(s - mx) for s in scores]
            tot = sum(w)
            for i in range(d):
                acc = sum(w[t] * float(case.value_cache[int(case.block_tables[b, t // 4]),
                                                        t % 4, g, i]) for t in range(ctx))
                assert abs(acc / tot - float(ref[b, h, i])) < 1e-9


def test_decode_invariants():
    case = cfg1_decode()
    ref = decode_attention_ref(case.query, case.key_cache, case.value_cache,
                               case.block_tables, case.context_lens, case.scale)
    assert not torch.isnan(ref).any()  # NaN-filled unused blocks never read
    # ctx = 1 returns v_0 of the right kv head
    one = decode_attention_ref(case.query, case.key_cache, case.value_cache,
                               case.block_tables, torch.tensor([1]), case.scale)
    v0 = case.value_cache[int(case.block_tables[0, 0]), 0].float()
    assert torch.equal(one[0, 5], v0[5 // 3])
    # ctx = 0 rows are zeros
    zero = decode_attention_ref(case.query, case.key_cache, case.value_cache,
                                case.block_tables, torch.tensor([0]), case.scale)
    assert torch.count_nonzero(zero) == 0


def test_decode_block_table_permutation_invariance():
    case = make_decode_case(3, 2, [50, 33], nan_pool=True)
    ref = decode_attention_ref(case.query, case.key_cache, case.value_cache,
                               case.block_tables, case.context_lens, case.scale)
    nb = case.key_cache.shape[0]
    perm = torch.randperm(nb, generator=gen(0))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(nb)
    ref2 = decode_attention_ref(case.query, case.key_cache[perm], case.value_cache[perm],
                                inv[case.block_tables.long()], case.context_lens, case.scale)
    assert torch.allclose(ref, ref2, atol=1e-6)


# --------------------------------------------------------------- prefill
@pytest.mark.parametrize("hq,hkv", [(6, 2), (4, 4)])
def test_prefill_matches_causal_sdpa(hq, hkv):
    case = make_prefill_case(4, 2, 37, hq, hkv)
    ref = prefill_attention_ref(case.query, case.key, case.value, case.scale, acc=torch.float64)
    q = case.query.double().transpose(1, 2)
    k = case.key.double().transpose(1, 2)
    v = case.value.double().transpose(1, 2)
    out = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=case.scale,
                                         enable_gqa=True).transpose(1, 2)
    assert torch.allclose(ref, out, atol=1e-10)


def test_prefill_scalar_brute_force_and_row0():
    case = make_prefill_case(5, 1, 6, 2, 1, head_dim=4)
    ref = prefill_attention_ref(case.query, case.key, case.value, case.scale, acc=torch.float64)
    for s in range(6):
        for h in range(2):
            sc = [sum(float(case.query[0, s, h, i]) * float(case.key[0, t, 0, i])
                      for i in range(4)) * case.scale for t in range(s + 1)]
            mx = max(sc)
            w = [math.exp(x - mx) for x in sc]
            for i in range(4):
                want = sum(w[t] * float(case.value[0, t, 0, i]) for t in range(s + 1)) / sum(w)
                assert abs(want - float(ref[0, s, h, i])) < 1e-9
    assert torch.equal(ref[0, 0, 1], case.value[0, 0, 0].double())  # row 0 = v_0


# ---------------------------------------------------------------- RMSNorm
def test_rmsnorm_matches_library_and_brute_force():
    x = torch.randn(5, 64, generator=gen(6))
    w = torch.randn(64, generator=gen(7))
    ref = rmsnorm_ref(x, w, 1e-5, acc=torch.float64)
    lib = F.rms_norm(x.double(), (64,), w.double(), eps=1e-5)
    assert torch.allclose(ref, lib, atol=1e-12)
    row = [float(v) for v in x[2]]
    inv = 1.0 / math.sqrt(sum(v * v for v in row) / 64 + 1e-5)
    assert abs(float(ref[2, 7]) - row[7] * inv * float(w[7])) < 1e-12


# ------------------------------------------------------------------- RoPE
def test_rope_tables_formula():
    cos, sin = rope_tables(9, 8, 500000.0, acc=torch.float64)
    for p in (0, 3, 8):
        for i in range(4):
            ang = p * 500000.0 ** (-2 * i / 8)
            assert abs(float(cos[p, i]) - math.cos(ang)) < 1e-12
            assert abs(float(sin[p, i]) - math.sin(ang)) < 1e-12


def test_rope_equals_complex_rotation():
    cos, sin = rope_tables(64, 16, 500000.0, acc=torch.float64)
    x = torch.randn(2, 5, 3, 16, generator=gen(8), dtype=torch.float64)
    pos = torch.randint(0, 64, (2, 5), generator=gen(9))
    out = rope_ref(x, cos, sin, pos, acc=torch.float64)
    # (x_i + j x_{i+D/2}) * e^{j theta}, as a complex product
    z = torch.complex(x[..., :8], x[..., 8:])
    ang = torch.atan2(sin[pos], cos[pos]).unsqueeze(2)
    zr = z * torch.exp(torch.complex(torch.zeros_like(ang), ang))
    assert torch.allclose(out, torch.cat([zr.real, zr.imag], dim=-1), atol=1e-12)


def test_rope_invariants():
    cos, sin = rope_tables(32, 16, 500000.0, acc=torch.float64)
    x = torch.randn(1, 4, 2, 16, generator=gen(10), dtype=torch.float64)
    zero = rope_ref(x, cos, sin, torch.zeros(1, 4, dtype=torch.long), acc=torch.float64)
    assert torch.allclose(zero, x, atol=0)  # position 0 is the identity
    out = rope_ref(x, cos, sin, torch.tensor([[1, 5, 9, 31]]), acc=torch.float64)
    pair_norm = lambda t: t[..., :8] ** 2 + t[..., 8:] ** 2
    assert torch.allclose(pair_norm(out), pair_norm(x), atol=1e-12)
    # rotating by p then by q equals rotating by p + q
    a = rope_ref(rope_ref(x, cos, sin, torch.full((1, 4), 3), acc=torch.float64), cos, sin,
                 torch.full((1, 4), 4), acc=torch.float64)
    b = rope_ref(x, cos, sin, torch.full((1, 4), 7), acc=torch.float64)
    assert torch.allclose(a, b, atol=1e-12)


# ----------------------------------------------------------------- SwiGLU
def test_swiglu_matches_library_and_brute_force():
    x = torch.randn(4, 2 * 24, generator=gen(11))
    ref = swiglu_ref(x, acc=torch.float64)
    lib = F.silu(x[:, :24].double()) * x[:, 24:].double()
    assert torch.allclose(ref, lib, atol=1e-12)
    g, u = float(x[3, 5]), float(x[3, 29])
    assert abs(float(ref[3, 5]) - g / (1 + math.exp(-g)) * u) < 1e-12


# --------------------------------------------------------------- KV store
def test_kv_store_matches_scalar_loop():
    rng = np.random.default_rng(0)
    n, h, d, nb, bs = 20, 2, 8, 6, 4
    key = rng.standard_normal((n, h, d)).astype(np.float16)
    val = rng.standard_normal((n, h, d)).astype(np.float16)
    slots = rng.permutation(nb * bs)[:n].astype(np.int32)
    slots[[1, 7]] = -1
    slots[3] = nb * bs + 2
    kc = rng.standard_normal((nb, bs, h, d)).astype(np.float16)
    vc = rng.standard_normal((nb, bs, h, d)).astype(np.float16)
    kc2, vc2 = kc.copy(), vc.copy()
    kv_store_ref(key, val, kc, vc, slots)
    for i in range(n):
        s = int(slots[i])
        if s < 0 or s >= nb * bs:
            continue
        for hh in range(h):
            for dd in range(d):
                kc2[s // bs, s % bs, hh, dd] = key[i, hh, dd]
                vc2[s // bs, s % bs, hh, dd] = val[i, hh, dd]
    assert np.array_equal(kc.view(np.uint16), kc2.view(np.uint16))
    assert np.array_equal(vc.view(np.uint16), vc2.view(np.uint16))


# ------------------------------------------------ block allocator / slots
def test_block_allocator_fifo_and_padding():
    a = BlockAllocatorRef(10, 4)
    a.allocate_sequence(7, 9)     # ceil(9/4) = 3 blocks: 0, 1, 2
    a.allocate_sequence(3, 4)     # 1 block: 3
    assert a.tables == {7: [0, 1, 2], 3: [3]}
    a.append_token(3, 4)          # len 4 % 4 == 0 -> new block 4
    a.append_token(3, 5)          # no new block
    assert a.tables[3] == [3, 4]
    bt = a.block_table([3, 7], 4)
    assert bt.tolist() == [[3, 4, 0, 0], [0, 1, 2, 0]]
    with pytest.raises(RuntimeError):
        a.allocate_sequence(9, 100)


def test_slot_rules_brute_force():
    a = BlockAllocatorRef(16, 4)
    a.allocate_sequence(0, 10)
    a.allocate_sequence(1, 3)
    sm = slot_mapping_ref(a.tables, [0, 1], [10, 3], 4)
    assert sm.tolist() == [a.tables[0][2] * 4 + 1, a.tables[1][0] * 4 + 2]
    ps = prefill_slots_ref(a.tables, [0, 1], 3, 4).reshape(2, 3)
    for i, s in enumerate([0, 1]):
        for p in range(3):
            assert ps[i, p] == a.tables[s][p // 4] * 4 + p % 4


def test_decode_advance_follows_the_allocator_slot_rule():
    """One advance = the allocator's slot of the next position (hand-built
    tables), -1 once the position leaves the table width; positions and
    context lengths move by exactly one."""
    a = BlockAllocatorRef(16, 4)
    a.allocate_sequence(0, 10)   # blocks 0, 1, 2
    a.allocate_sequence(1, 3)    # block 3
    table = a.block_table([0, 1], 3)
    pos, ctx = np.array([9, 2], np.int32), np.array([10, 3], np.int32)
    p2, c2, sl = decode_advance_ref(table, pos, ctx, 4)
    assert p2.tolist() == [10, 3] and c2.tolist() == [11, 4]
    assert sl.tolist() == [a.tables[0][2] * 4 + 2, a.tables[1][0] * 4 + 3]
    # sequence 1 moves into its (zero-padded) second table entry, sequence 0 past the width
    p3, c3, sl3 = decode_advance_ref(table, [11, 3], [12, 4], 4)
    assert sl3.tolist() == [-1, 0 * 4 + 0]
    # agrees with slot_mapping_ref wherever the table has the block
    for step in range(6):
        q = np.array([2 + step, 1 + step], np.int32)
        _, cn, s_ = decode_advance_ref(table, q, q + 1, 4)
        want = slot_mapping_ref(a.tables, [0, 1], cn, 4) if cn[1] <= 4 else None
        if want is not None:
            assert s_.tolist() == want.tolist()


def test_argmax_rows_ref_tie_and_nan_rules():
    x = np.array([[1.0, 3.0, 3.0, -2.0],     # first of equal maxima
                  [-np.inf, -np.inf, -5.0, -5.0],
                  [0.0, np.nan, 7.0, np.nan],  # NaN above every number, first NaN
                  [2.0, 2.0, 2.0, 2.0],
                  [-1.0, -0.0, 0.0, -2.0]], np.float32)  # -0 equals +0: the first wins
    got = argmax_rows_ref(x)
    assert got.tolist() == [1, 2, 1, 0, 1]
    assert got.tolist() == torch.argmax(torch.from_numpy(x), dim=-1).tolist()


def test_prefill_paged_ref_is_the_tail_of_the_full_prefill():
    """The chunked restatement equals the last rows of the whole-sequence
    causal prefill whatever the earlier rows' queries are (causality), on a
    shuffled page pool, and with no prefix it is the whole prefill."""
    g = torch.Generator().manual_seed(9)
    bs, nb, hq, hkv, d = 4, 12, 4, 2, 16
    kc = torch.randn(nb, bs, hkv, d, generator=g)
    vc = torch.randn(nb, bs, hkv, d, generator=g)
    table = torch.randperm(nb, generator=g)[:6].tolist()
    ctx, s = 19, 5
    q_all = torch.randn(ctx, hq, d, generator=g)
    k = gather_kv(kc, table, ctx)
    v = gather_kv(vc, table, ctx)
    full = prefill_attention_ref(q_all[None], k[None], v[None], 0.3)[0]
    got = prefill_paged_ref(q_all[ctx - s:], kc, vc, table, ctx, 0.3)
    assert torch.allclose(got, full[ctx - s:], atol=1e-6)
    whole = prefill_paged_ref(q_all, kc, vc, table, ctx, 0.3)
    assert torch.allclose(whole, full, atol=1e-6)
