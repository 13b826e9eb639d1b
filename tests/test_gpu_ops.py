"""GPU parity of RMSNorm, SwiGLU, RoPE, the paged KV store, causal prefill
attention, the decode-sized GEMMs and the device-side decode-loop ops against
the CPU oracle.

Bars: KV store, argmax and decode-step preparation bit-exact; RMSNorm/SwiGLU/RoPE/prefill max-abs <= 1e-2 vs the
fp32 oracle (reference tolerance class: tests/test_ops.py:35,
tests/test_rope.py:56-57); RMSNorm/SwiGLU/RoPE additionally within one fp16
ulp-scale relative bound.
"""
import numpy as np
import pytest
import torch

import my_cuda_engine_cpp as ops
from oracle.alloc_ref import BlockAllocatorRef, prefill_slots_ref
from oracle.inputs import cfg3_prefill, make_prefill_case
from oracle.ops_ref import (kv_store_ref, prefill_attention_ref, prefill_paged_ref, rmsnorm_ref,
                            rope_ref, rope_tables, swiglu_ref)

TOL = 1e-2
pytestmark = pytest.mark.gpu


def gen(seed):
    return torch.Generator().manual_seed(seed)


def rel_close(out, ref, rel=2e-3, abs_=1e-3):
    """|out - ref| <= abs_ + rel * |ref|: fp16 rounding of an exact result."""
    d = (out.float() - ref).abs()
    bound = abs_ + rel * ref.abs()
    return bool((d <= bound).all()), d.max().item()


# ------------------------------------------------------------------ RMSNorm
@pytest.mark.parametrize("rows,hidden", [(8, 3072), (4096, 3072), (3, 4096), (5, 8192),
                                         (7, 1000), (2, 127), (4, 8200), (1, 8), (65, 512)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rmsnorm(dev, rows, hidden, dtype):
    x = torch.randn(rows, hidden, generator=gen(rows * 7 + hidden)).to(dtype)
    w = (1.0 + 0.5 * torch.randn(hidden, generator=gen(hidden))).to(dtype)
    out = ops.rmsnorm(x.to(dev), w.to(dev), 1e-5).cpu()
    ref = rmsnorm_ref(x, w, 1e-5)
    ok, err = rel_close(out, ref, rel=4e-3 if dtype == torch.float16 else 1.6e-2)
    assert ok, err
    if dtype == torch.float16:
        assert (out.float() - ref).abs().max().item() <= TOL


def test_rmsnorm_3d_input(dev):
    x = torch.randn(2, 5, 3072, generator=gen(1)).half()
    w = torch.ones(3072).half()
    out = ops.rmsnorm(x.to(dev), w.to(dev), 1e-5).cpu()
    assert out.shape == x.shape
    assert (out.float() - rmsnorm_ref(x, w, 1e-5)).abs().max() <= TOL


# ------------------------------------------------------------------- SwiGLU
@pytest.mark.parametrize("shape", [(8, 16384), (4096, 16384), (1, 16), (3, 14), (2, 7, 64),
                                   (5, 1000)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_swiglu_all_rows(dev, shape, dtype):
    x = (2.0 * torch.randn(*shape, generator=gen(sum(shape)))).to(dtype)
    out = ops.swiglu(x.to(dev)).cpu()
    ref = swiglu_ref(x)
    assert out.shape == ref.shape
    ok, err = rel_close(out, ref, rel=4e-3 if dtype == torch.float16 else 1.6e-2)
    assert ok, err


# --------------------------------------------------------------------- RoPE
@pytest.mark.parametrize("b,s,hq,hkv", [(1, 2048, 24, 8), (8, 1, 24, 8), (16, 1, 32, 8),
                                        (2, 37, 6, 2)])
def test_rope_matches_oracle(dev, b, s, hq, hkv):
    cos, sin = rope_tables(4096, 128, 500000.0)
    q = torch.randn(b, s, hq, 128, generator=gen(b + s)).half()
    k = torch.randn(b, s, hkv, 128, generator=gen(b * s + 1)).half()
    pos = torch.randint(0, 4096, (b, s), generator=gen(3), dtype=torch.int32)
    if s > 1:
        pos = torch.arange(s, dtype=torch.int32).repeat(b, 1)
    qd, kd = q.to(dev), k.to(dev)
    ops.rope_inplace(qd, kd, cos.to(dev), sin.to(dev), pos.to(dev))
    for got, x in ((qd.cpu(), q), (kd.cpu(), k)):
        ref = rope_ref(x, cos, sin, pos)
        ok, err = rel_close(got, ref, rel=4e-3, abs_=2e-3)
        assert ok, err


def test_rope_strided_views_and_no_key(dev):
    """Q/K as views into a fused [B, S, (Hq + 2 Hkv) * D] projection."""
    b, s, hq, hkv, d = 2, 9, 24, 8, 128
    cos, sin = rope_tables(64, d, 500000.0)
    fused = torch.randn(b, s, (hq + 2 * hkv) * d, generator=gen(4)).half()
    fd = fused.to(dev)
    qv = fd[..., : hq * d].view(b, s, hq, d)
    kv = fd[..., hq * d:(hq + hkv) * d].view(b, s, hkv, d)
    pos = torch.arange(s, dtype=torch.int32).repeat(b, 1) + 5
    ops.rope_inplace(qv, kv, cos.to(dev), sin.to(dev), pos.to(dev))
    got = fd.cpu()
    q_ref = rope_ref(fused[..., : hq * d].view(b, s, hq, d), cos, sin, pos)
    k_ref = rope_ref(fused[..., hq * d:(hq + hkv) * d].view(b, s, hkv, d), cos, sin, pos)
    assert rel_close(got[..., : hq * d].view(b, s, hq, d), q_ref, 4e-3, 2e-3)[0]
    assert rel_close(got[..., hq * d:(hq + hkv) * d].view(b, s, hkv, d), k_ref, 4e-3, 2e-3)[0]
    assert torch.equal(got[..., (hq + hkv) * d:], fused[..., (hq + hkv) * d:])  # V untouched
    q2 = torch.randn(1, 3, 4, d, generator=gen(5)).half()
    q2d = q2.to(dev)
    ops.rope_inplace(q2d, None, cos.to(dev), sin.to(dev), torch.tensor([[0, 1, 2]], dtype=torch.int32, device=dev))
    assert rel_close(q2d.cpu(), rope_ref(q2, cos, sin, torch.tensor([[0, 1, 2]])), 4e-3, 2e-3)[0]


def test_rope_out_of_table_positions_untouched(dev):
    cos, sin = rope_tables(16, 128, 500000.0)
    q = torch.randn(1, 4, 2, 128, generator=gen(6)).half()
    k = torch.randn(1, 4, 1, 128, generator=gen(7)).half()
    pos = torch.tensor([[3, 16, -1, 15]], dtype=torch.int32)
    qd, kd = q.to(dev), k.to(dev)
    ops.rope_inplace(qd, kd, cos.to(dev), sin.to(dev), pos.to(dev))
    assert torch.equal(qd.cpu()[:, 1:3], q[:, 1:3]) and torch.equal(kd.cpu()[:, 1:3], k[:, 1:3])


# ----------------------------------------------------------------- KV store
@pytest.mark.parametrize("bs", [16, 8, 32])
def test_kv_store_bit_exact(dev, bs):
    n, hkv, d, nb = 300, 8, 128, 64
    key = torch.randn(n, hkv, d, generator=gen(8)).half()
    val = torch.randn(n, hkv, d, generator=gen(9)).half()
    slots = torch.randperm(nb * bs, generator=gen(10))[:n].to(torch.int32)
    slots[::7] = -1
    slots[5] = nb * bs + 3  # past the pool: skipped
    kc = torch.randn(nb, bs, hkv, d, generator=gen(11)).half()
    vc = torch.randn(nb, bs, hkv, d, generator=gen(12)).half()
    kcd, vcd = kc.to(dev), vc.to(dev)
    ops.paged_kv_store(key.to(dev), val.to(dev), kcd, vcd, slots.to(dev))
    kr, vr = kc.numpy().copy(), vc.numpy().copy()
    kv_store_ref(key.numpy(), val.numpy(), kr, vr, slots.numpy())
    assert torch.equal(kcd.cpu(), torch.from_numpy(kr))
    assert torch.equal(vcd.cpu(), torch.from_numpy(vr))


def test_kv_store_strided_token_views(dev):
    """k[:, p] of a [B, S, Hkv, D] tensor, as the reference's prefill driver passes
    (benchmarks/benchmark_engine.py:71-73); all S positions in one launch too."""
    b, s, hkv, d, bs = 3, 20, 8, 128, 16
    k = torch.randn(b, s, hkv, d, generator=gen(13)).half()
    v = torch.randn(b, s, hkv, d, generator=gen(14)).half()
    alloc = BlockAllocatorRef(16, bs)
    for i in range(b):
        alloc.allocate_sequence(i, s)
    slots = torch.from_numpy(prefill_slots_ref(alloc.tables, list(range(b)), s, bs))
    kc = torch.zeros(16, bs, hkv, d).half()
    vc = torch.zeros(16, bs, hkv, d).half()
    kcd, vcd = kc.clone().to(dev), vc.clone().to(dev)
    kd, vd = k.to(dev), v.to(dev)
    sl = slots.view(b, s)
    for p in range(s):  # per-position views (token stride s * hkv * d)
        ops.paged_kv_store(kd[:, p], vd[:, p], kcd, vcd, sl[:, p].contiguous().to(dev))
    kcd2, vcd2 = kc.clone().to(dev), vc.clone().to(dev)
    ops.paged_kv_store(kd.view(b * s, hkv, d), vd.view(b * s, hkv, d), kcd2, vcd2, slots.to(dev))
    kr, vr = kc.numpy().copy(), vc.numpy().copy()
    kv_store_ref(k.reshape(b * s, hkv, d).numpy(), v.reshape(b * s, hkv, d).numpy(), kr, vr,
                 slots.numpy())
    for got in (kcd.cpu(), kcd2.cpu()):
        assert torch.equal(got, torch.from_numpy(kr))
    for got in (vcd.cpu(), vcd2.cpu()):
        assert torch.equal(got, torch.from_numpy(vr))


def test_rope_and_kv_store_kernels_agree_across_layouts(dev):
    """16-byte aligned head_dim-128 rows take the workgroup-per-token kernels;
    the same values in rows offset by 8 bytes take the generic vector
    kernels: bit-identical results (same rotation arithmetic), and head_dim
    64 (generic kernels) bit-exact / within the bar against the oracle."""
    n, hq, hkv = 37, 6, 2
    cos, sin = rope_tables(128, 128, 500000.0)
    g = gen(77)
    q = torch.randn(n, 1, hq, 128, generator=g).half()
    k = torch.randn(n, 1, hkv, 128, generator=g).half()
    pos = torch.randint(0, 128, (n, 1), generator=g, dtype=torch.int32).to(dev)
    outs = []
    for shift in (0, 4):  # elements: 0 -> 16-byte aligned rows, 4 -> 8-byte aligned
        qb = torch.zeros(n * hq * 128 + 8, dtype=torch.float16, device=dev)
        kb = torch.zeros(n * hkv * 128 + 8, dtype=torch.float16, device=dev)
        qv = qb[shift:shift + n * hq * 128].view(n, 1, hq, 128)
        kv = kb[shift:shift + n * hkv * 128].view(n, 1, hkv, 128)
        qv.copy_(q.to(dev))
        kv.copy_(k.to(dev))
        ops.rope_inplace(qv, kv, cos.to(dev), sin.to(dev), pos)
        outs.append((qv.cpu(), kv.cpu()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    # kv store: aligned d128 rows vs 16-byte aligned head_dim 64 (generic kernel)
    for d in (128, 64):
        key = torch.randn(n, hkv, d, generator=g).half()
        val = torch.randn(n, hkv, d, generator=g).half()
        slots = torch.randperm(40 * 16, generator=g)[:n].to(torch.int32)
        slots[3] = -1
        kc = torch.zeros(40, 16, hkv, d).half()
        vc = torch.zeros(40, 16, hkv, d).half()
        kcd, vcd = kc.to(dev), vc.to(dev)
        ops.paged_kv_store(key.to(dev), val.to(dev), kcd, vcd, slots.to(dev))
        kr, vr = kc.numpy().copy(), vc.numpy().copy()
        kv_store_ref(key.numpy(), val.numpy(), kr, vr, slots.numpy())
        assert torch.equal(kcd.cpu(), torch.from_numpy(kr)) and torch.equal(vcd.cpu(), torch.from_numpy(vr))
    cos64, sin64 = rope_tables(128, 64, 500000.0)
    q64 = torch.randn(2, 5, 4, 64, generator=g).half()
    p64 = torch.arange(5, dtype=torch.int32).repeat(2, 1)
    q64d = q64.to(dev)
    ops.rope_inplace(q64d, None, cos64.to(dev), sin64.to(dev), p64.to(dev))
    assert rel_close(q64d.cpu(), rope_ref(q64, cos64, sin64, p64), 4e-3, 2e-3)[0]


# ------------------------------------------------------------ causal prefill
@pytest.mark.parametrize("s", [1, 2, 17, 64, 127, 128, 129, 300, 512, 1000])
@pytest.mark.parametrize("hq,hkv", [(24, 8), (4, 4), (6, 2)])
def test_prefill_matches_oracle(dev, s, hq, hkv):
    case = make_prefill_case(20 + s, 2 if s <= 512 else 1, s, hq, hkv)
    out = ops.prefill_attention(case.query.to(dev), case.key.to(dev), case.value.to(dev),
                                case.scale).cpu()
    ref = prefill_attention_ref(case.query, case.key, case.value, case.scale)
    assert not torch.isnan(out).any()
    err = (out.float() - ref).abs().max().item()
    assert err <= TOL, err


@pytest.mark.parametrize("b,s,hq,hkv", [(1, 300, 24, 8), (2, 129, 6, 2), (1, 1, 4, 4),
                                         (8, 512, 24, 8)])
def test_prefill_bf16_matches_oracle(dev, b, s, hq, hkv):
    """bf16 Q/K/V (bf16 MFMA, exact Q, scores scaled in fp32, P as bf16) on
    both kernel shapes (the last case is a large grid)."""
    case = make_prefill_case(90 + s, b, s, hq, hkv, dtype=torch.bfloat16)
    out = ops.prefill_attention(case.query.to(dev), case.key.to(dev), case.value.to(dev),
                                case.scale).cpu()
    assert out.dtype == torch.bfloat16 and not torch.isnan(out).any()
    ref = prefill_attention_ref(case.query, case.key, case.value, case.scale)
    err = (out.float() - ref).abs().max().item()
    assert err <= TOL, err


@pytest.mark.parametrize("b,s", [(8, 512), (6, 700), (64, 16), (128, 5), (48, 43)])
def test_prefill_large_grid_matches_oracle(dev, b, s):
    """Grids of at least two workgroups per CU take the kernel without the
    in-workgroup key split (the small cases above take the split one),
    including many short prompts in one call (items of one sequence's
    few rows, partial last items)."""
    case = make_prefill_case(60 + s + b, b, s)
    out = ops.prefill_attention(case.query.to(dev), case.key.to(dev), case.value.to(dev),
                                case.scale).cpu()
    ref = prefill_attention_ref(case.query, case.key, case.value, case.scale)
    assert not torch.isnan(out).any()
    err = (out.float() - ref).abs().max().item()
    assert err <= TOL, err


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_small_and_full_grid_layouts_agree(dev, dtype):
    """The two two-stream launches compute each row identically: a causal
    row depends only on the keys up to its position, so the first 1536
    positions of an S = 1792 call (336 items of 128 rows: 8-wave workgroups)
    equal, bit for bit, an S = 1536 call on that prefix (288 items: the
    64-row, 4-wave launch of small grids).  The long call is also checked
    against the oracle."""
    case = make_prefill_case(77, 1, 1792, dtype=dtype)
    q, k, v = (t.to(dev) for t in (case.query, case.key, case.value))
    full = ops.prefill_attention(q, k, v, case.scale)
    pre = ops.prefill_attention(q[:, :1536].contiguous(), k[:, :1536].contiguous(),
                                v[:, :1536].contiguous(), case.scale)
    torch.cuda.synchronize()
    assert torch.equal(full[:, :1536].view(torch.int16), pre.view(torch.int16))
    ref = prefill_attention_ref(case.query, case.key, case.value, case.scale)
    err = (full.cpu().float() - ref).abs().max().item()
    assert err <= TOL, err


def test_prefill_first_row_is_v0(dev):
    """Row 0 attends to key 0 only, so its output is v_0 up to the rounding of
    p (exactly 1 when the running max is that score) and of the fp16 store."""
    case = make_prefill_case(30, 1, 200)
    out = ops.prefill_attention(case.query.to(dev), case.key.to(dev), case.value.to(dev),
                                case.scale).cpu()
    v0 = case.value[0, 0].repeat_interleave(3, dim=0).float()
    assert (out[0, 0].float() - v0).abs().max().item() <= 2e-3 * (1 + v0.abs().max().item())


@pytest.mark.parametrize("n_tok,hq,hkv,strided", [(8, 24, 8, True), (74, 24, 8, False),
                                                   (5, 6, 2, True)])
def test_rope_kv_store_equals_separate_ops(dev, n_tok, hq, hkv, strided):
    """The engine's fused RoPE + paged store gives the same bits as rope_inplace
    followed by paged_kv_store, and both match the oracle: strided q/k/v views
    of one fused projection row (rotated q written to a separate contiguous
    query_out), an out-of-table position (left unrotated) and invalid slots
    (-1, past the pool: skipped)."""
    from mycustomcudaengine_amd.ops import rope_kv_store
    d, nb, bs = 128, 12, 16
    g = gen(70 + n_tok)
    if strided:
        qkv = torch.randn(n_tok, (hq + 2 * hkv) * d, generator=g).half()
        q0 = qkv[:, : hq * d].view(n_tok, hq, d)
        k0 = qkv[:, hq * d:(hq + hkv) * d].view(n_tok, hkv, d)
        v0 = qkv[:, (hq + hkv) * d:].view(n_tok, hkv, d)
    else:
        q0 = torch.randn(n_tok, hq, d, generator=g).half()
        k0 = torch.randn(n_tok, hkv, d, generator=g).half()
        v0 = torch.randn(n_tok, hkv, d, generator=g).half()
    cos, sin = rope_tables(64, d, 500000.0)
    pos = torch.randint(0, 64, (n_tok,), generator=g, dtype=torch.int32)
    pos[1] = 64  # outside the table
    slots = torch.randperm(nb * bs, generator=g)[:n_tok].to(torch.int32)
    slots[0] = -1
    slots[-1] = nb * bs + 3
    caches = []
    for fused in (True, False):
        base = qkv.clone().to(dev) if strided else None
        if strided:
            q = base[:, : hq * d].view(n_tok, hq, d)
            k = base[:, hq * d:(hq + hkv) * d].view(n_tok, hkv, d)
            v = base[:, (hq + hkv) * d:].view(n_tok, hkv, d)
        else:
            q, k, v = q0.clone().to(dev), k0.clone().to(dev), v0.clone().to(dev)
        kc = torch.full((nb, bs, hkv, d), 7.0, dtype=torch.float16, device=dev)
        vc = torch.full_like(kc, -3.0)
        if fused:
            q_out = torch.empty(n_tok, hq, d, dtype=torch.float16, device=dev) if strided else None
            q_before = q.clone()
            rope_kv_store(q, k, v, kc, vc, cos.to(dev), sin.to(dev), pos.to(dev), slots.to(dev),
                          query_out=q_out)
            if strided:  # rotated q went to q_out; the strided view is untouched
                assert torch.equal(q, q_before)
                q = q_out
        else:
            ops.rope_inplace(q.view(n_tok, 1, hq, d), k.view(n_tok, 1, hkv, d), cos.to(dev),
                             sin.to(dev), pos.view(n_tok, 1).to(dev))
            ops.paged_kv_store(k, v, kc, vc, slots.to(dev))
        caches.append((q.cpu(), k.cpu(), kc.cpu(), vc.cpu()))
    for a, b in zip(*caches):
        assert torch.equal(a, b)
    inside = torch.arange(n_tok) != 1  # the oracle's tables end at position 63
    q_ref = rope_ref(q0[inside].view(-1, 1, hq, d), cos, sin,
                     pos[inside].view(-1, 1)).view(-1, hq, d)
    assert rel_close(caches[0][0][inside], q_ref, 4e-3, 2e-3)[0]
    assert torch.equal(caches[0][0][1], q0[1])  # out-of-table position untouched
    kr = torch.full((nb, bs, hkv, d), 7.0, dtype=torch.float16).numpy()
    vr = torch.full((nb, bs, hkv, d), -3.0, dtype=torch.float16).numpy()
    kv_store_ref(caches[0][1].numpy(), v0.numpy(), kr, vr, slots.numpy())
    assert torch.equal(caches[0][2], torch.from_numpy(kr))
    assert torch.equal(caches[0][3], torch.from_numpy(vr))


def test_cfg3_rope_kvstore_prefill_pipeline(dev):
    """cfg3: RoPE (theta 5e5, positions 0..2047) in place, all 2048 K/V rows
    into 16-token pages of a permuted table (bit-exact), then causal attention."""
    case = cfg3_prefill()
    b, s, hq, d = case.query.shape
    hkv = case.key.shape[2]
    cos, sin = rope_tables(4096, d, 500000.0)
    pos = torch.arange(s, dtype=torch.int32).view(1, s)
    q, k, v = case.query.to(dev), case.key.to(dev), case.value.to(dev)
    ops.rope_inplace(q, k, cos.to(dev), sin.to(dev), pos.to(dev))
    q_ref = rope_ref(case.query, cos, sin, pos)
    k_ref = rope_ref(case.key, cos, sin, pos)
    assert rel_close(q.cpu(), q_ref, 4e-3, 2e-3)[0] and rel_close(k.cpu(), k_ref, 4e-3, 2e-3)[0]
    nb = 160
    table = torch.randperm(nb, generator=gen(44))[: s // 16]
    slots = (table.repeat_interleave(16) * 16 + torch.arange(s) % 16).to(torch.int32)
    kc = torch.zeros(nb, 16, hkv, d, dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    ops.paged_kv_store(k[0], v[0], kc, vc, slots.to(dev))
    kr = torch.zeros(nb, 16, hkv, d, dtype=torch.float16).numpy()
    vr = kr.copy()
    kv_store_ref(k[0].cpu().numpy(), v[0].cpu().numpy(), kr, vr, slots.numpy())
    assert torch.equal(kc.cpu(), torch.from_numpy(kr)) and torch.equal(vc.cpu(), torch.from_numpy(vr))
    out = ops.prefill_attention(q, k, v, case.scale).cpu()
    ref = prefill_attention_ref(q.cpu(), k.cpu(), v.cpu(), case.scale)
    err = (out.float() - ref).abs().max().item()
    assert err <= TOL, err


# ------------------------------------------------------- decode-sized GEMM
GEMM_SHAPES = [(5120, 3072, "store"), (3072, 3072, "add"), (8192, 3072, "swiglu"),
               (3072, 8192, "add"), (1024, 2048, "store"), (512, 4096, "swiglu")]


# k = 8192 is taken for m <= 8 only (128 KB of staged x); m = 16 there is
# refused with MCE_ERR_UNSUPPORTED (tests/test_abi.py)
@pytest.mark.parametrize("m,n,k,epi", [(m, *shape) for m in (1, 5, 8, 16) for shape in GEMM_SHAPES
                                       if not (shape[1] == 8192 and m > 8)])
def test_decode_gemm_matches_fp32(dev, m, n, k, epi):
    """x . W^T for the decode step's projection shapes with the fused
    epilogues, against fp32 torch on the same fp16 inputs: plain store,
    in-place residual add (o_proj / down_proj), SwiGLU over the fused
    [gate; up] weight (gate_up + SwiGLU).  x rows are strided (a view into a
    wider buffer) as the engine passes them."""
    from mycustomcudaengine_amd.ops import decode_gemm
    g = gen(80 + m + n // 512)
    rows = 2 * n if epi == "swiglu" else n
    xbuf = torch.randn(m, k + 64, generator=g).half()
    x = xbuf[:, 32:32 + k]
    w = (torch.randn(rows, k, generator=g) * 0.02).half()
    acc = x.float() @ w.float().T
    if epi == "swiglu":
        gt, up = acc[:, :n], acc[:, n:]
        ref = gt * torch.sigmoid(gt) * up
    elif epi == "add":
        res = torch.randn(m, n, generator=g).half()
        ref = res.float() + acc
    else:
        ref = acc
    xd = xbuf.to(dev)[:, 32:32 + k]
    if epi == "add":
        out = res.to(dev)
        decode_gemm(xd, w.to(dev), out=out, epilogue="add")
    else:
        out = decode_gemm(xd, w.to(dev), epilogue=epi)
    ok, err = rel_close(out.cpu(), ref, 4e-3, 2e-3)
    assert ok, err


@pytest.mark.parametrize("m", [1, 3, 8, 12, 16])
@pytest.mark.parametrize("n,k,epi", [(5120, 3072, "store"), (8192, 3072, "swiglu"),
                                     (1024, 2048, "add"), (512, 4096, "swiglu")])
def test_rmsnorm_decode_gemm_equals_rmsnorm_then_gemm(dev, m, n, k, epi):
    """The fused RMSNorm + projection gives exactly the bits of rmsnorm()
    followed by decode_gemm() (same normalised rows, same GEMM), and matches
    an fp32 reference of RMSNorm + projection (+ SwiGLU / residual add)."""
    import my_cuda_engine_cpp as ops
    from mycustomcudaengine_amd.ops import decode_gemm, rmsnorm_decode_gemm
    g = gen(120 + m + n // 512)
    rows = 2 * n if epi == "swiglu" else n
    xbuf = (torch.randn(m, k + 64, generator=g) * 2).half()
    nw = (1 + 0.1 * torch.randn(k, generator=g)).half()
    w = (torch.randn(rows, k, generator=g) * 0.02).half()
    res = torch.randn(m, n, generator=g).half()
    xd, nwd, wd = xbuf.to(dev)[:, 32:32 + k], nw.to(dev), w.to(dev)
    eps = 1e-5
    if epi == "add":
        fused, split = res.to(dev), res.to(dev)
        rmsnorm_decode_gemm(xd, nwd, eps, wd, out=fused, epilogue="add")
        decode_gemm(ops.rmsnorm(xd, nwd, eps), wd, out=split, epilogue="add")
    else:
        fused = rmsnorm_decode_gemm(xd, nwd, eps, wd, epilogue=epi)
        split = decode_gemm(ops.rmsnorm(xd, nwd, eps), wd, epilogue=epi)
    assert torch.equal(fused.view(torch.int16), split.view(torch.int16))
    x = xbuf[:, 32:32 + k].float()
    xn = x / torch.sqrt((x * x).mean(dim=1, keepdim=True) + eps) * nw.float()
    acc = xn @ w.float().T
    if epi == "swiglu":
        ref = acc[:, :n] * torch.sigmoid(acc[:, :n]) * acc[:, n:]
    elif epi == "add":
        ref = res.float() + acc
    else:
        ref = acc
    ok, err = rel_close(fused.cpu(), ref, 4e-3, 2e-3)
    assert ok, err


def test_rmsnorm_engine_width_matches_fp32(dev):
    """mce_rmsnorm's rows against an fp32 reference at the engine's width."""
    import my_cuda_engine_cpp as ops
    g = gen(140)
    x = (torch.randn(8, 3072, generator=g) * 3).half()
    w = (1 + 0.1 * torch.randn(3072, generator=g)).half()
    y = ops.rmsnorm(x.to(dev), w.to(dev), 1e-5).cpu().float()
    xf = x.float()
    ref = xf / torch.sqrt((xf * xf).mean(dim=1, keepdim=True) + 1e-5) * w.float()
    assert (y - ref).abs().max().item() <= 2e-2


def test_decode_gemm_rejects_unsupported_shapes(dev):
    from mycustomcudaengine_amd import _lib
    from mycustomcudaengine_amd.ops import decode_gemm
    x = torch.zeros(17, 512, dtype=torch.float16, device=dev)
    w = torch.zeros(64, 512, dtype=torch.float16, device=dev)
    with pytest.raises(_lib.MCEError) as ei:
        decode_gemm(x, w)
    assert ei.value.code == _lib.MCE_ERR_UNSUPPORTED



# ------------------------------------------------ device-side decode loop
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,cols,stride", [(8, 128256, 128256), (3, 1000, 1008),
                                              (4, 1003, 1008), (2, 300007, 300016),
                                              (3, 1000, 1011), (1, 1, 9)])
def test_argmax_rows_matches_torch(dev, dtype, rows, cols, stride):
    """Greedy tokens equal torch.argmax (and the numpy oracle) exactly,
    including rows whose maximum repeats, a row with NaNs and a row whose
    maximum is a -0 / +0 tie; strided rows.  Row strides that are multiples of
    8 take the 16-byte-load kernel (with a tail when cols % 8 != 0, and more
    than one pass per thread past 131072 columns), other strides the scalar
    one."""
    from mycustomcudaengine_amd.ops import argmax_rows
    from oracle.alloc_ref import argmax_rows_ref
    g = gen(150 + rows + cols % 7)
    buf = (torch.randn(rows, stride, generator=g) * 4).to(dtype)
    x = buf[:, :cols]
    if cols > 10:
        x[0, cols // 3] = x[0].max() + 1
        x[0, cols // 2] = x[0, cols // 3]          # tie: the first wins
        if rows > 1:
            x[1, 5] = float("nan")
            x[1, cols - 3] = float("nan")          # NaN ranks first, first NaN wins
        if rows > 2:
            x[2] = -x[2].abs() - 1
            x[2, 7] = -0.0
            x[2, cols - 1] = 0.0                    # equal to -0: index 7 wins
    got = argmax_rows(buf.to(dev)[:, :cols]).cpu()
    assert got.tolist() == torch.argmax(x.float(), dim=-1).tolist()
    assert got.tolist() == argmax_rows_ref(x.float().numpy()).tolist()


def test_argmax_rows_many_unaligned_rows(dev):
    """Rows whose stride is not a multiple of 8 take one workgroup per row on
    grid.x, so row counts past the split path's 65535 (grid.y) are accepted
    and equal torch.argmax."""
    from mycustomcudaengine_amd.ops import argmax_rows
    g = gen(171)
    x = (torch.randn(70001, 9, generator=g) * 4).half()
    got = argmax_rows(x.to(dev)).cpu()
    assert got.tolist() == torch.argmax(x.float(), dim=-1).tolist()


def test_decode_advance_matches_oracle_and_replays(dev):
    """Device-side step preparation equals the oracle step after step
    (positions, context lengths, slots from the zero-padded table, -1 past its
    width, the token log), eagerly and as a captured graph replayed several
    times with host checks between the replays."""
    from mycustomcudaengine_amd.ops import decode_advance
    from oracle.alloc_ref import BlockAllocatorRef, decode_advance_ref
    bs, width = 16, 5
    a = BlockAllocatorRef(64, bs)
    rng = np.random.default_rng(3)
    lens = [70, 33, 16, 80]
    for s_, n in enumerate(lens):
        a.allocate_sequence(s_, n)
    table = a.block_table(list(range(4)), width)
    pos = np.array([n - 1 for n in lens], np.int32) - 3
    ctx = pos + 1
    d_tab = torch.from_numpy(table).to(dev)
    d_pos, d_ctx = torch.from_numpy(pos.copy()).to(dev), torch.from_numpy(ctx.copy()).to(dev)
    d_slot = torch.zeros(4, dtype=torch.int32, device=dev)
    ids = torch.zeros(4, dtype=torch.int64, device=dev)
    log = torch.full((6, 4), -7, dtype=torch.int64, device=dev)
    ctr = torch.zeros(1, dtype=torch.int32, device=dev)
    for step in range(3):  # eager
        ids.copy_(torch.from_numpy(rng.integers(0, 1000, 4)))
        want_ids = ids.cpu().clone()
        decode_advance(d_tab, d_pos, d_ctx, d_slot, bs, input_ids=ids, token_log=log,
                       step_counter=ctr)
        pos, ctx, slots = decode_advance_ref(table, pos, ctx, bs)
        assert d_pos.cpu().tolist() == pos.tolist() and d_ctx.cpu().tolist() == ctx.tolist()
        assert d_slot.cpu().tolist() == slots.tolist()
        assert log[step].cpu().tolist() == want_ids.tolist() and int(ctr.item()) == step + 1
    graph = torch.cuda.CUDAGraph()
    s_ = torch.cuda.Stream()
    s_.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s_):
        with torch.cuda.graph(graph, stream=s_):
            decode_advance(d_tab, d_pos, d_ctx, d_slot, bs, input_ids=ids, token_log=log,
                           step_counter=ctr)
    torch.cuda.current_stream().wait_stream(s_)
    torch.cuda.synchronize()
    for step in range(3, 8):  # replays (the log holds 6 rows: later steps are not logged)
        ids.copy_(torch.from_numpy(rng.integers(0, 1000, 4)))
        want_ids = ids.cpu().clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        pos, ctx, slots = decode_advance_ref(table, pos, ctx, bs)
        assert d_pos.cpu().tolist() == pos.tolist() and d_ctx.cpu().tolist() == ctx.tolist()
        assert d_slot.cpu().tolist() == slots.tolist()
        if step < 6:
            assert log[step].cpu().tolist() == want_ids.tolist()
        assert int(ctr.item()) == step + 1
    assert (slots == -1).any()  # a sequence ran past the table width



# ------------------------------------------------ chunked prefill from the page pool
def _paged_case(seed, prefixes, s, dtype=torch.float16, hq=24, hkv=8, bs=16):
    """Per-sequence prefix lengths, chunk of s queries; a shuffled pool whose
    unused pages hold NaN (a read outside the tables would poison rows)."""
    g = gen(seed)
    b = len(prefixes)
    ctx = [p_ + s for p_ in prefixes]
    width = max((c + bs - 1) // bs for c in ctx) + 1
    nb = b * width + 5
    kc = torch.full((nb, bs, hkv, 128), float("nan"), dtype=dtype)
    vc = torch.full((nb, bs, hkv, 128), float("nan"), dtype=dtype)
    perm = torch.randperm(nb, generator=g)
    table = torch.zeros(b, width, dtype=torch.int32)
    for i in range(b):
        blocks = perm[i * width:(i + 1) * width]
        table[i] = blocks.to(torch.int32)
        used = (ctx[i] + bs - 1) // bs
        kc[blocks[:used]] = torch.randn(used, bs, hkv, 128, generator=g).to(dtype)
        vc[blocks[:used]] = torch.randn(used, bs, hkv, 128, generator=g).to(dtype)
    q = torch.randn(b, s, hq, 128, generator=g).to(dtype)
    return q, kc, vc, table, torch.tensor(ctx, dtype=torch.int32)


# Grids of at most 128 workgroups (B x Hkv x ceil(3 s / 128), on a 256-CU
# MI355X) take the key-split kernel, which cuts a query block's keys into
# parts of at least 16 tiles (512 keys) merged by a second launch: the prefix
# 2000 / 3584 / 1500 cases run 4, 5 and 3 parts (the 700-token sequence next
# to the 1500 one stays whole), the other small grids one part (the output
# written by the attention kernel); the last two cases are larger grids.
@pytest.mark.parametrize("prefixes,s,dtype", [([0, 37], 64, torch.float16),
                                              ([100, 5, 300], 17, torch.float16),
                                              ([700], 1, torch.float16),
                                              ([129], 300, torch.float16),
                                              ([2000], 48, torch.float16),
                                              ([0, 64], 96, torch.bfloat16),
                                              ([3584], 512, torch.float16),
                                              ([1500, 700], 64, torch.bfloat16),
                                              ([0, 37, 500], 300, torch.float16),
                                              ([1000, 0, 3000, 17], 200, torch.bfloat16)])
def test_prefill_paged_matches_oracle(dev, prefixes, s, dtype):
    from mycustomcudaengine_amd.ops import prefill_attention_paged
    q, kc, vc, table, ctx = _paged_case(160 + s + len(prefixes), prefixes, s, dtype)
    scale = 1.0 / 128 ** 0.5
    args = (q.to(dev), kc.to(dev), vc.to(dev), table.to(dev), ctx.to(dev), scale)
    refs = [prefill_paged_ref(q[i], kc, vc, table[i].tolist(), int(ctx[i]), scale)
            for i in range(len(prefixes))]
    for split in (True, False):  # with and without the key split of small grids
        out = prefill_attention_paged(*args, split_keys=split).cpu()
        assert not torch.isnan(out).any()
        for i, ref in enumerate(refs):
            err = (out[i].float() - ref).abs().max().item()
            assert err <= TOL, (split, i, err)


@pytest.mark.parametrize("b,s", [(1, 2048), (3, 333), (8, 512), (1, 300), (2, 64)])
def test_prefill_paged_without_prefix_equals_contiguous(dev, b, s):
    """No cached prefix (context == chunk): the paged kernel gives exactly the
    bits of mce_prefill_attention on the same K/V laid out contiguously, also
    from the key-split kernel of small grids (the last two cases: one part
    per query block, so the same arithmetic in the same order)."""
    from mycustomcudaengine_amd.ops import prefill_attention_paged
    q, kc, vc, table, ctx = _paged_case(170 + b, [0] * b, s)
    k = torch.stack([gather_kv_rows(kc, table[i], s) for i in range(b)])
    v = torch.stack([gather_kv_rows(vc, table[i], s) for i in range(b)])
    scale = 1.0 / 128 ** 0.5
    paged = prefill_attention_paged(q.to(dev), kc.to(dev), vc.to(dev), table.to(dev),
                                    ctx.to(dev), scale)
    contig = ops.prefill_attention(q.to(dev), k.to(dev), v.to(dev), scale)
    assert torch.equal(paged.view(torch.int16), contig.view(torch.int16))


def gather_kv_rows(cache, row, n):
    from oracle.ops_ref import gather_kv
    return gather_kv(cache, row.tolist(), n)


def test_prefill_paged_key_split_graph_replays(dev):
    """The key split (attention + merge launches, torch-allocated workspace)
    captured in a HIP graph and replayed several times, with an eager call
    of another shape in between: every replay equals the eager result bit
    for bit."""
    from mycustomcudaengine_amd.ops import prefill_attention_paged
    q, kc, vc, table, ctx = (t.to(dev) for t in _paged_case(180, [2000], 48))
    other = [t.to(dev) for t in _paged_case(181, [1500, 700], 64)]
    scale = 1.0 / 128 ** 0.5
    eager = prefill_attention_paged(q, kc, vc, table, ctx, scale)
    s_ = torch.cuda.Stream(device=dev)
    s_.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s_):
        prefill_attention_paged(q, kc, vc, table, ctx, scale)
    torch.cuda.current_stream(dev).wait_stream(s_)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = prefill_attention_paged(q, kc, vc, table, ctx, scale)
    other_eager = prefill_attention_paged(*other, scale)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16))
        again = prefill_attention_paged(*other, scale)
        torch.cuda.synchronize()
        assert torch.equal(again.view(torch.int16), other_eager.view(torch.int16))
