"""GPU: seeded random sweeps over the engine-side kernels' valid shapes, each
against the CPU oracle or fp32 torch (the bars of test_gpu_ops.py and
test_gpu_decode.py).

  * fused RoPE + KV append + decode attention: batch 1-24, 1-8 kv heads,
    GQA group 1-8, pages of 8-64 tokens, table capacities up to 1024
    tokens; bit-identical to rope_kv_store(query_out=...) +
    paged_attention_decode (output and both caches) and within 1e-2 of the
    oracle (RoPE, store, attention);
  * decode-sized GEMMs: 1-16 tokens, K in {2048, 3072, 4096} (8192 for at
    most 8 tokens without RMSNorm / SwiGLU), N multiples of 16 from 16 to
    20480 plus many-round widths (32768-35200), every epilogue, with and without the fused
    RMSNorm, strided x rows; |err| <= 2e-3 + 4e-3 |ref| against fp32;
  * greedy argmax: 1-64 rows, 1-200000 columns, aligned and unaligned row
    strides, planted ties, NaN, -0 / +0 ties, fp16 and bf16; bit-exact;
  * RMSNorm, SwiGLU, RoPE and the paged KV store (alone and fused) over
    random sizes, strides and positions.

MCE_SWEEP_CASES sets the number of seeds per family (default 12).
"""
import os
import random

import pytest
import torch

import my_cuda_engine_cpp as ops
from mycustomcudaengine_amd.ops import (argmax_rows, decode_gemm, decode_rope_attention,
                                        rmsnorm_decode_gemm, rope_kv_store)
from oracle.alloc_ref import argmax_rows_ref
from oracle.inputs import make_decode_case
from oracle.ops_ref import (decode_attention_ref, kv_store_ref, rmsnorm_ref, rope_ref, rope_tables,
                            swiglu_ref)

TOL = 1e-2
N = int(os.environ.get("MCE_SWEEP_CASES", "12"))
pytestmark = pytest.mark.gpu


def rel_close(out, ref, rel, abs_):
    d = (out.float() - ref).abs()
    return bool((d <= abs_ + rel * ref.abs()).all()), d.max().item()


@pytest.mark.parametrize("i", range(N))
def test_fused_rope_decode_sweep(dev, i):
    r = random.Random(5000 + i)
    b = r.randint(1, 24)
    hkv = r.choice([1, 2, 4, 8])
    g = r.randint(1, 8)
    hq, d = hkv * g, 128
    bs = r.choice([8, 16, 32, 64])
    mb = r.randint(1, 1024 // bs)
    rows = 1100
    ctx = [r.choice([1, r.randint(1, mb * bs), mb * bs]) for _ in range(b)]
    desc = f"B={b} hkv={hkv} G={g} bs={bs} width={mb} ctx={ctx[:6]}"
    print(desc, flush=True)
    case = make_decode_case(6000 + i, b, ctx, num_heads=hq, num_kv_heads=hkv, block_size=bs,
                            max_blocks=mb)
    gen = torch.Generator().manual_seed(7000 + i)
    bt = case.block_tables
    pos = torch.tensor([c - 1 for c in ctx], dtype=torch.int32)
    slots = torch.tensor([int(bt[j, (c - 1) // bs]) * bs + (c - 1) % bs for j, c in enumerate(ctx)],
                         dtype=torch.int32)
    if b > 2 and r.random() < 0.5:
        slots[r.randrange(b)] = -1                   # no store for this row
    if b > 2 and r.random() < 0.5:
        pos[r.randrange(b)] = rows + r.randint(0, 50)  # outside the table: not rotated
    cos, sin = rope_tables(rows, d, 500000.0)
    qkv = torch.randn(b, (hq + 2 * hkv) * d, generator=gen).half()

    def views(buf):
        return (buf[:, :hq * d].view(b, hq, d), buf[:, hq * d:(hq + hkv) * d].view(b, hkv, d),
                buf[:, (hq + hkv) * d:].view(b, hkv, d))

    to = lambda t: t.to(dev)
    args = tuple(map(to, (cos, sin, pos, slots, bt, case.context_lens)))
    qkv1, kc1, vc1 = to(qkv.clone()), to(case.key_cache.clone()), to(case.value_cache.clone())
    out1 = decode_rope_attention(*views(qkv1), kc1, vc1, *args, mb, case.scale)
    qkv2, kc2, vc2 = to(qkv.clone()), to(case.key_cache.clone()), to(case.value_cache.clone())
    q2, k2, v2 = views(qkv2)
    q_rot = torch.empty(b, hq, d, dtype=torch.float16, device=dev)
    rope_kv_store(q2, k2, v2, kc2, vc2, *args[:4], query_out=q_rot)
    out2 = ops.paged_attention_decode(q_rot, kc2, vc2, args[4], args[5], mb, bs, case.scale)
    torch.cuda.synchronize()
    bits = lambda t: t.view(torch.int16)
    assert torch.equal(bits(kc1), bits(kc2)) and torch.equal(bits(vc1), bits(vc2)), desc
    assert torch.equal(bits(out1), bits(out2)), desc
    # oracle: rotate q and k (rows with positions in the table), store k / v, attend
    q, k, v = (t.clone() for t in views(qkv))
    in_tab = (pos >= 0) & (pos < rows)
    pos_c = pos.clamp(0, rows - 1).view(b, 1)
    q_r = rope_ref(q.view(b, 1, hq, d), cos, sin, pos_c).view(b, hq, d)
    k_r = rope_ref(k.view(b, 1, hkv, d), cos, sin, pos_c).view(b, hkv, d)
    q_r = torch.where(in_tab.view(b, 1, 1), q_r, q.float())
    k_r = torch.where(in_tab.view(b, 1, 1), k_r, k.float())
    kr, vr = case.key_cache.numpy().copy(), case.value_cache.numpy().copy()
    kv_store_ref(k_r.half().numpy(), v.numpy(), kr, vr, slots.numpy())
    ref = decode_attention_ref(q_r.half(), torch.from_numpy(kr), torch.from_numpy(vr), bt,
                               case.context_lens, case.scale)
    assert torch.equal(bits(kc1.cpu()), bits(torch.from_numpy(kr))), desc
    err = (out1.float().cpu() - ref).abs().max().item()
    assert err <= TOL, (desc, err)


@pytest.mark.parametrize("i", range(N))
def test_decode_gemm_sweep(dev, i):
    r = random.Random(8000 + i)
    m = r.randint(1, 16)
    epi = r.choice(["store", "add", "swiglu"])
    norm = r.random() < 0.5
    ks = [2048, 3072, 4096] + ([8192] if m <= 8 and not norm and epi != "swiglu" else [])
    k = r.choice(ks)
    n = 16 * r.choice([r.randint(1, 64), r.randint(64, 1280)])
    if epi != "swiglu" and r.random() < 0.25:
        n, k = 16 * r.randint(2048, 2200), r.choice([2048, 3072])  # many rounds of workgroups
    desc = f"m={m} n={n} k={k} {epi} norm={norm}"
    print(desc, flush=True)
    g = torch.Generator().manual_seed(9000 + i)
    rows = 2 * n if epi == "swiglu" else n
    xbuf = (torch.randn(m, k + 64, generator=g) * (2 if norm else 1)).half()
    x = xbuf[:, 32:32 + k]
    nw = (1 + 0.1 * torch.randn(k, generator=g)).half()
    w = (torch.randn(rows, k, generator=g) * 0.02).half()
    xf = x.float()
    if norm:
        # the MFMA operands are fp16: the kernel, like the unfused rmsnorm op
        # followed by the product, rounds the normalised rows to fp16
        xf = xf / torch.sqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5) * nw.float()
        xf = xf.half().float()
    acc = xf @ w.float().T
    res = torch.randn(m, n, generator=g).half()
    if epi == "swiglu":
        ref = acc[:, :n] * torch.sigmoid(acc[:, :n]) * acc[:, n:]
    elif epi == "add":
        ref = res.float() + acc
    else:
        ref = acc
    xd = xbuf.to(dev)[:, 32:32 + k]
    out = res.to(dev) if epi == "add" else None
    if norm:
        got = rmsnorm_decode_gemm(xd, nw.to(dev), 1e-5, w.to(dev), out=out, epilogue=epi)
    else:
        got = decode_gemm(xd, w.to(dev), out=out, epilogue=epi)
    ok, err = rel_close(got.cpu(), ref, 4e-3, 2e-3)
    assert ok, (desc, err)


@pytest.mark.parametrize("i", range(N))
def test_argmax_sweep(dev, i):
    r = random.Random(10000 + i)
    rows = r.randint(1, 64)
    cols = r.choice([r.randint(1, 64), r.randint(64, 5000), r.randint(5000, 200000)])
    stride = cols + r.choice([0, 0, r.randint(1, 9), 8 * r.randint(1, 4)])
    dtype = r.choice([torch.float16, torch.bfloat16])
    desc = f"rows={rows} cols={cols} stride={stride} {dtype}"
    print(desc, flush=True)
    g = torch.Generator().manual_seed(11000 + i)
    buf = (torch.randn(rows, stride, generator=g) * 3).to(dtype)
    x = buf[:, :cols]
    for row in range(rows):
        kind = r.random()
        if kind < 0.2 and cols > 2:                  # repeated maximum: the first wins
            a, c = sorted(r.sample(range(cols), 2))
            x[row, a] = x[row].max() + 1
            x[row, c] = x[row, a]
        elif kind < 0.3:                             # NaN ranks first
            x[row, r.randrange(cols)] = float("nan")
        elif kind < 0.4 and cols > 2:                # -0 / +0 tie at the top
            x[row] = -x[row].abs() - 1
            a, c = sorted(r.sample(range(cols), 2))
            x[row, a] = -0.0
            x[row, c] = 0.0
    got = argmax_rows(buf.to(dev)[:, :cols]).cpu()
    assert got.tolist() == argmax_rows_ref(x.float().numpy()).tolist(), desc


@pytest.mark.parametrize("i", range(N))
def test_elementwise_sweep(dev, i):
    r = random.Random(12000 + i)
    g = torch.Generator().manual_seed(13000 + i)
    dtype = r.choice([torch.float16, torch.bfloat16])
    # RMSNorm
    rows, hidden = r.randint(1, 300), r.choice([r.randint(1, 600), 8 * r.randint(1, 1100)])
    x = torch.randn(rows, hidden, generator=g).to(dtype)
    w = (1 + 0.3 * torch.randn(hidden, generator=g)).to(dtype)
    out = ops.rmsnorm(x.to(dev), w.to(dev), 1e-5).cpu()
    ok, err = rel_close(out, rmsnorm_ref(x, w, 1e-5), 4e-3 if dtype == torch.float16 else 1.6e-2,
                        1e-3)
    assert ok, ("rmsnorm", rows, hidden, dtype, err)
    # SwiGLU
    rows, inter = r.randint(1, 300), r.choice([r.randint(1, 600), 8 * r.randint(1, 1100)])
    gu = torch.randn(rows, 2 * inter, generator=g).to(dtype)
    out = ops.swiglu(gu.to(dev)).cpu()
    ok, err = rel_close(out, swiglu_ref(gu), 4e-3 if dtype == torch.float16 else 1.6e-2, 1e-3)
    assert ok, ("swiglu", rows, inter, dtype, err)
    # RoPE (views into a fused projection) + the paged KV store, alone and fused (fp16)
    b, s = r.randint(1, 4), r.randint(1, 300)
    hkv = r.choice([1, 2, 4, 8])
    hq, d, bs = hkv * r.randint(1, 8), 128, r.choice([8, 16, 32])
    table = 2048
    cos, sin = rope_tables(table, d, 500000.0)
    fused = torch.randn(b, s, (hq + 2 * hkv) * d, generator=g).half()
    pos = torch.randint(0, table + 40, (b, s), generator=g, dtype=torch.int32)  # some outside
    nb = (b * s + bs - 1) // bs + 4
    slots = torch.randperm(nb * bs, generator=g)[:b * s].to(torch.int32)
    slots[torch.rand(b * s, generator=g) < 0.1] = -1
    kc0 = torch.randn(nb, bs, hkv, d, generator=g).half()
    vc0 = torch.randn(nb, bs, hkv, d, generator=g).half()

    def split(t):
        return (t[..., :hq * d].view(b, s, hq, d), t[..., hq * d:(hq + hkv) * d].view(b, s, hkv, d),
                t[..., (hq + hkv) * d:].view(b, s, hkv, d))

    q, k, v = split(fused)
    inside = ((pos >= 0) & (pos < table)).view(b, s, 1, 1)
    pc = pos.clamp(0, table - 1)
    q_ref = torch.where(inside, rope_ref(q, cos, sin, pc), q.float())
    k_ref = torch.where(inside, rope_ref(k, cos, sin, pc), k.float())
    fd = fused.to(dev)
    qd, kd, vd = split(fd)
    ops.rope_inplace(qd, kd, cos.to(dev), sin.to(dev), pos.to(dev))
    qg, kg = qd.cpu(), kd.cpu()
    assert rel_close(qg, q_ref, 4e-3, 2e-3)[0] and rel_close(kg, k_ref, 4e-3, 2e-3)[0], \
        ("rope", b, s, hq, hkv)
    kc, vc = kc0.clone().to(dev), vc0.clone().to(dev)
    ops.paged_kv_store(kd.reshape(b * s, hkv, d), vd.reshape(b * s, hkv, d), kc, vc, slots.to(dev))
    kr, vr = kc0.numpy().copy(), vc0.numpy().copy()
    kv_store_ref(kg.reshape(b * s, hkv, d).numpy(), v.reshape(b * s, hkv, d).numpy(), kr, vr,
                 slots.numpy())
    assert torch.equal(kc.cpu(), torch.from_numpy(kr)) and torch.equal(vc.cpu(), torch.from_numpy(vr))
    # fused RoPE + store from the unrotated projection: same bits as the two ops
    fd2 = fused.to(dev)
    q2, k2, v2 = split(fd2)
    kc2, vc2 = kc0.clone().to(dev), vc0.clone().to(dev)
    rope_kv_store(q2.reshape(b * s, hq, d), k2.reshape(b * s, hkv, d), v2.reshape(b * s, hkv, d),
                  kc2, vc2, cos.to(dev), sin.to(dev), pos.reshape(-1).to(dev), slots.to(dev))
    assert torch.equal(fd2.cpu()[..., :(hq + hkv) * d], fd.cpu()[..., :(hq + hkv) * d])
    assert torch.equal(kc2.cpu(), kc.cpu()) and torch.equal(vc2.cpu(), vc.cpu())
