"""GPU parity of paged decode attention against the CPU oracle.

Bar: max |gpu - fp32 oracle| <= 1e-2 (the reference's tolerance class,
tests/test_paged_attention.py:86, tightened to max-abs per BASELINE), no NaN,
block-table handling exact (NaN-filled unused pool blocks must not leak).
"""
import math

import pytest
import torch

import my_cuda_engine_cpp as ops
from mycustomcudaengine_amd.ops import decode_rope_attention, rope_kv_store
from oracle.inputs import cfg1_decode, cfg2_decode, cfg4_decode, make_decode_case
from oracle.ops_ref import decode_attention_ref

TOL = 1e-2
pytestmark = pytest.mark.gpu


def run_gpu(case, dev):
    out = ops.paged_attention_decode(
        case.query.to(dev), case.key_cache.to(dev), case.value_cache.to(dev),
        case.block_tables.to(dev), case.context_lens.to(dev), case.max_blocks,
        case.block_size, case.scale)
    torch.cuda.synchronize()
    return out.cpu()


def check(case, dev, tol=TOL):
    out = run_gpu(case, dev)
    ref = decode_attention_ref(case.query, case.key_cache, case.value_cache,
                               case.block_tables, case.context_lens, case.scale)
    assert out.shape == ref.shape and out.dtype == case.query.dtype
    assert not torch.isnan(out).any(), "NaN in output (pool sentinel leaked?)"
    err = (out.float() - ref).abs().max().item()
    assert err <= tol, f"max abs err {err}"
    return out, ref


def test_cfg1(dev):
    check(cfg1_decode(), dev)


def test_cfg2_batched_mixed_context(dev):
    check(cfg2_decode(nan_pool=True), dev)


def test_cfg4_long_context_split_k(dev):
    check(cfg4_decode(), dev)


def reference_harness_case(dev):
    """The reference's own decode test shape (tests/test_paged_attention.py:12-54):
    B=16, Hq = Hkv = 32 (no GQA), D=128, ctx 2048, 16-token blocks from
    KVCacheManager (contiguous ascending tables), Q/K/V ~ N(0, 1) fp16 drawn
    with a seeded CPU generator."""
    from mycustomcudaengine_amd.engine.cache import KVCacheManager
    b, h, d, ctx, bs = 16, 32, 128, 2048, 16
    mgr = KVCacheManager(num_blocks=b * ctx // bs, block_size=bs, num_layers=1, num_heads=h,
                         head_dim=d, device=dev)
    for s in range(b):
        mgr.allocate_sequence(s, ctx)
    g = torch.Generator().manual_seed(42)
    mgr.kv_cache.copy_(torch.randn(mgr.kv_cache.shape, generator=g).half())
    q = torch.randn(b, h, d, generator=g).half()
    bt = mgr.get_block_table_tensor(list(range(b)), ctx // bs)
    cl = torch.full((b,), ctx, dtype=torch.int32)
    return q, mgr.kv_cache[0, 0], mgr.kv_cache[0, 1], bt, cl, ctx // bs, bs, 1.0 / math.sqrt(d)


def test_reference_harness_shape(dev):
    """The reference's decode harness (B=16, 32/32 heads, ctx 2048, ascending
    tables): max-abs 1e-2 of the fp32 oracle, and the reference's own check,
    allclose(atol=1e-2, rtol=1e-2) against fp16 SDPA on contiguous copies
    (tests/test_paged_attention.py:65-86), here computed on the CPU."""
    q, kc, vc, bt, cl, mb, bs, scale = reference_harness_case(dev)
    assert bt.cpu().view(-1).tolist() == list(range(16 * mb))  # contiguous ascending
    out = ops.paged_attention_decode(q.to(dev), kc, vc, bt, cl.to(dev), mb, bs, scale).cpu()
    ref = decode_attention_ref(q, kc.cpu(), vc.cpu(), bt.cpu(), cl, scale)
    assert (out.float() - ref).abs().max().item() <= TOL
    # the reference's fp16 SDPA check, run on the CPU
    k = kc.cpu().view(16, 2048, 32, 128).transpose(1, 2).contiguous()
    v = vc.cpu().view(16, 2048, 32, 128).transpose(1, 2).contiguous()
    sdpa = torch.nn.functional.scaled_dot_product_attention(q.unsqueeze(2), k, v,
                                                            scale=scale).squeeze(2)
    assert sdpa.dtype == torch.float16
    assert torch.allclose(out, sdpa, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("ctx", [1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129,
                                 255, 256, 257, 511, 513, 1000, 1024, 1025, 2049])
def test_context_edges(dev, ctx):
    check(make_decode_case(100 + ctx, 2, [ctx, max(1, ctx // 2 + 3)]), dev)


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (24, 8), (32, 8), (40, 8), (64, 8),
                                    (6, 2), (3, 1)])
def test_gqa_groups(dev, hq, hkv):
    check(make_decode_case(7 + hq, 3, [300, 17, 1100], num_heads=hq, num_kv_heads=hkv), dev)


@pytest.mark.parametrize("hq,hkv,b", [(8, 8, 3), (24, 8, 3), (24, 8, 8), (32, 8, 16), (48, 8, 8),
                                      (64, 8, 8), (64, 8, 4), (6, 2, 5), (3, 1, 7), (24, 8, 40)])
def test_gqa_groups_per_sequence_mode(dev, hq, hkv, b):
    """Contexts within 1024 tokens of table capacity (one workgroup per
    sequence and kv head, or per query-head slice of a kv head when the grid
    would leave CUs idle): every split of the G query heads, including none."""
    ctxs = torch.randint(1, 641, (b,), generator=torch.Generator().manual_seed(hq * 100 + b))
    check(make_decode_case(60 + hq + b, b, ctxs.tolist(), num_heads=hq, num_kv_heads=hkv,
                           max_blocks=40), dev)


@pytest.mark.parametrize("bs", [8, 16, 32, 64, 256])
def test_block_sizes(dev, bs):
    check(make_decode_case(11 + bs, 3, [700, 5, 1500], block_size=bs), dev)


def test_ctx_one_returns_v0(dev):
    case = make_decode_case(5, 4, [1, 1, 1, 1])
    out = run_gpu(case, dev)
    hkv = case.key_cache.shape[2]
    grp = case.query.shape[1] // hkv
    for b in range(4):
        blk = int(case.block_tables[b, 0])
        v0 = case.value_cache[blk, 0].repeat_interleave(grp, dim=0)
        assert torch.equal(out[b], v0)


def test_zero_context_rows_are_zero(dev):
    case = make_decode_case(6, 3, [0, 40, 0])
    out, ref = check(case, dev)
    assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[2]) == 0


def test_block_table_permutation_invariance(dev):
    """Physically relocating a sequence's blocks must not change its output."""
    case = make_decode_case(8, 2, [400, 333], nan_pool=True)
    out1 = run_gpu(case, dev)
    kc, vc, bt = case.key_cache.clone(), case.value_cache.clone(), case.block_tables.clone()
    nb = kc.shape[0]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(3))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(nb)
    kc2, vc2 = kc[perm], vc[perm]  # new block j holds old block perm[j]
    bt2 = inv[bt.long()].to(torch.int32)
    case.key_cache, case.value_cache, case.block_tables = kc2, vc2, bt2
    out2 = run_gpu(case, dev)
    assert torch.equal(out1, out2)


def test_graph_capture_replay(dev):
    """hipGraph capture through torch.cuda.graph; replays match eager."""
    case = make_decode_case(9, 8, [513, 600, 17, 4000, 1, 256, 257, 3000])
    q = case.query.to(dev)
    kc, vc = case.key_cache.to(dev), case.value_cache.to(dev)
    bt, cl = case.block_tables.to(dev), case.context_lens.to(dev)
    args = (kc, vc, bt, cl, case.max_blocks, case.block_size, case.scale)
    eager = ops.paged_attention_decode(q, *args)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.paged_attention_decode(q, *args)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_out = ops.paged_attention_decode(q, *args)
    for i in range(4):
        q.copy_(case.query.to(dev) * (1.0 + 0.1 * i))
        g.replay()
        torch.cuda.synchronize()
        want = ops.paged_attention_decode(q, *args)
        torch.cuda.synchronize()
        assert torch.equal(static_out, want), f"replay {i} differs from eager"
    q.copy_(case.query.to(dev))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(static_out, eager)


def test_rejects_bad_inputs(dev):
    case = make_decode_case(10, 1, [64])
    q = case.query.to(dev)
    kc, vc = case.key_cache.to(dev), case.value_cache.to(dev)
    bt, cl = case.block_tables.to(dev), case.context_lens.to(dev)
    with pytest.raises(RuntimeError):
        ops.paged_attention_decode(q.float(), kc, vc, bt, cl, case.max_blocks, 16, case.scale)
    with pytest.raises(RuntimeError):
        ops.paged_attention_decode(q, kc, vc, bt.long(), cl, case.max_blocks, 16, case.scale)
    with pytest.raises(RuntimeError):
        ops.paged_attention_decode(q, kc, vc, bt, cl, case.max_blocks, 8, case.scale)
    with pytest.raises(RuntimeError):
        ops.paged_attention_decode(q[..., :64].contiguous(), kc[..., :64].contiguous(),
                                   vc[..., :64].contiguous(), bt, cl, case.max_blocks, 16,
                                   case.scale)


@pytest.mark.parametrize("b,hi,mb", [(2048, 64, 72), (700, 300, 72), (700, 400, 25)])
def test_large_batches(dev, b, hi, mb):
    """Batches past one pass of the split partition's context-length prefix
    sum (512 sequences per pass, up to the 2048 sequences a call takes), with
    empty rows mixed in: the split mode (table capacity 1152 tokens) and the
    per-sequence mode (400), on a NaN-filled pool."""
    g = torch.Generator().manual_seed(700 + b + hi)
    ctxs = torch.randint(0, hi + 1, (b,), generator=g).tolist()
    check(make_decode_case(71 + b, b, ctxs, max_blocks=mb), dev)


def test_rejects_batch_over_limit(dev):
    """2049 sequences exceed what one call takes: an error before any launch."""
    case = make_decode_case(72, 2049, [1] * 2049)
    with pytest.raises(RuntimeError, match="batch 2049"):
        run_gpu(case, dev)


@pytest.mark.parametrize("ctxs,mb", [([512], None), ([3000, 129, 2048, 4096], None),
                                     ([600] * 8, 48), ([9000, 700], 1024), ([0, 33, 1], 4)])
def test_bf16(dev, ctxs, mb):
    """bf16 caches and query (v_dot2_f32_bf16 scores and P V, p packed as
    bf16): split-K and per-sequence modes, empty and one-token rows."""
    case = make_decode_case(50 + len(ctxs) + sum(ctxs) % 7, len(ctxs), ctxs, max_blocks=mb,
                            dtype=torch.bfloat16)
    check(case, dev)


def test_workspace_reuse_across_shapes(dev):
    """Alternate multi-part shapes through fresh workspaces and re-check each
    (partials of one call never leak into the next)."""
    cases = [make_decode_case(40, 4, [3000, 129, 2048, 4096]),
             make_decode_case(41, 2, [9000, 700], max_blocks=1024),
             make_decode_case(42, 8, [600] * 8)]
    for rep in range(2):
        for case in cases:
            check(case, dev)


def test_split_decode_graph_replays(dev):
    """Split-K decode (decode + merge launches, torch-allocated workspace)
    captured in a HIP graph and replayed several times, with eager calls of
    another shape in between: every replay equals the eager result bit for
    bit."""
    case = make_decode_case(44, 6, [3000, 129, 4096, 0, 2048, 1500])
    other = make_decode_case(45, 3, [5000, 64, 2200])
    q, kc, vc, bt, cl = (t.to(dev) for t in (case.query, case.key_cache, case.value_cache,
                                             case.block_tables, case.context_lens))
    mb, bs = bt.shape[1], kc.shape[1]
    eager = ops.paged_attention_decode(q, kc, vc, bt, cl, mb, bs, case.scale)
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        ops.paged_attention_decode(q, kc, vc, bt, cl, mb, bs, case.scale)
    torch.cuda.current_stream(dev).wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ops.paged_attention_decode(q, kc, vc, bt, cl, mb, bs, case.scale)
    other_ref = run_gpu(other, dev)
    for _ in range(4):
        g.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(out, eager)
        assert torch.equal(run_gpu(other, dev), other_ref)


@pytest.mark.parametrize("hq,hkv,b", [(24, 8, 8), (24, 8, 40), (32, 8, 16), (8, 8, 3), (3, 1, 5)])
def test_fused_rope_decode_equals_separate_ops(dev, hq, hkv, b):
    """decode_rope_attention (RoPE + KV append + attention in one launch) is
    bit-identical to rope_kv_store(query_out=...) + paged_attention_decode:
    output, key cache and value cache.  q/k/v are views into one fused
    projection row; one position lies outside the RoPE table (not rotated),
    one slot is -1 (no store) and one lies at an earlier position of its
    sequence (the row the attention reads there is the new one), as the
    separate ops treat them."""
    d, bs, mb, rows = 128, 16, 40, 700
    gen = torch.Generator().manual_seed(hq * 31 + b)
    ctx = torch.randint(1, mb * bs + 1, (b,), generator=gen).tolist()
    case = make_decode_case(90 + hq + b, b, ctx, num_heads=hq, num_kv_heads=hkv, max_blocks=mb)
    pos = torch.tensor([c - 1 for c in ctx], dtype=torch.int32)
    bt = case.block_tables
    slots = torch.tensor([int(bt[i, (c - 1) // bs]) * bs + (c - 1) % bs for i, c in enumerate(ctx)],
                         dtype=torch.int32)
    if b > 2:
        slots[1] = -1
        pos[2] = rows + 5  # outside the table
    if b > 3 and ctx[3] > 1:
        p3 = ctx[3] // 2  # an earlier token of sequence 3 takes the new k / v
        slots[3] = int(bt[3, p3 // bs]) * bs + p3 % bs
    inv = 1.0 / (500000.0 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    ang = torch.outer(torch.arange(rows, dtype=torch.float32), inv)
    cos, sin = ang.cos().contiguous(), ang.sin().contiguous()
    qkv = torch.randn(b, (hq + 2 * hkv) * d, generator=gen).half()
    to = lambda t: t.to(dev)
    cos_d, sin_d, pos_d, slots_d, bt_d, cl_d = map(to, (cos, sin, pos, slots, bt, case.context_lens))

    def views(buf):
        return (buf[:, :hq * d].view(b, hq, d), buf[:, hq * d:(hq + hkv) * d].view(b, hkv, d),
                buf[:, (hq + hkv) * d:].view(b, hkv, d))

    qkv1, kc1, vc1 = to(qkv.clone()), to(case.key_cache.clone()), to(case.value_cache.clone())
    q1, k1, v1 = views(qkv1)
    out1 = decode_rope_attention(q1, k1, v1, kc1, vc1, cos_d, sin_d, pos_d, slots_d, bt_d, cl_d,
                                 mb, case.scale)
    qkv2, kc2, vc2 = to(qkv.clone()), to(case.key_cache.clone()), to(case.value_cache.clone())
    q2, k2, v2 = views(qkv2)
    q_rot = torch.empty(b, hq, d, dtype=torch.float16, device=dev)
    rope_kv_store(q2, k2, v2, kc2, vc2, cos_d, sin_d, pos_d, slots_d, query_out=q_rot)
    out2 = ops.paged_attention_decode(q_rot, kc2, vc2, bt_d, cl_d, mb, bs, case.scale)
    torch.cuda.synchronize()
    assert torch.equal(qkv1[:, :hq * d], qkv.to(dev)[:, :hq * d])  # query untouched
    bits = lambda t: t.view(torch.int16)  # the pools hold NaN sentinels
    assert torch.equal(bits(kc1), bits(kc2)) and torch.equal(bits(vc1), bits(vc2))
    assert torch.equal(bits(out1), bits(out2))


def test_fused_rope_decode_rejects_long_tables(dev):
    case = make_decode_case(3, 1, [100], max_blocks=128)
    q = torch.zeros(1, 24, 128, dtype=torch.float16, device=dev)
    k = torch.zeros(1, 8, 128, dtype=torch.float16, device=dev)
    tab = torch.zeros(16, 64, device=dev)
    one = torch.zeros(1, dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="capacity"):
        decode_rope_attention(q, k, k, case.key_cache.to(dev), case.value_cache.to(dev), tab,
                              tab, one, one, case.block_tables.to(dev), one, 128, 0.1)


def test_cfg2_repeat_calls_identical(dev):
    """Back-to-back calls on the same inputs give bit-identical outputs."""
    case = make_decode_case(43, 16, [4096, 1000, 300, 2500] * 4)
    first = run_gpu(case, dev)
    for _ in range(3):
        assert torch.equal(run_gpu(case, dev), first)


@pytest.mark.parametrize("pad", ["minus_one", "past_pool", "nan_block"])
@pytest.mark.parametrize("mb", [40, 80])
def test_padded_tables_short_contexts(dev, pad, mb):
    """Table entries past a sequence's blocks are never used: padding of -1,
    ids past the pool, or ids of NaN-filled pool blocks leave the result
    unchanged.  The fused per-sequence kernel reads each wave's first tile's
    block id straight from the table row, also for tiles past a short context
    (waves 1-7 of a 1-token sequence); the split mode (capacity 1280 tokens,
    mb = 80) reads ids inside the context only.  Plain decode against the
    oracle (mb = 40: per-sequence mode, 80: split), fused decode against the
    separate ops bit for bit and against the oracle on the updated cache."""
    d, bs, b, rows = 128, 16, 8, 1400
    ctx = [1, 5, 16, 17, 33, 100, 255, 257]
    case = make_decode_case(140 + mb, b, ctx, max_blocks=mb)
    pool = case.key_cache.shape[0]
    bt = case.block_tables.clone()
    used = {int(v) for i, c in enumerate(ctx) for v in bt[i, :(c + bs - 1) // bs]}
    nan_ids = [i for i in range(pool) if i not in used]
    assert nan_ids and torch.isnan(case.key_cache[nan_ids[0]]).all()
    fill = {"minus_one": -1, "past_pool": pool + 12345, "nan_block": nan_ids[0]}[pad]
    for i, c in enumerate(ctx):
        bt[i, (c + bs - 1) // bs:] = fill
    padded = type(case)(case.query, case.key_cache, case.value_cache, bt, case.context_lens,
                        case.block_size, case.scale)
    check(padded, dev)
    if mb * bs > 1024:
        return  # the fused kernel takes tables of at most 1024 tokens
    gen = torch.Generator().manual_seed(141)
    pos = torch.tensor([c - 1 for c in ctx], dtype=torch.int32)
    slots = torch.tensor([int(bt[i, (c - 1) // bs]) * bs + (c - 1) % bs for i, c in enumerate(ctx)],
                         dtype=torch.int32)
    inv = 1.0 / (500000.0 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    ang = torch.outer(torch.arange(rows, dtype=torch.float32), inv)
    cos, sin = ang.cos().contiguous(), ang.sin().contiguous()
    hq, hkv = 24, 8
    qkv = torch.randn(b, (hq + 2 * hkv) * d, generator=gen).half()
    to = lambda t: t.to(dev)
    cos_d, sin_d, pos_d, slots_d, bt_d, cl_d = map(to, (cos, sin, pos, slots, bt, case.context_lens))

    def views(buf):
        return (buf[:, :hq * d].view(b, hq, d), buf[:, hq * d:(hq + hkv) * d].view(b, hkv, d),
                buf[:, (hq + hkv) * d:].view(b, hkv, d))

    qkv1, kc1, vc1 = to(qkv.clone()), to(case.key_cache.clone()), to(case.value_cache.clone())
    out1 = decode_rope_attention(*views(qkv1), kc1, vc1, cos_d, sin_d, pos_d, slots_d, bt_d, cl_d,
                                 mb, case.scale)
    qkv2, kc2, vc2 = to(qkv.clone()), to(case.key_cache.clone()), to(case.value_cache.clone())
    q_rot = torch.empty(b, hq, d, dtype=torch.float16, device=dev)
    rope_kv_store(*views(qkv2), kc2, vc2, cos_d, sin_d, pos_d, slots_d, query_out=q_rot)
    out2 = ops.paged_attention_decode(q_rot, kc2, vc2, bt_d, cl_d, mb, bs, case.scale)
    torch.cuda.synchronize()
    bits = lambda t: t.view(torch.int16)
    assert torch.equal(bits(out1), bits(out2))
    assert torch.equal(bits(kc1), bits(kc2)) and torch.equal(bits(vc1), bits(vc2))
    ref = decode_attention_ref(q_rot.cpu(), kc1.cpu(), vc1.cpu(), bt, case.context_lens, case.scale)
    out = out1.cpu()
    assert not torch.isnan(out).any()
    assert (out.float() - ref).abs().max().item() <= TOL
