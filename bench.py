"""Benchmark of the attention hot path on one MI355X.

Headline (`value`): paged decode attention at cfg2 (B=32, ctx ~ U[128, 4096],
24/8 heads, D=128, 16-token pages, shuffled block tables) in algorithmic HBM
GB/s: every K/V byte once, q and out once, the block-table entries used.
One "step" = one paged_attention_decode call over the whole batch, inputs
resident in HBM.  Timed with HIP events on the launch stream over K
back-to-back calls, after W warm-up calls and at least DECODE_WARMUP_MS of
them; `value` is the median of 5 such windows, each started behind a few
queued untimed calls (the same op captured in a hipGraph and replayed is
timed too and reported beside it).

Extra fields on the same JSON line:
  prefill   cfg3 causal prefill (S=2048, 24/8 heads): algorithmic TFLOP/s
            (2 * D * Hq * S * (S+1)) and fraction of dense fp16 MFMA peak;
            the cfg3 pipeline's other legs beside it: RoPE in place of q and
            k, the paged KV store of the 2048 tokens, and the two fused; and
            the reference's prefill benchmark (benchmark_prefill_attn.py: B=1,
            S = 128 .. 2048) timed beside torch SDPA (causal, fused backends).
  splitk    cfg4 long-context decode (B=8, ctx 32768): GB/s.
  ref_harness  the reference's own decode harness shape (B=16, 32/32 heads,
            ctx 2048, ascending tables; tests/test_paged_attention.py:12-125)
            timed beside torch SDPA (fp16, contiguous K/V) on the same GPU.
  norms     RMSNorm at the reference's harness shape (8 x 2048 x 4096,
            tests/test_ops.py:17-61) and cfg5's 4096 x 3072, SwiGLU at
            [4096, 16384]: us, GB/s, fraction of HBM peak, beside torch.
  model     cfg5 Llama-3.2-3B random-init, B=8, prefill 512 then 128 greedy
            decode steps replayed via hipGraph: tok/s, ms/step, TTFT.
  model_b1  the same at B=1, the shape the reference's engine benchmark
            prints TTFT, inter-token latency and tok/s for.
  measured_ceilings  context beside the published peaks (which stay the
            roofline denominators): a 1 GiB device copy's GB/s and a hipBLASLt
            fp16 8192^3 GEMM's TFLOP/s, with the decode and prefill figures as
            fractions of them.
  cpu_baseline  the CPU oracle on the same cfg2 inputs, on this host's cores
            (prefill, splitk and model carry their own: cfg3, cfg4, and a
            bounded cfg5 sample -- B=8 prefill of the 512-token prompts then 4
            greedy steps at positions 512-515 of the fp32 model oracle).

  chunked   (--only chunked; not in the default run) chunked prefill from the
            page pool, B=1 chunk 512 behind 0-7680 cached tokens and B=4 chunk
            128 behind 2048, with and without the key split: us, TFLOP/s.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                       [--only decode|prefill|legs|splitk|harness|norms|model|chunked|ceilings]
(--only runs one workload; only the default run prints the full result line.)
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import platform
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, vendor spec
ROOT = os.path.dirname(os.path.abspath(__file__))
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_hbm_traffic.json")
DECODE_SOURCE = os.path.join(ROOT, "mycustomcudaengine_amd", "csrc", "decode_attention.hip")
FP16_DENSE_TFLOPS = 2500.0     # MI355X dense fp16 MFMA, vendor spec
METRIC = "decode-attn HBM GB/s (% peak); prefill-attn TFLOPS (% MFMA); 3B decode tok/s"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# Untimed calls issued in front of every timing window: the start event is
# recorded behind them, so it fires while the GPU is already busy and the host
# is ahead of it; the window then holds the K calls' GPU time, not the host's
# latency to its first launch (~15 us of Python per call, which 20 calls of a
# 55 us kernel would otherwise average in).
LEAD_CALLS = 5


def time_gpu(fn, steps: int, warmup: int, rounds: int = 5) -> float:
    """Average ms per call of fn(), issued eagerly from Python, measured with
    HIP events on the current stream over `steps` back-to-back calls after
    LEAD_CALLS queued untimed ones (the host's per-call work still counts
    whenever the GPU work is shorter than the Python call).  The median of
    `rounds` such windows (the first windows after other work can run at lower
    clocks)."""
    for _ in range(warmup):
        fn()
    stream = torch.cuda.current_stream()
    times = []
    for _ in range(rounds):
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        for _ in range(LEAD_CALLS):
            fn()
        start.record(stream)
        for _ in range(steps):
            fn()
        stop.record(stream)
        torch.cuda.synchronize()
        times.append(start.elapsed_time(stop) / steps)
    return sorted(times)[len(times) // 2]


def time_graph_batch(fn, calls: int = 20, replays: int = 20, warmup: int = 3) -> float:
    """Average ms per call of fn() with `calls` back-to-back calls captured in
    one hipGraph, replayed `replays` times (HIP events around the replays;
    the median of 5 such windows):
    per-kernel time plus the gap between consecutive kernels, without the
    host's per-call Python work (which exceeds a few-microsecond kernel)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(max(1, warmup)):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    for _ in range(warmup):
        graph.replay()
    stream = torch.cuda.current_stream()
    times = []
    for _ in range(5):  # median of 5 windows
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(replays):
            graph.replay()
        stop.record(stream)
        torch.cuda.synchronize()
        times.append(start.elapsed_time(stop) / (replays * calls))
    return sorted(times)[2]


def cpu_info() -> dict:
    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "torch": torch.__version__}


# Warm-up of a decode benchmark, in milliseconds of back-to-back calls: the
# first milliseconds of load after the GPU idled (input generation on the host)
# run at lower clocks (measured: cfg2 57.2-57.5 us per call after 100 warm-up
# calls, 55.2-55.3 us after 2000 ~ 110 ms, equal to the graph-replayed figure).
DECODE_WARMUP_MS = 250.0


def bench_decode(case, dev, steps, warmup, rounds=5):
    """Decode attention on `case`: back-to-back eager op calls (decode kernel +
    merge kernel) timed with HIP events after at least DECODE_WARMUP_MS of
    warm-up calls (the median of `rounds` windows of `steps` calls), plus the
    same call captured 20 times in one hipGraph."""
    import my_cuda_engine_cpp as ops
    q = case.query.to(dev)
    kc, vc = case.key_cache.to(dev), case.value_cache.to(dev)
    bt, cl = case.block_tables.to(dev), case.context_lens.to(dev)
    fn = lambda: ops.paged_attention_decode(q, kc, vc, bt, cl, case.max_blocks,
                                            case.block_size, case.scale)
    probe = time_gpu(fn, 10, 2, rounds=1)  # ms per call, to size the warm-up
    warm = max(warmup, int(DECODE_WARMUP_MS / max(probe, 1e-3)))
    ms = time_gpu(fn, steps, warm, rounds)
    graph_ms = time_graph_batch(fn)
    nbytes = case.algorithmic_bytes()
    return ms, nbytes, nbytes / (ms * 1e-3) / 1e9, graph_ms, warm


# Warm-up calls before an MFMA-bound workload is timed: after memory-bound
# work the first few milliseconds of matrix load run at a lower clock
# (measured: the first 50-call window of cfg3 prefill 44.5 us per call, every
# later window 40.0-40.5 us), so ~10 ms of calls precede the timed windows.
MFMA_WARMUP_CALLS = 250


def bench_prefill(case, dev, steps, warmup):
    """cfg3 causal prefill: back-to-back eager calls (one kernel each) timed
    with HIP events after MFMA_WARMUP_CALLS warm-up calls, plus the same call
    captured 20 times in one hipGraph and replayed."""
    import my_cuda_engine_cpp as ops
    q, k, v = case.query.to(dev), case.key.to(dev), case.value.to(dev)
    fn = lambda: ops.prefill_attention(q, k, v, case.scale)
    ms = time_gpu(fn, steps, max(warmup, MFMA_WARMUP_CALLS), rounds=5)
    graph_ms = time_graph_batch(fn)
    flops = case.algorithmic_flops()
    return ms, flops, flops / (ms * 1e-3) / 1e12, graph_ms


def bench_prefill_legs(case, dev, steps, warmup) -> dict:
    """cfg3's other legs, each timed alone (20 back-to-back calls captured in
    one hipGraph and replayed; the eager per-call time, which the host's
    Python work bounds for kernels this short, is reported beside it): RoPE in place of q [1, 2048, 24, 128] and k [1, 2048, 8, 128]
    (theta 5e5, positions 0..2047), the paged KV store of the 2048 tokens'
    k and v into a shuffled 16-token page pool (136 blocks, 128 used), and
    the two fused in one launch (rope_kv_store).  Algorithmic bytes: RoPE
    reads and writes q and k once and reads one cos and one sin row per token
    (2048 x 64 x 4 B each) and the positions; the store reads k and v and
    writes them once, plus the slots; the fused op rotates k in place and
    also stores it."""
    import my_cuda_engine_cpp as ops
    from mycustomcudaengine_amd.engine.models.llama import rope_tables
    from mycustomcudaengine_amd.ops import rope_kv_store
    b, s, hq, hkv, d, bs = 1, 2048, 24, 8, 128, 16
    q, k, v = case.query.to(dev), case.key.to(dev), case.value.to(dev)
    cos, sin = rope_tables(4096, d, 500000.0, dev)
    pos = torch.arange(s, dtype=torch.int32, device=dev).view(b, s)
    nb = s // bs + 8
    g = torch.Generator().manual_seed(44)
    blocks = torch.randperm(nb, generator=g)[: s // bs].to(torch.int64)
    t = torch.arange(s)
    slots = (blocks[t // bs] * bs + t % bs).to(torch.int32).to(dev)
    kc = torch.zeros(nb, bs, hkv, d, dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    qk_bytes = (q.numel() + k.numel()) * 2
    table_bytes = 2 * s * (d // 2) * 4 + s * 4
    kv_bytes = (k.numel() + v.numel()) * 2
    rope_b = 2 * qk_bytes + table_bytes
    store_b = 2 * kv_bytes + s * 4
    # fused: q read and written, k read, written in place and to its page,
    # v read and written to its page
    fused_b = 2 * q.numel() * 2 + 3 * k.numel() * 2 + 2 * v.numel() * 2 + table_bytes + s * 4
    out = {}
    for name, fn, nbytes in (
            ("rope_inplace", lambda: ops.rope_inplace(q, k, cos, sin, pos), rope_b),
            ("paged_kv_store", lambda: ops.paged_kv_store(k.view(s, hkv, d), v.view(s, hkv, d),
                                                          kc, vc, slots), store_b),
            ("rope_kv_store", lambda: rope_kv_store(q.view(s, hq, d), k.view(s, hkv, d),
                                                    v.view(s, hkv, d), kc, vc, cos, sin,
                                                    pos.view(-1), slots), fused_b)):
        ms = time_graph_batch(fn)
        eager_ms = time_gpu(fn, steps, warmup, rounds=5)
        out[name] = {"us": round(ms * 1e3, 2), "bytes": int(nbytes),
                     "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "eager_us": round(eager_ms * 1e3, 2)}
        log(f"cfg3 {name}: {out[name]['us']} us, {out[name]['gbs']} GB/s")
    return out


def bench_norms(dev, steps: int, warmup: int, compiled: bool = False) -> dict:
    """RMSNorm and SwiGLU, the reference's only ops with published kernel figures
    (rmsnorm_report.txt:2-12: 811.84 us, 88.67 % of DRAM for 8 x 2048 x 4096 fp16).
    RMSNorm at the reference harness shape (tests/test_ops.py:17-61:
    [8, 2048, 4096] fp16, eps 1e-5) and at cfg5's prefill rows (8 x 512 tokens x
    3072); SwiGLU at cfg5's prefill gate_up [4096, 16384] -> [4096, 8192].  Each
    timed as 20 calls captured in one hipGraph and replayed (`us`; the Python
    call of an op takes longer than the few-microsecond kernels, so eager
    back-to-back calls measure the host; `eager_us` reports them too), beside
    what the reference compares with on the same GPU, timed the same way:
    torch's fused F.rms_norm (nn.RMSNorm) and the unfused formula, F.silu(g) * u
    for SwiGLU, and with `compiled` torch.compile of the unfused RMSNorm (a
    Triton kernel; --only norms; timed eagerly if its capture fails).
    Algorithmic bytes: the input read once, the output written once, plus the
    weight row.  `us` (and the rates) cycle each graph's calls through copies
    of the input totalling at least 512 MB, twice the 256 MB infinity cache,
    so every call reads its input from HBM; `us_cache_resident` repeats one
    input, which then stays in the infinity cache (as a layer's activations
    just written by the previous kernel do)."""
    import itertools
    import my_cuda_engine_cpp as ops
    g = torch.Generator(device=dev).manual_seed(48)
    out = {}

    def copy_ref(rot, like, gbs):
        """A device-to-device copy of the input (torch's copy_ from the same
        rotated inputs into one buffer), timed the same way: the read-plus-
        write rate HBM gives a plain streaming copy, beside the op's own rate."""
        dst = torch.empty_like(like)
        cms = time_graph_batch(lambda: dst.copy_(next(rot)))
        cgbs = 2 * dst.numel() * dst.element_size() / (cms * 1e-3) / 1e9
        return {"copy_us": round(cms * 1e3, 2), "copy_gbs": round(cgbs, 1),
                "rate_vs_copy": round(gbs / cgbs, 3)}

    def copies(t):  # the input and enough copies to exceed the infinity cache twice
        n = max(1, -(-(512 << 20) // (t.numel() * t.element_size())))
        return [t] + [t.clone() for _ in range(n - 1)]

    def rate(nbytes, ms):
        gbs = nbytes / (ms * 1e-3) / 1e9
        return {"us": round(ms * 1e3, 2), "gbs": round(gbs, 1),
                "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}

    for name, shape in (("rmsnorm_ref_harness", (8, 2048, 4096)), ("rmsnorm_cfg5_prefill",
                                                                   (8, 512, 3072))):
        h = shape[-1]
        x = torch.randn(*shape, generator=g, device=dev).half()
        w = (1.0 + 0.1 * torch.randn(h, generator=g, device=dev)).half()
        nbytes = 2 * x.numel() * 2 + h * 2
        xs = copies(x)
        rot = itertools.cycle(xs)
        ms = time_graph_batch(lambda: ops.rmsnorm(next(rot), w, 1e-5))
        row = {"shape": list(shape), "bytes": nbytes, **rate(nbytes, ms), "input_copies": len(xs),
               "us_cache_resident": round(time_graph_batch(lambda: ops.rmsnorm(x, w, 1e-5)) * 1e3, 2),
               "eager_us": round(time_gpu(lambda: ops.rmsnorm(x, w, 1e-5), steps, warmup) * 1e3, 2)}
        row.update(copy_ref(rot, x, row["gbs"]))
        nms = time_graph_batch(lambda: torch.nn.functional.rms_norm(next(rot), (h,), w, 1e-5))
        row["torch_rms_norm_us"] = round(nms * 1e3, 2)
        row["speedup_vs_torch_rms_norm"] = round(nms / ms, 2)

        def unfused(x_):
            return x_ * torch.rsqrt(x_.pow(2).mean(-1, keepdim=True) + 1e-5) * w
        ums = time_graph_batch(lambda: unfused(next(rot)))
        row["unfused_us"] = round(ums * 1e3, 2)
        if compiled:
            try:
                cfn = torch.compile(unfused)
                cfn(x)
                try:
                    cms = time_graph_batch(lambda: cfn(next(rot)))
                    row["torch_compile_timing"] = "hipGraph of 20 calls"
                except Exception:  # capture refused: time it eagerly
                    torch.cuda.synchronize()
                    cms = time_gpu(lambda: cfn(next(rot)), steps, warmup)
                    row["torch_compile_timing"] = "eager calls"
                row["torch_compile_us"] = round(cms * 1e3, 2)
                row["speedup_vs_torch_compile"] = round(cms / ms, 2)
            except Exception as e:  # no working compiler backend on this box
                row["torch_compile_error"] = str(e)[:200]
        out[name] = row
        log(f"{name}: {row['us']} us ({row['gbs']} GB/s; {row['us_cache_resident']} us cache-resident); "
            f"torch rms_norm {row['torch_rms_norm_us']} us")
        del x, xs, rot
    t, inter = 4096, 8192
    gu = torch.randn(t, 2 * inter, generator=g, device=dev).half()
    nbytes = gu.numel() * 2 + t * inter * 2
    gus = copies(gu)
    rot = itertools.cycle(gus)
    ms = time_graph_batch(lambda: ops.swiglu(next(rot)))
    row = {"shape": [t, 2 * inter], "bytes": nbytes, **rate(nbytes, ms), "input_copies": len(gus),
           "us_cache_resident": round(time_graph_batch(lambda: ops.swiglu(gu)) * 1e3, 2),
           "eager_us": round(time_gpu(lambda: ops.swiglu(gu), steps, warmup) * 1e3, 2)}
    row.update(copy_ref(rot, gu, row["gbs"]))

    def silu_mul(x_):
        return torch.nn.functional.silu(x_[:, :inter]) * x_[:, inter:]
    tms = time_graph_batch(lambda: silu_mul(next(rot)))
    row["torch_silu_mul_us"] = round(tms * 1e3, 2)
    row["speedup_vs_torch"] = round(tms / ms, 2)
    out["swiglu_cfg5_prefill"] = row
    log(f"swiglu: {row['us']} us ({row['gbs']} GB/s; {row['us_cache_resident']} us cache-resident); "
        f"torch silu*up {row['torch_silu_mul_us']} us")
    del gu, gus, rot
    return out


def bench_harness(dev, steps: int, warmup: int) -> dict:
    """The reference's decode harness shape (tests/test_paged_attention.py:12-125):
    B=16, Hq = Hkv = 32, D=128, ctx 2048, 16-token blocks from KVCacheManager
    (contiguous ascending tables), fp16 ~ N(0, 1).  paged_attention_decode is
    timed beside torch.nn.functional.scaled_dot_product_attention on
    contiguous [B, H, ctx, D] copies of the same K/V (the reference's
    comparison, README.md:6), both with HIP events over back-to-back calls;
    GB/s over the same algorithmic bytes (K and V once, q and out)."""
    import my_cuda_engine_cpp as ops
    from mycustomcudaengine_amd.engine.cache import KVCacheManager
    b, h, d, ctx, bs = 16, 32, 128, 2048, 16
    mgr = KVCacheManager(num_blocks=b * ctx // bs, block_size=bs, num_layers=1, num_heads=h,
                         head_dim=d, device=dev)
    for i in range(b):
        mgr.allocate_sequence(i, ctx)
    g = torch.Generator(device=dev).manual_seed(42)
    mgr.kv_cache.normal_(generator=g)
    q = torch.randn(b, h, d, generator=g, device=dev).half()
    bt = mgr.get_block_table_tensor(list(range(b)), ctx // bs)
    cl = torch.full((b,), ctx, dtype=torch.int32, device=dev)
    kc, vc = mgr.kv_cache[0, 0], mgr.kv_cache[0, 1]
    scale = d ** -0.5
    nbytes = 2 * b * ctx * h * d * 2 + 2 * b * h * d * 2
    ms = time_gpu(lambda: ops.paged_attention_decode(q, kc, vc, bt, cl, ctx // bs, bs, scale),
                  steps, warmup, rounds=5)
    out = {"workload": "reference decode harness: B=16, 32/32 heads, D=128, ctx 2048, "
                       "ascending tables, fp16",
           "us": round(ms * 1e3, 2), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
           "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    k = kc.view(b, ctx, h, d).transpose(1, 2).contiguous()
    v = vc.view(b, ctx, h, d).transpose(1, 2).contiguous()
    q4 = q.unsqueeze(2).contiguous()
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        # fused backends only (no math fallback through batched GEMMs)
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            sms = time_gpu(lambda: torch.nn.functional.scaled_dot_product_attention(
                q4, k, v, scale=scale), steps, warmup, rounds=5)
        out["sdpa_us"] = round(sms * 1e3, 2)
        out["sdpa_gbs"] = round(nbytes / (sms * 1e-3) / 1e9, 1)
        out["speedup_vs_sdpa"] = round(sms / ms, 3)
    except RuntimeError as e:  # no fused SDPA backend for this shape on this build
        out["sdpa_us"] = None
        out["sdpa_error"] = str(e)[:200]
    log(f"reference harness: {out['us']} us ({out['gbs']} GB/s); SDPA {out.get('sdpa_us')} us")
    del mgr, k, v
    return out


def bench_prefill_vs_sdpa(dev, steps: int) -> list:
    """The reference's prefill benchmark (benchmarks/benchmark_prefill_attn.py:6-67): B=1,
    24 / 8 heads, D=128, fp16 ~ N(0, 1), S = 128 .. 2048; prefill_attention timed beside
    torch.nn.functional.scaled_dot_product_attention(is_causal=True) on the K/V
    repeat-interleaved to 24 heads (its comparison), both with HIP events over back-to-back
    calls after MFMA_WARMUP_CALLS warm-up calls; TFLOP/s over the causal pairs.  At small S
    an eager Python call outlasts the kernel, so both are also timed as 20-call hipGraphs
    (`graph_us`, `sdpa_graph_us`): the kernels' own time per call."""
    import my_cuda_engine_cpp as ops
    from torch.nn.attention import SDPBackend, sdpa_kernel
    rows = []
    g = torch.Generator(device=dev).manual_seed(44)
    for s in (128, 256, 512, 1024, 2048):
        q = torch.randn(1, s, 24, 128, generator=g, device=dev).half()
        k = torch.randn(1, s, 8, 128, generator=g, device=dev).half()
        v = torch.randn(1, s, 8, 128, generator=g, device=dev).half()
        scale = 128 ** -0.5
        flops = 2 * 128 * 24 * s * (s + 1)
        ms = time_gpu(lambda: ops.prefill_attention(q, k, v, scale), steps, MFMA_WARMUP_CALLS,
                      rounds=3)
        row = {"seq_len": s, "us": round(ms * 1e3, 2),
               "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}
        gms = time_graph_batch(lambda: ops.prefill_attention(q, k, v, scale))
        row["graph_us"] = round(gms * 1e3, 2)
        qh = q.transpose(1, 2).contiguous()
        kh = k.transpose(1, 2).repeat_interleave(3, dim=1).contiguous()
        vh = v.transpose(1, 2).repeat_interleave(3, dim=1).contiguous()
        try:
            # fused backends only (no math fallback through batched GEMMs)
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                sms = time_gpu(lambda: torch.nn.functional.scaled_dot_product_attention(
                    qh, kh, vh, is_causal=True, scale=scale), steps, MFMA_WARMUP_CALLS, rounds=3)
            row["sdpa_us"] = round(sms * 1e3, 2)
            row["speedup_vs_sdpa"] = round(sms / ms, 2)
            try:
                with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                    sgms = time_graph_batch(lambda: torch.nn.functional.scaled_dot_product_attention(
                        qh, kh, vh, is_causal=True, scale=scale))
                row["sdpa_graph_us"] = round(sgms * 1e3, 2)
                row["speedup_vs_sdpa_graph"] = round(sgms / gms, 2)
            except RuntimeError as e:  # SDPA refused capture
                row["sdpa_graph_error"] = str(e)[:200]
        except RuntimeError as e:  # no fused SDPA backend on this build
            row["sdpa_us"] = None
            row["sdpa_error"] = str(e)[:200]
        rows.append(row)
        log(f"prefill S={s}: {row['us']} us ({row['tflops']} TFLOP/s), {row['graph_us']} us in a graph; "
            f"SDPA {row.get('sdpa_us')} us, {row.get('sdpa_graph_us')} us in a graph")
    return rows


def bench_ceilings(dev, steps: int = 20) -> dict:
    """Measured ceilings of this GPU, reported beside the published peaks as
    context (the roofline denominators stay the published 8 TB/s and 2.5
    PFLOP/s): a 1 GiB device-to-device copy (read + write bytes) and a
    library fp16 GEMM (torch.matmul -> hipBLASLt, 8192^3, fp32 accumulate)."""
    out = {}
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    ms = time_gpu(lambda: dst.copy_(src), steps, 60)  # ~25 ms of warm-up
    out["copy"] = {"bytes": 2 * n, "us": round(ms * 1e3, 2),
                   "gbs": round(2 * n / (ms * 1e-3) / 1e9, 1),
                   "frac_of_hbm_peak": round(2 * n / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    del src, dst
    m = 8192
    g = torch.Generator(device=dev).manual_seed(9)
    a = torch.randn(m, m, generator=g, device=dev).half()
    b = torch.randn(m, m, generator=g, device=dev).half()
    ms = time_gpu(lambda: torch.matmul(a, b), steps, 30)
    tf = 2 * m ** 3 / (ms * 1e-3) / 1e12
    out["gemm_fp16"] = {"shape": [m, m, m], "us": round(ms * 1e3, 2), "tflops": round(tf, 1),
                        "frac_of_fp16_dense_peak": round(tf / FP16_DENSE_TFLOPS, 4)}
    del a, b
    torch.cuda.empty_cache()
    log(f"ceilings: copy {out['copy']['gbs']} GB/s, fp16 GEMM {out['gemm_fp16']['tflops']} TFLOP/s")
    return out


def bench_chunked(dev, steps: int, warmup: int) -> dict:
    """Chunked prefill attention from the page pool (ops.prefill_attention_paged):
    synthetic fp16 Q/K/V ~ N(0, 1), 24/8 heads, 16-token pages in a shuffled
    pool, every sequence's chunk behind `prefix` cached tokens; timed with the
    key split allowed (split_keys=True) and not.  Algorithmic FLOPs: QK^T and
    PV over the causal pairs, 4 * D * Hq * sum_i (prefix + i + 1) per sequence."""
    from mycustomcudaengine_amd.ops import prefill_attention_paged
    g = torch.Generator(device=dev).manual_seed(47)
    out = {}
    for b, prefix, s in ((1, 0, 512), (1, 1536, 512), (1, 3584, 512), (1, 7680, 512),
                         (4, 2048, 128)):
        ctx, bs, hq, hkv, d = prefix + s, 16, 24, 8, 128
        width = (ctx + bs - 1) // bs
        nb = b * width
        kc = torch.randn(nb, bs, hkv, d, generator=g, device=dev).half()
        vc = torch.randn(nb, bs, hkv, d, generator=g, device=dev).half()
        table = torch.randperm(nb, generator=g, device=dev).view(b, width).to(torch.int32)
        q = torch.randn(b, s, hq, d, generator=g, device=dev).half()
        cl = torch.full((b,), ctx, dtype=torch.int32, device=dev)
        flops = 4 * d * hq * b * sum(prefix + i + 1 for i in range(s))
        row = {}
        for split in (True, False):
            ms = time_gpu(lambda: prefill_attention_paged(q, kc, vc, table, cl, d ** -0.5,
                                                          split_keys=split), steps, warmup,
                          rounds=5)
            row["split" if split else "whole"] = {"us": round(ms * 1e3, 2),
                                                  "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}
        key = f"B{b}_prefix{prefix}_chunk{s}"
        out[key] = row
        log(f"chunked {key}: key split {row['split']['us']} us, whole {row['whole']['us']} us")
        del kc, vc, q
    return out


def bench_model(dev, steps: int = 128, batch: int = 8, prompt: int = 512, seed: int = 46,
                cpu: bool = True) -> dict:
    """cfg5: random-init Llama-3.2-3B (28 layers, fp16 weights ~ N(0, 0.02),
    RMSNorm weights 1, tied lm_head), B=8 prefill of 512 uniform-random token
    ids, then `steps` greedy decode steps replayed through the hipGraph runner.
    tok/s = B * steps / wall time of the decode loop: the captured step also
    takes the greedy token and prepares the next step's positions and slots on
    the device, so the loop is `steps` back-to-back replays.  The same steps
    prepared on the host before every replay (the reference's loop shape:
    slots/tables copied in, argmax between replays) are reported as
    tok_s_host_prepared."""
    from mycustomcudaengine_amd.engine import (CUDAGraphRunner, KVCacheManager, Llama3BConfig,
                                               Llama3BEngineModel, prefill_step)
    cfg = Llama3BConfig({})
    g = torch.Generator(device=dev).manual_seed(seed)
    h, inter, d = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
    hq, hkv = cfg.num_attention_heads, cfg.num_key_value_heads

    def rnd(*shape):
        return (torch.randn(*shape, generator=g, device=dev, dtype=torch.float32) * 0.02).half()

    w = {"model.embed_tokens.weight": rnd(cfg.vocab_size, h),
         "model.norm.weight": torch.ones(h, dtype=torch.float16, device=dev)}
    for l in range(cfg.num_hidden_layers):
        p = f"model.layers.{l}"
        w[f"{p}.input_layernorm.weight"] = torch.ones(h, dtype=torch.float16, device=dev)
        w[f"{p}.post_attention_layernorm.weight"] = torch.ones(h, dtype=torch.float16, device=dev)
        w[f"{p}.self_attn.q_proj.weight"] = rnd(hq * d, h)
        w[f"{p}.self_attn.k_proj.weight"] = rnd(hkv * d, h)
        w[f"{p}.self_attn.v_proj.weight"] = rnd(hkv * d, h)
        w[f"{p}.self_attn.o_proj.weight"] = rnd(h, hq * d)
        w[f"{p}.mlp.gate_proj.weight"] = rnd(inter, h)
        w[f"{p}.mlp.up_proj.weight"] = rnd(inter, h)
        w[f"{p}.mlp.down_proj.weight"] = rnd(h, inter)
    weight_bytes = sum(t.numel() * t.element_size() for t in w.values())
    total = prompt + 8 + 2 * steps + 2
    blocks_per_seq = (total + 15) // 16
    cache = KVCacheManager(batch * blocks_per_seq + 16, 16, cfg.num_hidden_layers, hkv, d,
                           device=dev)
    model = Llama3BEngineModel(cfg, w, cache)
    seq = list(range(batch))
    for s in seq:
        cache.allocate_sequence(s, total)
    ids = torch.randint(0, cfg.vocab_size, (batch, prompt), generator=g, device=dev)
    prefill_step(model, ids, seq)  # warm-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits = prefill_step(model, ids, seq)
    torch.cuda.synchronize()
    ttft_ms = (time.perf_counter() - t0) * 1e3
    tok = logits.argmax(-1, keepdim=True)
    runner = CUDAGraphRunner(model, max_batch_size=batch)
    runner.capture_graph(tok, torch.full((batch, 1), prompt, dtype=torch.int32, device=dev), seq,
                         [prompt + 1] * batch, device_steps=steps)
    pos_buf = torch.empty((batch, 1), dtype=torch.int32, device=dev)
    # per-step latency with a sync around each step (the reference's ITL)
    itl = []
    for i in range(8):
        p = prompt + i
        pos_buf.fill_(p)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        out = runner.execute(tok, pos_buf, seq, [p + 1] * batch)
        torch.cuda.synchronize()
        itl.append((time.perf_counter() - t1) * 1e3)
        tok = out.argmax(-1, keepdim=True)
    # host-prepared loop: slots / tables prepared on the host before each replay
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for i in range(steps):
        p = prompt + 8 + i
        pos_buf.fill_(p)
        out = runner.execute(tok, pos_buf, seq, [p + 1] * batch)
        tok = out.argmax(-1, keepdim=True)
    torch.cuda.synchronize()
    host_s = time.perf_counter() - t1
    # throughput: `steps` back-to-back replays, each preparing the next on the device
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    runner.run_device_loop(steps)
    torch.cuda.synchronize()
    loop_s = time.perf_counter() - t1
    step_ms = loop_s / steps * 1e3
    mean_ctx = prompt + 8 + steps + steps / 2  # positions of the timed device loop
    kv_bytes = batch * mean_ctx * cfg.num_hidden_layers * hkv * d * 2 * 2
    cpu_base = None
    if cpu:
        del runner, cache
        torch.cuda.empty_cache()
        cpu_base = cpu_baseline_model(cfg, w, ids.cpu())
    return {"workload": "cfg5 Llama-3.2-3B random-init fp16, B=8, prefill 512, "
                        f"{steps} greedy decode steps replayed via hipGraph",
            "tok_s": round(batch * steps / loop_s, 1),
            "tok_s_host_prepared": round(batch * steps / host_s, 1),
            "steps_per_s": round(steps / loop_s, 2),
            "ms_per_step": round(step_ms, 4),
            "itl_ms_synced": round(sorted(itl)[len(itl) // 2], 4),
            "ttft_ms": round(ttft_ms, 2),
            "bytes_per_step": int(weight_bytes + kv_bytes),
            "gbs": round((weight_bytes + kv_bytes) / (step_ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round((weight_bytes + kv_bytes) / (step_ms * 1e-3) / 1e9
                                      / HBM_PEAK_GBS, 4),
            "cpu_baseline": cpu_base}


def cpu_baseline_model(cfg, weights: dict, ids: torch.Tensor, prompt: int = 512,
                       steps: int = 4) -> dict:
    """A bounded cfg5 sample on the CPU, on the planned workload
    (benchmarks/benchmark_engine.py:226-268): the fp32 model oracle
    (oracle/model_ref.py) with the benchmark's own weights (copied to the host
    as fp32) prefills the benchmark's 8 prompts of `prompt` tokens, then takes
    `steps` greedy decode steps at positions prompt .. prompt + steps - 1, so
    each step pays attention over cfg5's context as the GPU steps do.  value =
    decode tokens/s (8 sequences x steps over the decode wall time); the
    prefill time is reported beside it."""
    from oracle.model_ref import LlamaRef
    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    hf = dict(hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
              num_hidden_layers=cfg.num_hidden_layers,
              num_attention_heads=cfg.num_attention_heads,
              num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
              vocab_size=cfg.vocab_size, rms_norm_eps=cfg.rms_norm_eps, rope_theta=cfg.rope_theta)
    names = [k for k in weights if not k.startswith("lm_head")]
    ref = LlamaRef(hf, {k: weights[k] for k in names})
    b = ids.shape[0]
    seq = list(range(b))
    t0 = time.perf_counter()
    logits = ref.prefill(ids[:, :prompt], seq)
    prefill_s = time.perf_counter() - t0
    tok = logits.argmax(-1, keepdim=True)
    t0 = time.perf_counter()
    for i in range(steps):
        logits = ref.decode(tok, [prompt + i] * b, seq)
        tok = logits.argmax(-1, keepdim=True)
    decode_s = time.perf_counter() - t0
    info = cpu_info()
    return {"value": round(b * steps / decode_s, 3), "unit": "tok/s", "cores": n, "kind": "port",
            "prompt": prompt, "decode_steps": steps,
            "prefill_ms": round(prefill_s * 1e3, 1),
            "ms_per_step": round(decode_s / steps * 1e3, 1),
            "sample": f"cfg5 geometry with the benchmark's weights, fp32 torch model oracle: "
                      f"B={b} prefill of prompt {prompt} ({prefill_s * 1e3:.0f} ms), then "
                      f"k={steps} greedy decode steps ({decode_s / steps * 1e3:.0f} ms/step, "
                      f"positions {prompt}-{prompt + steps - 1}); {info['cpu_model']}; "
                      f"torch {info['torch']}"}


def cpu_baseline_decode(case) -> dict:
    """The CPU oracle (fp32, torch on this host's cores) on the same inputs."""
    from oracle.ops_ref import decode_attention_ref
    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    args = (case.query, case.key_cache, case.value_cache, case.block_tables,
            case.context_lens, case.scale)
    for _ in range(2):
        decode_attention_ref(*args)
    times = []
    t_end = time.perf_counter() + 20.0
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        decode_attention_ref(*args)
        times.append(time.perf_counter() - t0)
        if len(times) >= 5 and time.perf_counter() > t_end:
            break
    times.sort()
    med = times[len(times) // 2]
    gbs = case.algorithmic_bytes() / med / 1e9
    info = cpu_info()
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": n, "kind": "port",
            "sample": f"full cfg2 batch (32 seqs, {int(case.context_lens.sum())} tokens), "
                      f"fp32 torch oracle, median of {len(times)} runs after 2 warmups, "
                      f"{med * 1e3:.1f} ms/run; {info['cpu_model']}; torch {info['torch']}"}


def cpu_median_s(fn, runs: int = 3, warmup: int = 1) -> tuple:
    """Median wall seconds of `runs` calls of a CPU oracle function (after
    `warmup` calls), on all of this host's cores."""
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_baseline_prefill(case) -> dict:
    """cfg3 on the CPU: the fp32 causal-attention oracle on the same inputs."""
    from oracle.ops_ref import prefill_attention_ref
    med, n = cpu_median_s(lambda: prefill_attention_ref(case.query, case.key, case.value,
                                                        case.scale))
    info = cpu_info()
    return {"value": round(case.algorithmic_flops() / med / 1e12, 4), "unit": "TFLOP/s",
            "cores": len(os.sched_getaffinity(0)), "kind": "port",
            "sample": f"full cfg3 (B=1, S=2048), fp32 torch oracle, median of {n} runs after "
                      f"1 warmup, {med * 1e3:.1f} ms/run; {info['cpu_model']}; "
                      f"torch {info['torch']}"}


def cpu_baseline_splitk(case) -> dict:
    """cfg4 on the CPU: the fp32 decode-attention oracle on the same inputs."""
    from oracle.ops_ref import decode_attention_ref
    med, n = cpu_median_s(lambda: decode_attention_ref(
        case.query, case.key_cache, case.value_cache, case.block_tables, case.context_lens,
        case.scale))
    info = cpu_info()
    return {"value": round(case.algorithmic_bytes() / med / 1e9, 3), "unit": "GB/s",
            "cores": len(os.sched_getaffinity(0)), "kind": "port",
            "sample": f"full cfg4 (B=8, ctx 32768), fp32 torch oracle, median of {n} runs after "
                      f"1 warmup, {med * 1e3:.1f} ms/run; {info['cpu_model']}; "
                      f"torch {info['torch']}"}


def source_sha(path: str = DECODE_SOURCE) -> str:
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def measured_traffic():
    """HBM bytes per decode-kernel launch from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE passes (calibrated against a 256 MiB copy), or None
    when that summary is absent or was collected on another version of the
    decode kernel source (its recorded sha256 prefix differs)."""
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)
        if rec.get("decode_source_sha16") != source_sha():
            return None
        return int(rec["traffic_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", choices=["decode", "prefill", "legs", "splitk", "harness", "norms",
                                       "model", "chunked", "ceilings"],
                    default=None)
    ap.add_argument("--calibration-copy", action="store_true",
                    help="first copy 256 MiB device-to-device (a kernel of known traffic, "
                         "used to scale rocprofv3 FETCH_SIZE/WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not "
              "supported (the hot path's multi-GPU sharding is a design note, not built)",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from mycustomcudaengine_amd import _lib
    _lib.load()
    from oracle.inputs import cfg2_decode, cfg3_prefill, cfg4_decode

    dev = torch.device("cuda:0")
    if args.calibration_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    result = {}
    case2 = None
    if args.only in (None, "decode"):
        log("generating cfg2 inputs")
        case2 = cfg2_decode()
        ms, nbytes, gbs, graph_ms, warm2 = bench_decode(case2, dev, args.steps, args.warmup)
        log(f"cfg2 decode: {ms * 1e3:.1f} us/step ({gbs:.1f} GB/s); in a 20-call hipGraph "
            f"{graph_ms * 1e3:.1f} us/step")
        result["decode"] = (ms, nbytes, gbs, graph_ms, warm2)

    extra = {}
    if args.only in (None, "prefill"):
        log("cfg3 prefill")
        case3 = cfg3_prefill()
        pms, flops, tfs, pgms = bench_prefill(case3, dev, max(20, args.steps // 4), 5)
        log(f"cfg3 prefill: {pms * 1e3:.1f} us, {tfs:.1f} TFLOP/s; in a 20-call hipGraph "
            f"{pgms * 1e3:.1f} us")
        extra["prefill"] = {"workload": "cfg3 causal prefill B=1 S=2048 24/8 heads D=128 fp16",
                            "us": round(pms * 1e3, 2), "flop": flops,
                            "tflops": round(tfs, 2),
                            "frac_of_fp16_dense_peak": round(tfs / FP16_DENSE_TFLOPS, 4),
                            "timing": f"back-to-back eager calls after {MFMA_WARMUP_CALLS} "
                                      "warm-up calls, HIP events",
                            "graph_us_per_call": round(pgms * 1e3, 2)}
        extra["prefill"]["legs"] = bench_prefill_legs(case3, dev, max(20, args.steps // 4), 5)
        extra["prefill"]["vs_sdpa"] = bench_prefill_vs_sdpa(dev, max(20, args.steps // 4))
        torch.cuda.empty_cache()
        if not args.no_cpu:
            extra["prefill"]["cpu_baseline"] = cpu_baseline_prefill(case3)
            log(f"cfg3 CPU baseline: {extra['prefill']['cpu_baseline']['value']} TFLOP/s")
        del case3
    # the ceilings right after the two headline kernels, under the same
    # conditions (before the long legs warm the part)
    if args.only in (None, "ceilings"):
        extra["measured_ceilings"] = bench_ceilings(dev)
        c = extra["measured_ceilings"]
        if "decode" in result:
            c["decode_frac_of_copy"] = round(result["decode"][2] / c["copy"]["gbs"], 4)
        if "prefill" in extra:
            c["prefill_frac_of_gemm"] = round(extra["prefill"]["tflops"] / c["gemm_fp16"]["tflops"], 4)
    if args.only == "legs":
        extra["legs"] = bench_prefill_legs(cfg3_prefill(), dev, max(20, args.steps // 4), 5)
    if args.only in (None, "splitk"):
        log("generating cfg4 inputs")
        case4 = cfg4_decode()
        kms, kbytes, kgbs, _, _ = bench_decode(case4, dev, max(20, args.steps // 4), 5, rounds=5)
        log(f"cfg4 split-K decode: {kms * 1e3:.1f} us, {kgbs:.1f} GB/s")
        extra["splitk"] = {"workload": "cfg4 paged decode B=8 ctx=32768 24/8 heads D=128",
                           "us": round(kms * 1e3, 2), "bytes": kbytes,
                           "gbs": round(kgbs, 1), "frac_of_hbm_peak": round(kgbs / HBM_PEAK_GBS, 4)}
        if not args.no_cpu:
            extra["splitk"]["cpu_baseline"] = cpu_baseline_splitk(case4)
            log(f"cfg4 CPU baseline: {extra['splitk']['cpu_baseline']['value']} GB/s")
        del case4
        torch.cuda.empty_cache()

    if args.only in (None, "harness"):
        extra["ref_harness"] = bench_harness(dev, max(20, args.steps // 4), 5)
        torch.cuda.empty_cache()

    if args.only in (None, "norms"):
        extra["norms"] = bench_norms(dev, max(20, args.steps // 4), 20,
                                     compiled=args.only == "norms")
        torch.cuda.empty_cache()

    if args.only in (None, "model"):
        log("cfg5 Llama-3.2-3B decode")
        extra["model"] = bench_model(dev, cpu=not args.no_cpu)
        if extra["model"]["cpu_baseline"]:
            log(f"cfg5 CPU baseline: {extra['model']['cpu_baseline']['value']} tok/s")
        log(f"cfg5 model: {extra['model']['tok_s']} tok/s, {extra['model']['ms_per_step']} ms/step "
            f"(host-prepared steps: {extra['model']['tok_s_host_prepared']} tok/s)")
        torch.cuda.empty_cache()
        # the reference's own engine benchmark shape: one sequence
        # (benchmarks/benchmark_engine.py:198-271: TTFT, inter-token latency, tok/s)
        m1 = bench_model(dev, batch=1, cpu=False)
        m1["workload"] = ("reference engine benchmark shape: Llama-3.2-3B random-init fp16, B=1, "
                          "prefill 512, 128 greedy decode steps replayed via hipGraph")
        extra["model_b1"] = m1
        log(f"B=1 model: TTFT {m1['ttft_ms']} ms, ITL {m1['itl_ms_synced']} ms, {m1['tok_s']} tok/s "
            f"(host-prepared steps: {m1['tok_s_host_prepared']} tok/s)")
        torch.cuda.empty_cache()

    if args.only == "chunked":
        extra["chunked"] = bench_chunked(dev, max(20, args.steps // 4), 5)

    if "decode" not in result:  # a single non-headline workload was asked for
        print(json.dumps({"metric": METRIC, "only": args.only, **extra}), flush=True)
        return

    cpu = None
    if not args.no_cpu:
        log("CPU baseline (oracle on host cores)")
        cpu = cpu_baseline_decode(case2)
        log(f"CPU baseline: {cpu['value']} GB/s on {cpu['cores']} cores")

    ms, nbytes, gbs, graph_ms, warm2 = result["decode"]
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "cfg2 paged decode attention: B=32, ctx~U[128,4096] (seed 43), "
                               "24 Q / 8 KV heads, D=128, 16-token pages, shuffled tables",
                   "batch": 32, "tokens": int(case2.context_lens.sum()),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic()},
        "cpu_baseline": cpu,
        "timing": {"method": "K back-to-back op calls from Python (decode kernel + LSE "
                             "merge kernel each), HIP events on the launch stream, after "
                             f"{warm2} warm-up calls (W, and at least {DECODE_WARMUP_MS:.0f} ms "
                             f"of calls); the median of 5 windows of K calls, each behind "
                             f"{LEAD_CALLS} queued untimed calls",
                   "warmup_calls": warm2, "windows": 5, "lead_calls": LEAD_CALLS,
                   "graph_us_per_step": round(graph_ms * 1e3, 2),
                   "graph": "20 op calls captured in one hipGraph, replayed; per call",
                   "algorithmic_bytes_per_step": nbytes},
        **extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
