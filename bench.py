"""Benchmark of the attention hot path on one MI355X.

Headline (`value`): paged decode attention at cfg2 (B=32, ctx ~ U[128, 4096],
24/8 heads, D=128, 16-token pages, shuffled block tables) in algorithmic HBM
GB/s: every K/V byte once, q and out once, the block-table entries used.
One "step" = one paged_attention_decode call over the whole batch, inputs
resident in HBM.  Timed with HIP events on the launch stream over K
back-to-back calls (the same op captured in a hipGraph and replayed is timed
too and reported beside it).

Extra fields on the same JSON line:
  prefill   cfg3 causal prefill (S=2048, 24/8 heads): algorithmic TFLOP/s
            (2 * D * Hq * S * (S+1)) and fraction of dense fp16 MFMA peak.
  splitk    cfg4 long-context decode (B=8, ctx 32768): GB/s.
  model     cfg5 Llama-3.2-3B random-init, B=8, prefill 512 then 128 greedy
            decode steps replayed via hipGraph: tok/s, ms/step, TTFT.
  cpu_baseline  the CPU oracle on the same cfg2 inputs, on this host's cores
            (prefill and splitk carry their own, on cfg3 / cfg4; cfg5 has none:
            an fp32 CPU forward of the 3B model is not a bounded sample).

  chunked   (--only chunked; not in the default run) chunked prefill from the
            page pool, B=1 chunk 512 behind 0-7680 cached tokens and B=4 chunk
            128 behind 2048, with and without the key split: us, TFLOP/s.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                       [--only decode|prefill|splitk|model|chunked]
(--only runs one workload; only the default run prints the full result line.)
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, vendor spec
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "decode_hbm_traffic.json")
FP16_DENSE_TFLOPS = 2500.0     # MI355X dense fp16 MFMA, vendor spec
METRIC = "decode-attn HBM GB/s (% peak); prefill-attn TFLOPS (% MFMA); 3B decode tok/s"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_gpu(fn, steps: int, warmup: int) -> float:
    """Average ms per call of fn(), issued eagerly from Python, measured with
    HIP events on the current stream (includes host launch overhead when the
    GPU work is shorter than the Python call)."""
    for _ in range(warmup):
        fn()
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def time_graph(fn, steps: int, warmup: int) -> float:
    """Average ms per call of fn() captured once in a hipGraph (torch.cuda.graph)
    and replayed `steps` times back to back; HIP events on the replay stream
    bracket the replays.  This is how the engine issues its decode step."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(max(1, warmup)):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    for _ in range(warmup):
        graph.replay()
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        graph.replay()
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


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


def bench_decode(case, dev, steps, warmup):
    import my_cuda_engine_cpp as ops
    q = case.query.to(dev)
    kc, vc = case.key_cache.to(dev), case.value_cache.to(dev)
    bt, cl = case.block_tables.to(dev), case.context_lens.to(dev)
    fn = lambda: ops.paged_attention_decode(q, kc, vc, bt, cl, case.max_blocks,
                                            case.block_size, case.scale)
    ms = time_gpu(fn, steps, warmup)
    graph_ms = time_graph(fn, steps, warmup)
    nbytes = case.algorithmic_bytes()
    return ms, nbytes, nbytes / (ms * 1e-3) / 1e9, graph_ms


def bench_prefill(case, dev, steps, warmup):
    """cfg3 causal prefill: back-to-back eager calls (one kernel each) timed
    with HIP events, plus the same call replayed from a captured hipGraph."""
    import my_cuda_engine_cpp as ops
    q, k, v = case.query.to(dev), case.key.to(dev), case.value.to(dev)
    fn = lambda: ops.prefill_attention(q, k, v, case.scale)
    ms = time_gpu(fn, steps, warmup)
    graph_ms = time_graph(fn, steps, warmup)
    flops = case.algorithmic_flops()
    return ms, flops, flops / (ms * 1e-3) / 1e12, graph_ms


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
                                                          split_keys=split), steps, warmup)
            row["split" if split else "whole"] = {"us": round(ms * 1e3, 2),
                                                  "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}
        key = f"B{b}_prefix{prefix}_chunk{s}"
        out[key] = row
        log(f"chunked {key}: key split {row['split']['us']} us, whole {row['whole']['us']} us")
        del kc, vc, q
    return out


def bench_model(dev, steps: int = 128, batch: int = 8, prompt: int = 512, seed: int = 46) -> dict:
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
                                      / HBM_PEAK_GBS, 4)}


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
    return {"value": round(case.algorithmic_flops() / med / 1e12, 4), "unit": "TFLOP/s",
            "cores": len(os.sched_getaffinity(0)), "kind": "port",
            "sample": f"full cfg3 (B=1, S=2048), fp32 torch oracle, median of {n} runs after "
                      f"1 warmup, {med * 1e3:.1f} ms/run"}


def cpu_baseline_splitk(case) -> dict:
    """cfg4 on the CPU: the fp32 decode-attention oracle on the same inputs."""
    from oracle.ops_ref import decode_attention_ref
    med, n = cpu_median_s(lambda: decode_attention_ref(
        case.query, case.key_cache, case.value_cache, case.block_tables, case.context_lens,
        case.scale))
    return {"value": round(case.algorithmic_bytes() / med / 1e9, 3), "unit": "GB/s",
            "cores": len(os.sched_getaffinity(0)), "kind": "port",
            "sample": f"full cfg4 (B=8, ctx 32768), fp32 torch oracle, median of {n} runs after "
                      f"1 warmup, {med * 1e3:.1f} ms/run"}


def measured_traffic():
    """HBM bytes per decode-kernel launch from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE passes (calibrated against a 256 MiB copy), or None
    when that summary is absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            return int(json.load(f)["traffic_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", choices=["decode", "prefill", "splitk", "model", "chunked"],
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
        ms, nbytes, gbs, graph_ms = bench_decode(case2, dev, args.steps, args.warmup)
        log(f"cfg2 decode: {ms * 1e3:.1f} us/step ({gbs:.1f} GB/s); as hipGraph replays "
            f"{graph_ms * 1e3:.1f} us/step")
        result["decode"] = (ms, nbytes, gbs, graph_ms)

    extra = {}
    if args.only in (None, "prefill"):
        log("cfg3 prefill")
        case3 = cfg3_prefill()
        pms, flops, tfs, pgms = bench_prefill(case3, dev, max(20, args.steps // 4), 5)
        log(f"cfg3 prefill: {pms * 1e3:.1f} us, {tfs:.1f} TFLOP/s; as hipGraph replays "
            f"{pgms * 1e3:.1f} us")
        extra["prefill"] = {"workload": "cfg3 causal prefill B=1 S=2048 24/8 heads D=128 fp16",
                            "us": round(pms * 1e3, 2), "flop": flops,
                            "tflops": round(tfs, 2),
                            "frac_of_fp16_dense_peak": round(tfs / FP16_DENSE_TFLOPS, 4),
                            "timing": "back-to-back eager calls, HIP events",
                            "graph_replay_us": round(pgms * 1e3, 2)}
        if not args.no_cpu:
            extra["prefill"]["cpu_baseline"] = cpu_baseline_prefill(case3)
            log(f"cfg3 CPU baseline: {extra['prefill']['cpu_baseline']['value']} TFLOP/s")
        del case3
    if args.only in (None, "splitk"):
        log("generating cfg4 inputs")
        case4 = cfg4_decode()
        kms, kbytes, kgbs, _ = bench_decode(case4, dev, max(20, args.steps // 4), 5)
        log(f"cfg4 split-K decode: {kms * 1e3:.1f} us, {kgbs:.1f} GB/s")
        extra["splitk"] = {"workload": "cfg4 paged decode B=8 ctx=32768 24/8 heads D=128",
                           "us": round(kms * 1e3, 2), "bytes": kbytes,
                           "gbs": round(kgbs, 1), "frac_of_hbm_peak": round(kgbs / HBM_PEAK_GBS, 4)}
        if not args.no_cpu:
            extra["splitk"]["cpu_baseline"] = cpu_baseline_splitk(case4)
            log(f"cfg4 CPU baseline: {extra['splitk']['cpu_baseline']['value']} GB/s")
        del case4
        torch.cuda.empty_cache()

    if args.only in (None, "model"):
        log("cfg5 Llama-3.2-3B decode")
        extra["model"] = bench_model(dev)
        log(f"cfg5 model: {extra['model']['tok_s']} tok/s, {extra['model']['ms_per_step']} ms/step "
            f"(host-prepared steps: {extra['model']['tok_s_host_prepared']} tok/s)")
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

    ms, nbytes, gbs, graph_ms = result["decode"]
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
                             "merge kernel each), HIP events on the launch stream",
                   "graph_replay_us_per_step": round(graph_ms * 1e3, 2),
                   "algorithmic_bytes_per_step": nbytes},
        **extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
