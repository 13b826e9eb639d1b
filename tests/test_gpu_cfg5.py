"""GPU: cfg5, the full Llama-3.2-3B geometry (28 layers, hidden 3072, 24/8
heads, SwiGLU 8192, vocab 128256), the workload of the reference's engine
benchmark (benchmarks/benchmark_engine.py:132-271).

  * full size through properties: random-init fp16 weights ~ N(0, 0.02),
    RMSNorm weights 1, tied lm_head, B=8, prefill of 512 tokens, a graph
    captured with 128 device steps; no NaN/Inf in any logits, and the 128
    greedy tokens of run_device_loop equal, exactly, those of the same steps
    prepared on the host (execute + torch.argmax, the reference's loop shape);
  * depth and vocabulary parity: the same geometry with non-unit norm weights,
    B=8, a 16-token prompt and two decode steps against the fp32 CPU model
    oracle (oracle/model_ref.py), within the engine tests' bar;
  * the lm_head launch at this shape: RMSNorm + [8, 3072] x [128256, 3072]^T
    (8016 workgroups) against fp32 torch.

Weights are drawn on the GPU from a seeded generator (3.2 B values) and, for
the oracle, copied to the host, so both sides see the same values.
"""
import pytest
import torch

from mycustomcudaengine_amd.engine import (CUDAGraphRunner, KVCacheManager, Llama3BConfig,
                                           Llama3BEngineModel, prefill_step)

pytestmark = pytest.mark.gpu


def random_weights(cfg: Llama3BConfig, dev, seed: int, norm_std: float = 0.0) -> dict:
    g = torch.Generator(device=dev).manual_seed(seed)
    h, inter, d = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
    hq, hkv = cfg.num_attention_heads, cfg.num_key_value_heads

    def rnd(*shape):
        return (torch.randn(*shape, generator=g, device=dev) * 0.02).half()

    def norm():
        w = torch.ones(h, device=dev)
        if norm_std:
            w += torch.randn(h, generator=g, device=dev) * norm_std
        return w.half()

    w = {"model.embed_tokens.weight": rnd(cfg.vocab_size, h), "model.norm.weight": norm()}
    for l in range(cfg.num_hidden_layers):
        p = f"model.layers.{l}"
        w[f"{p}.input_layernorm.weight"] = norm()
        w[f"{p}.post_attention_layernorm.weight"] = norm()
        w[f"{p}.self_attn.q_proj.weight"] = rnd(hq * d, h)
        w[f"{p}.self_attn.k_proj.weight"] = rnd(hkv * d, h)
        w[f"{p}.self_attn.v_proj.weight"] = rnd(hkv * d, h)
        w[f"{p}.self_attn.o_proj.weight"] = rnd(h, hq * d)
        w[f"{p}.mlp.gate_proj.weight"] = rnd(inter, h)
        w[f"{p}.mlp.up_proj.weight"] = rnd(inter, h)
        w[f"{p}.mlp.down_proj.weight"] = rnd(h, inter)
    return w


def test_cfg5_full_size_device_loop_equals_host_prepared_steps(dev):
    cfg = Llama3BConfig({})
    assert (cfg.num_hidden_layers, cfg.vocab_size) == (28, 128256)
    batch, prompt, steps = 8, 512, 128
    w = random_weights(cfg, dev, seed=46)
    cache = KVCacheManager(batch * ((prompt + steps + 2 + 15) // 16) + 16, 16,
                           cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim,
                           device=dev)
    model = Llama3BEngineModel(cfg, w, cache)
    seq = list(range(batch))
    for s in seq:
        cache.allocate_sequence(s, prompt + steps + 2)
    ids = torch.randint(0, cfg.vocab_size, (batch, prompt),
                        generator=torch.Generator(device=dev).manual_seed(47), device=dev)
    logits = prefill_step(model, ids, seq)
    assert torch.isfinite(logits).all()
    tok0 = logits.argmax(-1, keepdim=True)
    runner = CUDAGraphRunner(model, max_batch_size=batch)
    runner.capture_graph(tok0, torch.full((batch, 1), prompt, dtype=torch.int32, device=dev),
                         seq, [prompt + 1] * batch, device_steps=steps)
    dev_tokens = runner.run_device_loop(steps).clone()
    assert torch.isfinite(runner.static_logits).all()
    tok = tok0
    host_tokens = []
    finite = True
    for i in range(steps):
        p = prompt + i
        out = runner.execute(tok, torch.full((batch, 1), p, dtype=torch.int32, device=dev), seq,
                             [p + 1] * batch)
        finite &= bool(torch.isfinite(out).all())
        tok = out.argmax(-1, keepdim=True)
        host_tokens.append(tok.view(-1))
    assert finite
    assert dev_tokens.cpu().tolist() == torch.stack(host_tokens).cpu().tolist()
    # the greedy path actually moves (not one token repeated by every sequence)
    assert len(set(dev_tokens.view(-1).tolist())) > batch


def test_cfg5_depth_and_vocab_match_oracle(dev):
    from oracle.model_ref import LlamaRef
    cfg = Llama3BConfig({})
    batch, prompt = 8, 16
    w = random_weights(cfg, dev, seed=48, norm_std=0.1)
    w_cpu = {k: v.cpu() for k, v in w.items()}
    cache = KVCacheManager(batch * 2 + 8, 16, cfg.num_hidden_layers, cfg.num_key_value_heads,
                           cfg.head_dim, device=dev)
    model = Llama3BEngineModel(cfg, w, cache)
    seq = list(range(batch))
    for s in seq:
        cache.allocate_sequence(s, prompt + 2)
    ids = torch.randint(0, cfg.vocab_size, (batch, prompt), generator=torch.Generator().manual_seed(49))
    hf = dict(hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
              num_hidden_layers=cfg.num_hidden_layers, num_attention_heads=cfg.num_attention_heads,
              num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
              vocab_size=cfg.vocab_size, rms_norm_eps=cfg.rms_norm_eps,
              rope_theta=cfg.rope_theta)
    ref = LlamaRef(hf, w_cpu)
    del w_cpu

    def close(gpu, want, rel=1e-2, abs_=5e-2):
        g = gpu.float().cpu()
        err = ((g - want).norm() / want.norm()).item()
        mx = (g - want).abs().max().item()
        assert err <= rel and mx <= abs_, (err, mx)

    logits = prefill_step(model, ids.to(dev), seq)
    want = ref.prefill(ids, seq)
    close(logits, want)
    tok = want.argmax(-1, keepdim=True)
    for i in range(2):
        p = prompt + i
        slots = torch.from_numpy(cache.slot_mapping(seq, [p + 1] * batch)).to(dev)
        mb = len(cache.block_tables[0])
        out = model.decode_step(tok.to(dev), torch.full((batch, 1), p, dtype=torch.int32, device=dev),
                                torch.full((batch,), p + 1, dtype=torch.int32, device=dev), slots,
                                cache.get_block_table_tensor(seq, mb), mb)
        want = ref.decode(tok, [p] * batch, seq)
        close(out, want)
        tok = want.argmax(-1, keepdim=True)


def test_lm_head_rmsnorm_decode_gemm_at_vocab_128256(dev):
    """The decode step's last launch at cfg5: RMSNorm (non-unit weight) fused
    in front of the [128256, 3072] tied head for 8 tokens, against fp32 torch
    (|err| <= 2e-3 + 4e-3 |ref|, the bound of the other decode-GEMM shapes)."""
    from mycustomcudaengine_amd.ops import rmsnorm_decode_gemm
    g = torch.Generator().manual_seed(50)
    m, n, k, eps = 8, 128256, 3072, 1e-5
    x = (torch.randn(m, k, generator=g) * 3).half()
    nw = (1 + 0.1 * torch.randn(k, generator=g)).half()
    w = (torch.randn(n, k, generator=g) * 0.02).half()
    xn = x.float() / torch.sqrt(x.float().pow(2).mean(-1, keepdim=True) + eps) * nw.float()
    ref = xn @ w.float().T
    out = rmsnorm_decode_gemm(x.to(dev), nw.to(dev), eps, w.to(dev)).float().cpu()
    err = (out - ref).abs()
    assert (err <= 2e-3 + 4e-3 * ref.abs()).all(), err.max().item()


@pytest.mark.parametrize("m,k,norm", [(12, 3072, True), (5, 2048, False), (8, 4096, True),
                                      (16, 2048, False)])
def test_many_round_decode_gemm_matches_fp32(dev, m, k, norm):
    """Launches of many rounds of workgroups (N = 65536: 4096 workgroups of 16
    columns) take the 128-byte-row W loads with the fragments rebuilt through
    LDS; every token-slot count, K and the fused / plain RMSNorm against fp32
    torch (|err| <= 2e-3 + 4e-3 |ref|)."""
    from mycustomcudaengine_amd.ops import decode_gemm, rmsnorm_decode_gemm
    g = torch.Generator().manual_seed(51 + m + k)
    n, eps = 65536, 1e-5
    x = (torch.randn(m, k, generator=g) * 2).half()
    nw = (1 + 0.1 * torch.randn(k, generator=g)).half()
    w = (torch.randn(n, k, generator=g) * 0.02).half()
    xf = x.float()
    if norm:
        xf = xf / torch.sqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * nw.float()
        out = rmsnorm_decode_gemm(x.to(dev), nw.to(dev), eps, w.to(dev))
    else:
        out = decode_gemm(x.to(dev), w.to(dev))
    ref = xf @ w.float().T
    err = (out.float().cpu() - ref).abs()
    assert (err <= 2e-3 + 4e-3 * ref.abs()).all(), err.max().item()
