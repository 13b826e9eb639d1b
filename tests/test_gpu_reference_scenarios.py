"""GPU: the reference's own test scenarios at their shapes, through the
reference's module surface (my_cuda_engine_cpp) and engine classes.

  * tests/test_rope.py:35-57: B=16, S=1, 32 query / 8 key heads, theta
    10000, positions uniform in [0, 2048); allclose(1e-2, 1e-2) against the
    rotation with fp16-cast tables (the reference's pytorch_apply_rope,
    :14-32), and this build's own bar against the fp32 oracle;
  * tests/test_all_ops.py:42-65: rmsnorm, rope, the paged KV store, decode
    attention at context 1 and SwiGLU captured in one hipGraph, every replay
    equal to the eager calls (bit for bit: the same kernels), with eager work
    and synchronisations between the replays;
  * tests/test_cuda_graph.py:15-141: a 4-layer model of Llama-3.2-3B layer
    geometry, one sequence at context 100, graph-replayed decode steps
    against eager decode steps within allclose(1e-2, 1e-2) (:138), greedy
    tokens identical.
"""
import pytest
import torch

import my_cuda_engine_cpp as ops
from mycustomcudaengine_amd.engine import (CUDAGraphRunner, KVCacheManager, Llama3BConfig,
                                           Llama3BEngineModel, prefill_step)
from oracle.model_ref import random_llama_weights
from oracle.ops_ref import rope_ref, rope_tables

pytestmark = pytest.mark.gpu


def gen(seed):
    return torch.Generator().manual_seed(seed)


def test_rope_reference_test_shape(dev):
    b, s, hq, hkv, d = 16, 1, 32, 8, 128
    cos, sin = rope_tables(2048, d, 10000.0)
    q = torch.randn(b, s, hq, d, generator=gen(300)).half()
    k = torch.randn(b, s, hkv, d, generator=gen(301)).half()
    pos = torch.randint(0, 2048, (b, s), generator=gen(302), dtype=torch.int32)
    qd, kd = q.to(dev), k.to(dev)
    ops.rope_inplace(qd, kd, cos.to(dev), sin.to(dev), pos.to(dev))
    cos16, sin16 = cos.half().float(), sin.half().float()
    for got, x in ((qd.cpu(), q), (kd.cpu(), k)):
        ref = rope_ref(x, cos, sin, pos)
        err = (got.float() - ref).abs()
        assert (err <= 2e-3 + 4e-3 * ref.abs()).all(), err.max().item()
        ref16 = rope_ref(x, cos16, sin16, pos)
        assert torch.allclose(got.float(), ref16, atol=1e-2, rtol=1e-2)


def test_all_ops_in_one_graph_equal_eager(dev):
    g = gen(310)
    x = torch.randn(8, 3072, generator=g).half().to(dev)
    w = (1 + 0.1 * torch.randn(3072, generator=g)).half().to(dev)
    cos, sin = (t.to(dev) for t in rope_tables(64, 128, 500000.0))
    q0 = torch.randn(2, 1, 24, 128, generator=g).half().to(dev)
    k0 = torch.randn(2, 1, 8, 128, generator=g).half().to(dev)
    pos = torch.tensor([[3], [17]], dtype=torch.int32, device=dev)
    nb = 6
    kc0 = torch.randn(nb, 16, 8, 128, generator=g).half().to(dev)
    vc0 = torch.randn(nb, 16, 8, 128, generator=g).half().to(dev)
    knew = torch.randn(2, 8, 128, generator=g).half().to(dev)
    vnew = torch.randn(2, 8, 128, generator=g).half().to(dev)
    slots = torch.tensor([2 * 16 + 0, 5 * 16 + 0], dtype=torch.int32, device=dev)
    qd = torch.randn(2, 24, 128, generator=g).half().to(dev)
    table = torch.tensor([[2], [5]], dtype=torch.int32, device=dev)
    ctx1 = torch.ones(2, dtype=torch.int32, device=dev)  # context 1: the new token only
    gate_up = torch.randn(3, 2 * 8192, generator=g).half().to(dev)
    q, k = q0.clone(), k0.clone()
    kc, vc = kc0.clone(), vc0.clone()

    def run():
        y = ops.rmsnorm(x, w, 1e-5)
        ops.rope_inplace(q, k, cos, sin, pos)
        ops.paged_kv_store(knew, vnew, kc, vc, slots)
        att = ops.paged_attention_decode(qd, kc, vc, table, ctx1, 1, 16, 128 ** -0.5)
        act = ops.swiglu(gate_up)
        return y, att, act

    def reset():
        q.copy_(q0)
        k.copy_(k0)
        kc.copy_(kc0)
        vc.copy_(vc0)

    eager = [t.clone() for t in run()] + [q.clone(), k.clone(), kc.clone(), vc.clone()]
    torch.cuda.synchronize()
    reset()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            outs = run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    bits = lambda t: t.view(torch.int16)
    for rep in range(3):
        reset()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = list(outs) + [q, k, kc, vc]
        for want, have in zip(eager, got):
            assert torch.equal(bits(want), bits(have)), rep
        # eager work between the replays
        (x.float() * 2).sum().item()
    # context 1: the output rows are the new tokens' v rows, the KV store's result
    want_att = vnew.repeat_interleave(3, dim=1)
    assert torch.equal(bits(eager[1]), bits(want_att))


def test_graph_vs_eager_reference_test_shape(dev):
    cfg = dict(hidden_size=3072, intermediate_size=8192, num_hidden_layers=4,
               num_attention_heads=24, num_key_value_heads=8, head_dim=128, vocab_size=4096,
               rms_norm_eps=1e-5, rope_theta=500000.0, max_position_embeddings=4096)
    w_cpu = random_llama_weights(cfg, seed=320, tied=True, norm_std=0.1)
    weights = {k_: v.to(dev) for k_, v in w_cpu.items()}
    prompt, steps = 99, 4
    cache = KVCacheManager(num_blocks=(prompt + steps + 16) // 16 + 4, block_size=16,
                           num_layers=4, num_heads=8, head_dim=128, device=dev)
    model = Llama3BEngineModel(Llama3BConfig(cfg), weights, cache)
    cache.allocate_sequence(0, prompt + steps + 1)
    ids = torch.randint(0, cfg["vocab_size"], (1, prompt), generator=gen(321))
    tok = prefill_step(model, ids.to(dev), [0]).argmax(-1, keepdim=True)
    runner = CUDAGraphRunner(model, max_batch_size=1)
    runner.capture_graph(tok, torch.full((1, 1), prompt, dtype=torch.int32, device=dev), [0],
                         torch.full((1,), prompt + 1, dtype=torch.int32, device=dev))
    for i in range(steps):
        p = prompt + i  # position 99: context 100 at the first step
        ctx = torch.full((1,), p + 1, dtype=torch.int32, device=dev)
        posd = torch.full((1, 1), p, dtype=torch.int32, device=dev)
        slots, bt, mb = runner._prepare_inputs([0], ctx, max_blocks=runner.max_blocks_per_seq)
        eager = model.decode_step(tok, posd, ctx, slots, bt, mb).clone()
        graph = runner.execute(tok, posd, [0], ctx).clone()
        torch.cuda.synchronize()
        assert torch.allclose(graph.float(), eager.float(), atol=1e-2, rtol=1e-2), i
        assert torch.equal(graph.argmax(-1), eager.argmax(-1))
        tok = graph.argmax(-1, keepdim=True)
