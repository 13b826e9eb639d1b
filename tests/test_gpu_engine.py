"""GPU: the engine end to end on a 2-layer model with Llama-3.2-3B layer
geometry (hidden 3072, 24/8 heads, head_dim 128, SwiGLU 8192) and a small
vocabulary, against the fp32 CPU model oracle (oracle/model_ref.py).

Bars: prefill and decode logits within a relative L2 error of 1e-2 and
max-abs 5e-2 of the fp32 oracle (fp16 activations through 2 layers); the
graph-replayed decode step equals the eager decode step within the
reference's allclose(1e-2, 1e-2) (tests/test_cuda_graph.py:138); token ids,
slots and block tables handled exactly (greedy tokens identical).
"""
import pytest
import torch

from mycustomcudaengine_amd.engine import (CUDAGraphRunner, KVCacheManager, Llama3BConfig,
                                           Llama3BEngineModel, prefill_step)
from oracle.model_ref import LlamaRef, random_llama_weights

pytestmark = pytest.mark.gpu

CFG = dict(hidden_size=3072, intermediate_size=8192, num_hidden_layers=2,
           num_attention_heads=24, num_key_value_heads=8, head_dim=128, vocab_size=4096,
           rms_norm_eps=1e-5, rope_theta=500000.0, max_position_embeddings=4096)


def build(dev, batch, prompt, gen, seed=5, tied=True):
    # non-unit RMSNorm weights, so a swapped or dropped norm weight shows
    w_cpu = random_llama_weights(CFG, seed=seed, tied=tied, norm_std=0.1)
    weights = {k: v.to(dev) for k, v in w_cpu.items()}
    cache = KVCacheManager(num_blocks=batch * ((prompt + gen + 15) // 16) + 8, block_size=16,
                           num_layers=CFG["num_hidden_layers"], num_heads=8, head_dim=128,
                           device=dev)
    model = Llama3BEngineModel(Llama3BConfig(CFG), weights, cache)
    for s in range(batch):
        cache.allocate_sequence(s, prompt + gen)
    return model, cache, LlamaRef(CFG, w_cpu)


def close(gpu, ref, rel=1e-2, abs_=5e-2):
    g = gpu.float().cpu()
    err = (g - ref).norm() / ref.norm()
    mx = (g - ref).abs().max().item()
    assert err.item() <= rel and mx <= abs_, (err.item(), mx)


@pytest.mark.parametrize("projections", ["decode_gemm", "library"])
def test_prefill_then_eager_decode_match_oracle(dev, projections, monkeypatch):
    """Both decode-step paths: the decode-sized GEMM kernels with RMSNorm /
    SwiGLU / residual fused (taken at this batch), and torch.matmul with the
    separate ops (taken for larger batches, forced here)."""
    b, s = 2, 37
    model, cache, ref = build(dev, b, s, 4, tied=False)
    assert model._decode_gemms_take(b)
    if projections == "library":
        monkeypatch.setattr(model, "_decode_gemms_take", lambda n: False)
    ids = torch.randint(0, CFG["vocab_size"], (b, s), generator=torch.Generator().manual_seed(1))
    logits = prefill_step(model, ids.to(dev), [0, 1], torch.full((b,), s, dtype=torch.int32))
    close(logits, ref.prefill(ids, [0, 1]))
    tok = logits.argmax(-1, keepdim=True)
    for i in range(3):
        pos = s + i
        slots = torch.from_numpy(cache.slot_mapping([0, 1], [pos + 1] * b)).to(dev)
        mb = len(cache.block_tables[0])
        bt = cache.get_block_table_tensor([0, 1], mb)
        out = model.decode_step(tok, torch.full((b, 1), pos, dtype=torch.int32, device=dev),
                                torch.full((b,), pos + 1, dtype=torch.int32, device=dev),
                                slots, bt, mb)
        want = ref.decode(tok.cpu(), [pos] * b, [0, 1])
        close(out, want)
        tok = want.argmax(-1, keepdim=True).to(dev)  # follow the oracle's greedy path


def test_one_token_prompt_and_reused_pages(dev):
    """A one-token prompt (prefill of S = 1) then decode steps match the
    oracle; then a finished sequence is freed and a new one is allocated on
    exactly its pages, which still hold the old sequence's K/V, and its
    prefill and decode steps match the oracle too: only the new sequence's own
    positions are ever read."""
    gen, v = 3, CFG["vocab_size"]
    w_cpu = random_llama_weights(CFG, seed=8, norm_std=0.1)
    weights = {k: t.to(dev) for k, t in w_cpu.items()}
    per_seq = (40 + gen + 15) // 16
    cache = KVCacheManager(num_blocks=2 * per_seq, block_size=16,
                           num_layers=CFG["num_hidden_layers"], num_heads=8, head_dim=128,
                           device=dev)
    model = Llama3BEngineModel(Llama3BConfig(CFG), weights, cache)
    ref = LlamaRef(CFG, w_cpu)
    g = torch.Generator().manual_seed(9)

    def run(seq, prompt_len):
        ids = torch.randint(0, v, (1, prompt_len), generator=g)
        logits = prefill_step(model, ids.to(dev), [seq])
        close(logits, ref.prefill(ids, [seq]))
        tok = logits.argmax(-1, keepdim=True)
        for i in range(gen):
            pos = prompt_len + i
            slots = torch.from_numpy(cache.slot_mapping([seq], [pos + 1])).to(dev)
            mb = len(cache.block_tables[seq])
            out = model.decode_step(tok, torch.full((1, 1), pos, dtype=torch.int32, device=dev),
                                    torch.full((1,), pos + 1, dtype=torch.int32, device=dev),
                                    slots, cache.get_block_table_tensor([seq], mb), mb)
            want = ref.decode(tok.cpu(), [pos], [seq])
            close(out, want)
            tok = want.argmax(-1, keepdim=True).to(dev)

    cache.allocate_sequence(0, 40 + gen)
    cache.allocate_sequence(1, 40 + gen)
    assert not cache.free_blocks  # the pool is exactly the two sequences
    run(0, 40)   # fills its pages with K/V
    run(1, 1)    # one-token prompt
    old = list(cache.block_tables[0])
    cache.free_sequence(0)
    cache.allocate_sequence(5, 20 + gen)
    assert cache.block_tables[5] == old[:len(cache.block_tables[5])]
    run(5, 20)   # on the freed pages


def test_graph_replay_matches_eager(dev):
    b, s, steps = 3, 20, 6
    model, cache, _ = build(dev, b, s, steps + 1, seed=6)
    seq = list(range(b))
    ids = torch.randint(0, CFG["vocab_size"], (b, s), generator=torch.Generator().manual_seed(2))
    logits = prefill_step(model, ids.to(dev), seq)
    tok = logits.argmax(-1, keepdim=True)
    runner = CUDAGraphRunner(model, max_batch_size=b)
    ctx = torch.full((b,), s + 1, dtype=torch.int32, device=dev)
    pos = torch.full((b, 1), s, dtype=torch.int32, device=dev)
    runner.capture_graph(tok, pos, seq, ctx)
    assert runner.max_blocks_per_seq == len(cache.block_tables[0])  # capacity, not ctx
    for i in range(steps):
        p = s + i
        ctx = torch.full((b,), p + 1, dtype=torch.int32, device=dev)
        pos = torch.full((b, 1), p, dtype=torch.int32, device=dev)
        # eager first: both write the same K/V slot, so the graph sees the same cache
        slots, bt, mb = runner._prepare_inputs(seq, ctx, max_blocks=runner.max_blocks_per_seq)
        eager = model.decode_step(tok, pos, ctx, slots, bt, mb).clone()
        graph = runner.execute(tok, pos, seq, ctx).clone()
        torch.cuda.synchronize()
        assert torch.allclose(graph.float(), eager.float(), atol=1e-2, rtol=1e-2), i
        assert torch.equal(graph.argmax(-1), eager.argmax(-1))
        tok = graph.argmax(-1, keepdim=True)


def test_decode_crosses_block_boundary_and_block_table_width(dev):
    """Decode past several 16-token blocks with the graph captured at the first
    step (the reference would read past its frozen table width here)."""
    b, s, steps = 2, 14, 40
    model, cache, ref = build(dev, b, s, steps + 1, seed=7)
    seq = [0, 1]
    ids = torch.randint(0, CFG["vocab_size"], (b, s), generator=torch.Generator().manual_seed(3))
    logits = prefill_step(model, ids.to(dev), seq)
    ref.prefill(ids, seq)
    tok = logits.argmax(-1, keepdim=True)
    runner = CUDAGraphRunner(model, max_batch_size=b)
    runner.capture_graph(tok, torch.full((b, 1), s, dtype=torch.int32, device=dev), seq,
                         torch.full((b,), s + 1, dtype=torch.int32))
    for i in range(steps):
        p = s + i
        out = runner.execute(tok, torch.full((b, 1), p, dtype=torch.int32, device=dev), seq,
                             torch.full((b,), p + 1, dtype=torch.int32))
        if i % 13 == 0 or i == steps - 1:
            want = ref.decode(tok.cpu(), [p] * b, seq)
            close(out, want)
            tok = want.argmax(-1, keepdim=True).to(dev)
        else:
            ref.decode(tok.cpu(), [p] * b, seq)  # keep the oracle's cache in step
            tok = out.argmax(-1, keepdim=True)



def test_device_loop_matches_host_prepared_steps(dev):
    """run_device_loop (greedy token and the next step's slots prepared on the
    device inside the graph) generates exactly the tokens of the same steps
    prepared on the host and replayed one by one (execute + torch.argmax)."""
    b, s, k = 3, 45, 6
    model, cache, _ = build(dev, b, s, k + 2)
    ids = torch.randint(0, CFG["vocab_size"], (b, s), generator=torch.Generator().manual_seed(4))
    seq = list(range(b))
    logits = prefill_step(model, ids.to(dev), seq, torch.full((b,), s, dtype=torch.int32))
    tok0 = logits.argmax(-1, keepdim=True)
    pos0 = torch.full((b, 1), s, dtype=torch.int32, device=dev)
    runner = CUDAGraphRunner(model, max_batch_size=b)
    runner.capture_graph(tok0, pos0, seq, [s + 1] * b, device_steps=k)
    dev_tokens = runner.run_device_loop(k).cpu()
    # host-prepared replays of the same steps (their KV writes are identical)
    tok = tok0
    host_tokens = []
    for i in range(k):
        p = s + i
        out = runner.execute(tok, torch.full((b, 1), p, dtype=torch.int32, device=dev), seq,
                             [p + 1] * b)
        tok = out.argmax(-1, keepdim=True)
        host_tokens.append(tok.view(-1).cpu())
    assert dev_tokens.tolist() == torch.stack(host_tokens).tolist()
    with pytest.raises(RuntimeError):
        runner.run_device_loop(k + 1)



def test_device_loop_sees_blocks_appended_after_capture(dev):
    """The graph is captured with a block table wider than the blocks the
    sequences own; blocks appended afterwards (append_token) must reach the
    replayed steps: run_device_loop copies the allocator's tables into the
    graph's table first (otherwise the new positions would map to block 0,
    another sequence's page).  Tokens equal the host-prepared steps'."""
    b, s, k = 2, 30, 6
    model, cache, _ = build(dev, b, s, 1)  # each sequence owns blocks for 31 tokens
    seq = [0, 1]
    ids = torch.randint(0, CFG["vocab_size"], (b, s), generator=torch.Generator().manual_seed(9))
    logits = prefill_step(model, ids.to(dev), seq)
    tok0 = logits.argmax(-1, keepdim=True)
    runner = CUDAGraphRunner(model, max_batch_size=b)
    runner.capture_graph(tok0, torch.full((b, 1), s, dtype=torch.int32, device=dev), seq,
                         [s + 1] * b, max_blocks=4, device_steps=k)
    assert all(len(cache.block_tables[q]) == 2 for q in seq)
    for q in seq:  # positions 32.. need a third block
        cache.append_token(q, 32)
    dev_tokens = runner.run_device_loop(k).cpu()
    tok = tok0
    host_tokens = []
    for i in range(k):
        p = s + i
        out = runner.execute(tok, torch.full((b, 1), p, dtype=torch.int32, device=dev), seq,
                             [p + 1] * b)
        tok = out.argmax(-1, keepdim=True)
        host_tokens.append(tok.view(-1).cpu())
    assert dev_tokens.tolist() == torch.stack(host_tokens).tolist()


def test_chunked_prefill_matches_one_shot_and_oracle(dev):
    """prefill_step with chunk_size: the same cache slots written with the
    same K/V up to the projections' rounding (the library GEMM may pick
    another kernel for the chunk's row count), last-token logits within the
    oracle bars like the one-shot prefill's."""
    b, s = 2, 70
    model, cache, ref = build(dev, b, s, 2, tied=False)
    ids = torch.randint(0, CFG["vocab_size"], (b, s), generator=torch.Generator().manual_seed(6))
    seq = [0, 1]
    cache.kv_cache.zero_()
    one = prefill_step(model, ids.to(dev), seq)
    kv_one = cache.kv_cache.clone()
    cache.kv_cache.zero_()
    chunked = prefill_step(model, ids.to(dev), seq, chunk_size=32)
    assert torch.equal(cache.kv_cache != 0, kv_one != 0)
    assert (cache.kv_cache.float() - kv_one.float()).abs().max().item() <= 2e-2
    want = ref.prefill(ids, seq)
    close(one, want)
    close(chunked, want)


def test_chunked_prefill_behind_long_prefix_splits_keys(dev):
    """A 2300-token prompt in 512-position chunks: the fourth and fifth
    chunks (512 and 252 positions) run behind 1536- and 2048-token cached
    prefixes, where prefill_step asks for the key split (one sequence: a small
    grid, so its query blocks' keys are cut in parts and merged); logits
    within the oracle bars."""
    b, s = 1, 2300
    model, cache, ref = build(dev, b, s, 2, tied=False)
    ids = torch.randint(0, CFG["vocab_size"], (b, s), generator=torch.Generator().manual_seed(8))
    chunked = prefill_step(model, ids.to(dev), [0], chunk_size=512)
    close(chunked, ref.prefill(ids, [0]))


def test_local_checkpoint_decode_step(dev, tmp_path):
    """The reference's real-checkpoint test (tests/test_real_model_forward.py:
    10-58: WeightLoader -> Llama3BConfig(loader.config) -> model, one decode
    step of two sequences at position 0 through runner._prepare_inputs, no
    NaN) on a synthetic local checkpoint in the Hugging Face layout: bf16
    tensors over three sorted shards with an index file, tied embeddings (no
    lm_head.weight), non-unit RMSNorm weights.  The logits are also checked
    against the fp32 oracle on the weights as loaded (bf16 -> fp16)."""
    import json
    from safetensors.torch import save_file
    from mycustomcudaengine_amd.engine.weight_loader import WeightLoader
    w = random_llama_weights(CFG, seed=11, tied=True)
    g = torch.Generator().manual_seed(12)
    for k in w:
        if k.endswith("norm.weight"):
            w[k] = (1 + 0.1 * torch.randn(w[k].shape, generator=g)).half()
    names = sorted(w)
    parts = [names[i::3] for i in range(3)]
    index = {"metadata": {}, "weight_map": {}}
    for i, part in enumerate(parts):
        fname = f"model-{i + 1:05d}-of-00003.safetensors"
        save_file({k: w[k].to(torch.bfloat16).contiguous() for k in part}, str(tmp_path / fname))
        index["weight_map"].update({k: fname for k in part})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(index))
    (tmp_path / "config.json").write_text(json.dumps(dict(
        CFG, architectures=["LlamaForCausalLM"], model_type="llama", torch_dtype="bfloat16",
        tie_word_embeddings=True, bos_token_id=1)))

    loader = WeightLoader(str(tmp_path), device=str(dev))
    weights = loader.load_weights()
    assert "lm_head.weight" not in weights and len(weights) == len(w)
    assert all(t.dtype == torch.float16 and t.device == dev for t in weights.values())
    config = Llama3BConfig(loader.config)
    cache = KVCacheManager(num_blocks=200, block_size=16, num_layers=config.num_hidden_layers,
                           num_heads=config.num_key_value_heads, head_dim=config.head_dim,
                           dtype=torch.float16, device=dev)
    model = Llama3BEngineModel(config, weights, cache)
    runner = CUDAGraphRunner(model, max_batch_size=2)
    ids = torch.tensor([[1], [1]], dtype=torch.int64, device=dev)
    positions = torch.zeros((2, 1), dtype=torch.int32, device=dev)
    context_lens = torch.ones(2, dtype=torch.int32, device=dev)
    cache.allocate_sequence(0, 1)
    cache.allocate_sequence(1, 1)
    slot_mapping, block_tables, max_blocks = runner._prepare_inputs([0, 1], context_lens)
    logits = model.decode_step(ids, positions, context_lens, slot_mapping, block_tables,
                               max_blocks)
    assert not torch.isnan(logits).any()
    ref = LlamaRef(CFG, {k: v.to(torch.bfloat16).half() for k, v in w.items()})
    close(logits, ref.decode(ids.cpu(), [0, 0], [0, 1]))
    # both sequences saw the same token at the same position
    assert torch.equal(logits[0], logits[1])
