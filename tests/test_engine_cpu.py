"""CPU: engine host logic -- block allocator, slot rules, weight loader,
config -- against the oracle's integer rules, plus a self-consistency check
of the model oracle (prefill of S tokens == prefill of S-1 then one decode)."""
import json
import os

import numpy as np
import pytest
import torch

from mycustomcudaengine_amd.engine.cache import KVCacheManager
from mycustomcudaengine_amd.engine.models.llama import Llama3BConfig
from mycustomcudaengine_amd.engine.weight_loader import WeightLoader
from oracle.alloc_ref import BlockAllocatorRef, prefill_slots_ref, slot_mapping_ref
from oracle.model_ref import LlamaRef, random_llama_weights


def test_allocator_matches_reference_rules():
    m = KVCacheManager(12, 4, num_layers=1, num_heads=2, head_dim=8, device="cpu")
    r = BlockAllocatorRef(12, 4)
    for seq, n in ((5, 9), (2, 1), (9, 4)):
        m.allocate_sequence(seq, n)
        r.allocate_sequence(seq, n)
    for seq, ln in ((2, 1), (2, 4), (9, 4), (9, 5), (5, 12)):
        m.append_token(seq, ln)
        r.append_token(seq, ln)
    assert m.block_tables == r.tables
    assert m.kv_cache.shape == (1, 2, 12, 4, 2, 8)
    bt = m.get_block_table_tensor([9, 5, 2], 5)
    assert bt.dtype == torch.int32 and bt.numpy().tolist() == r.block_table([9, 5, 2], 5).tolist()
    assert m.slot_mapping([5, 9], [10, 5]).tolist() == \
        slot_mapping_ref(r.tables, [5, 9], [10, 5], 4).tolist()
    assert m.prefill_slot_mapping([5, 9], 3).tolist() == \
        prefill_slots_ref(r.tables, [5, 9], 3, 4).tolist()
    with pytest.raises(RuntimeError):
        m.allocate_sequence(77, 100)


def test_free_sequence_returns_blocks_fifo():
    m = KVCacheManager(4, 4, 1, 1, 8, device="cpu")
    m.allocate_sequence(0, 8)
    m.free_sequence(0)
    m.allocate_sequence(1, 16)
    assert m.block_tables[1] == [2, 3, 0, 1]


def test_weight_loader_reads_sorted_shards(tmp_path):
    from safetensors.torch import save_file
    with pytest.raises(FileNotFoundError):
        WeightLoader(str(tmp_path), device="cpu")
    (tmp_path / "config.json").write_text(json.dumps({"hidden_size": 16, "vocab_size": 32}))
    loader = WeightLoader(str(tmp_path), device="cpu")
    with pytest.raises(FileNotFoundError):
        loader.load_weights()
    a = {"model.embed_tokens.weight": torch.randn(32, 16)}
    b = {"model.norm.weight": torch.ones(16, dtype=torch.bfloat16)}
    save_file(a, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file(b, str(tmp_path / "model-00002-of-00002.safetensors"))
    w = loader.load_weights()
    assert set(w) == {"model.embed_tokens.weight", "model.norm.weight"}
    assert all(t.dtype == torch.float16 for t in w.values())
    assert torch.equal(w["model.embed_tokens.weight"], a["model.embed_tokens.weight"].half())
    cfg = Llama3BConfig(loader.config)
    assert cfg.hidden_size == 16 and cfg.vocab_size == 32 and cfg.num_hidden_layers == 28


def test_config_defaults_are_llama_3_2_3b():
    c = Llama3BConfig({})
    assert (c.hidden_size, c.intermediate_size, c.num_hidden_layers) == (3072, 8192, 28)
    assert (c.num_attention_heads, c.num_key_value_heads, c.head_dim) == (24, 8, 128)
    assert (c.vocab_size, c.rms_norm_eps, c.rope_theta) == (128256, 1e-5, 500000.0)


SMALL = dict(hidden_size=64, intermediate_size=96, num_hidden_layers=2,
             num_attention_heads=6, num_key_value_heads=2, head_dim=16, vocab_size=50,
             rms_norm_eps=1e-5, rope_theta=500000.0)


def test_model_oracle_prefill_equals_prefill_plus_decode():
    w = random_llama_weights(SMALL, seed=3, std=0.2)
    ids = torch.randint(0, 50, (2, 7), generator=torch.Generator().manual_seed(4))
    full = LlamaRef(SMALL, w).prefill(ids, [0, 1])
    ref = LlamaRef(SMALL, w)
    ref.prefill(ids[:, :6], [0, 1])
    step = ref.decode(ids[:, 6:7], [6, 6], [0, 1])
    assert torch.allclose(full, step, atol=1e-5)


def test_reference_engine_import_path():
    """The reference's callers import engine.cache, engine.runner,
    engine.weight_loader and engine.models.llama (benchmarks/
    benchmark_engine.py:7-9, engine/runner.py:5); those paths resolve to this
    engine's classes."""
    import mycustomcudaengine_amd.engine as mine
    from engine.cache import KVCacheManager as A
    from engine.models.llama import Llama3BConfig as B, Llama3BEngineModel as C
    from engine.runner import CUDAGraphRunner as D
    from engine.weight_loader import WeightLoader as E
    assert (A, B, C, D, E) == (mine.KVCacheManager, mine.Llama3BConfig, mine.Llama3BEngineModel,
                               mine.CUDAGraphRunner, mine.WeightLoader)
