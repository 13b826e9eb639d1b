"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every fixture.  GPU: the kernels, run on the
fixture inputs through the my_cuda_engine_cpp surface, match the fixture
outputs (attention/norm/activation/rotation within max-abs 1e-2 of the fp32
values; the KV store bit-exactly).
"""
import os

import numpy as np
import pytest
import torch

from oracle.ops_ref import (decode_attention_ref, kv_store_ref, prefill_attention_ref,
                            rmsnorm_ref, rope_ref, swiglu_ref)

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-2


def load(name):
    with np.load(os.path.join(HERE, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


T = torch.from_numpy


def test_oracle_reproduces_decode_fixture():
    f = load("decode_small.npz")
    out = decode_attention_ref(T(f["query"]), T(f["key_cache"]), T(f["value_cache"]),
                               T(f["block_tables"]), T(f["context_lens"]), float(f["scale"]))
    assert np.allclose(out.numpy(), f["out"], atol=1e-6)


def test_oracle_reproduces_prefill_fixture():
    f = load("prefill_small.npz")
    out = prefill_attention_ref(T(f["query"]), T(f["key"]), T(f["value"]), float(f["scale"]))
    assert np.allclose(out.numpy(), f["out"], atol=1e-6)


def test_oracle_reproduces_elementwise_fixture():
    f = load("elementwise_small.npz")
    assert np.allclose(rmsnorm_ref(T(f["x"]), T(f["w"]), float(f["eps"])).numpy(),
                       f["rmsnorm"], atol=1e-6)
    assert np.allclose(swiglu_ref(T(f["gate_up"])).numpy(), f["swiglu"], atol=1e-6)
    cos, sin, pos = T(f["cos"]), T(f["sin"]), T(f["positions"])
    assert np.allclose(rope_ref(T(f["q"]), cos, sin, pos).numpy(), f["q_rot"], atol=1e-6)
    assert np.allclose(rope_ref(T(f["k"]), cos, sin, pos).numpy(), f["k_rot"], atol=1e-6)


def test_oracle_reproduces_kv_store_fixture():
    f = load("kv_store_small.npz")
    kc = np.zeros_like(f["key_cache"])
    vc = np.zeros_like(f["value_cache"])
    kv_store_ref(f["key"], f["value"], kc, vc, f["slots"])
    assert np.array_equal(kc.view(np.uint16), f["key_cache"].view(np.uint16))
    assert np.array_equal(vc.view(np.uint16), f["value_cache"].view(np.uint16))


@pytest.mark.gpu
def test_kernels_match_fixtures(dev):
    import my_cuda_engine_cpp as ops
    f = load("decode_small.npz")
    bt = T(f["block_tables"])
    out = ops.paged_attention_decode(T(f["query"]).to(dev), T(f["key_cache"]).to(dev),
                                     T(f["value_cache"]).to(dev), bt.to(dev),
                                     T(f["context_lens"]).to(dev), bt.shape[1],
                                     int(f["block_size"]), float(f["scale"])).cpu()
    assert np.abs(out.float().numpy() - f["out"]).max() <= TOL

    f = load("prefill_small.npz")
    out = ops.prefill_attention(T(f["query"]).to(dev), T(f["key"]).to(dev),
                                T(f["value"]).to(dev), float(f["scale"])).cpu()
    assert np.abs(out.float().numpy() - f["out"]).max() <= TOL

    f = load("elementwise_small.npz")
    out = ops.rmsnorm(T(f["x"]).to(dev), T(f["w"]).to(dev), float(f["eps"])).cpu()
    assert np.abs(out.float().numpy() - f["rmsnorm"]).max() <= TOL
    out = ops.swiglu(T(f["gate_up"]).to(dev)).cpu()
    assert np.abs(out.float().numpy() - f["swiglu"]).max() <= TOL
    q, k = T(f["q"]).to(dev), T(f["k"]).to(dev)
    ops.rope_inplace(q, k, T(f["cos"]).to(dev), T(f["sin"]).to(dev), T(f["positions"]).to(dev))
    assert np.abs(q.cpu().float().numpy() - f["q_rot"]).max() <= TOL
    assert np.abs(k.cpu().float().numpy() - f["k_rot"]).max() <= TOL

    f = load("kv_store_small.npz")
    kc = torch.zeros(f["key_cache"].shape, dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    ops.paged_kv_store(T(f["key"]).to(dev), T(f["value"]).to(dev), kc, vc, T(f["slots"]).to(dev))
    assert np.array_equal(kc.cpu().numpy().view(np.uint16), f["key_cache"].view(np.uint16))
    assert np.array_equal(vc.cpu().numpy().view(np.uint16), f["value_cache"].view(np.uint16))
