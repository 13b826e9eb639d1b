"""Writes the small golden fixtures in this folder from the CPU oracle.

Each .npz holds seeded inputs and the oracle's fp32 (or exact, for the KV
store) outputs, at sizes of a few tens of KB.  Run from the repo root:
    python tests/golden/make_golden.py
The reference repository commits no golden vectors of its own; these pin the
oracle's outputs (checked against library routines and brute force in
tests/test_oracle.py) so later changes to either side are caught.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.inputs import make_decode_case, make_prefill_case  # noqa: E402
from oracle.ops_ref import (decode_attention_ref, kv_store_ref, prefill_attention_ref,  # noqa: E402
                            rmsnorm_ref, rope_ref, rope_tables, swiglu_ref)


def f16(t):
    return t.to(torch.float16).numpy()


def main():
    g = torch.Generator().manual_seed(7)
    c = make_decode_case(71, 2, [40, 23], num_heads=6, num_kv_heads=2, spare=0.5,
                         nan_pool=True)
    out = decode_attention_ref(c.query, c.key_cache, c.value_cache, c.block_tables,
                               c.context_lens, c.scale)
    np.savez_compressed(os.path.join(HERE, "decode_small.npz"), query=f16(c.query),
             key_cache=f16(c.key_cache), value_cache=f16(c.value_cache),
             block_tables=c.block_tables.numpy(), context_lens=c.context_lens.numpy(),
             block_size=np.int32(c.block_size), scale=np.float32(c.scale), out=out.numpy())

    p = make_prefill_case(72, 1, 24, 6, 2)
    out = prefill_attention_ref(p.query, p.key, p.value, p.scale)
    np.savez_compressed(os.path.join(HERE, "prefill_small.npz"), query=f16(p.query), key=f16(p.key),
             value=f16(p.value), scale=np.float32(p.scale), out=out.numpy())

    x = torch.randn(3, 256, generator=g).half()
    w = (1 + 0.3 * torch.randn(256, generator=g)).half()
    gu = (2 * torch.randn(3, 2 * 96, generator=g)).half()
    cos, sin = rope_tables(64, 128, 500000.0)
    q = torch.randn(2, 3, 6, 128, generator=g).half()
    k = torch.randn(2, 3, 2, 128, generator=g).half()
    pos = torch.tensor([[0, 17, 63], [5, 6, 40]], dtype=torch.int32)
    np.savez_compressed(os.path.join(HERE, "elementwise_small.npz"), x=f16(x), w=f16(w), eps=np.float32(1e-5),
             rmsnorm=rmsnorm_ref(x, w, 1e-5).numpy(), gate_up=f16(gu),
             swiglu=swiglu_ref(gu).numpy(), q=f16(q), k=f16(k), positions=pos.numpy(),
             cos=cos[:64].numpy(), sin=sin[:64].numpy(),
             q_rot=rope_ref(q, cos, sin, pos).numpy(), k_rot=rope_ref(k, cos, sin, pos).numpy())

    rng = np.random.default_rng(73)
    key = rng.standard_normal((12, 2, 128)).astype(np.float16)
    val = rng.standard_normal((12, 2, 128)).astype(np.float16)
    slots = rng.permutation(5 * 16)[:12].astype(np.int32)
    slots[4] = -1
    kc = np.zeros((5, 16, 2, 128), np.float16)
    vc = np.zeros((5, 16, 2, 128), np.float16)
    kv_store_ref(key, val, kc, vc, slots)
    np.savez_compressed(os.path.join(HERE, "kv_store_small.npz"), key=key, value=val, slots=slots,
             key_cache=kc, value_cache=vc)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
