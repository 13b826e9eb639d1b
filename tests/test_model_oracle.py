"""CPU: pin the model oracle (oracle/model_ref.py LlamaRef) independently.

LlamaRef composes the pinned op oracles (rmsnorm_ref, rope_ref, an einsum
attention, swiglu_ref) in the layer order of the reference decode step
(engine/models/llama.py:59-174) and prefill driver
(benchmarks/benchmark_engine.py:12-129).  Every GPU engine test compares
against it, so its layer composition is checked here without reusing its
code:

  * closed form: with every projection weight zero, attention and MLP add
    nothing, each layer is the identity on the residual stream, and the
    logits are rms_norm(embed[ids]) @ embed^T (tied head, non-unit final
    norm weight);
  * an independent forward written only from library routines
    (F.embedding, F.rms_norm, F.linear, causal
    F.scaled_dot_product_attention with enable_gqa, F.silu) and a
    complex-exponential RoPE, in float64, on non-unit norm weights: equal to
    LlamaRef's prefill logits and to its prefill + decode logits;
  * negative controls: the same independent forward with one planted
    mistake each (a dropped residual add, gate and up swapped, RoPE applied
    to v, left off k, paired interleaved or with k one position off q, the
    two layer norms swapped or unweighted, an interleaved GQA head map, no
    causal mask) must land far outside the tolerance, so the comparison
    above would catch that mistake in LlamaRef.  (A uniform shift of all
    positions is invisible by construction: RoPE is relative.)
"""
import pytest
import torch
import torch.nn.functional as F

from oracle.model_ref import LlamaRef, random_llama_weights

CFG = dict(hidden_size=64, intermediate_size=96, num_hidden_layers=2,
           num_attention_heads=6, num_key_value_heads=2, head_dim=16, vocab_size=50,
           rms_norm_eps=1e-5, rope_theta=500000.0)
TOL = 1e-4  # fp32 oracle vs float64 library composition; logits are O(1)


def _rope_complex(x: torch.Tensor, pos: torch.Tensor, theta: float,
                  interleaved: bool = False) -> torch.Tensor:
    """x [B, H, S, D] rotated as complex numbers z_i = x_i + j x_{i+D/2} times
    exp(j pos theta^(-2i/D)) (the half-split pairing; interleaved=True pairs
    x_{2i} with x_{2i+1} instead, the other common convention)."""
    d = x.shape[-1]
    half = d // 2
    inv = theta ** (-torch.arange(0, d, 2, dtype=torch.float64) / d)
    ang = pos.to(torch.float64)[:, None] * inv[None, :]          # [S, D/2]
    rot = torch.polar(torch.ones_like(ang), ang)                  # exp(j ang)
    if interleaved:
        z = torch.complex(x[..., 0::2], x[..., 1::2]) * rot
        return torch.stack([z.real, z.imag], dim=-1).flatten(-2)
    z = torch.complex(x[..., :half], x[..., half:]) * rot
    return torch.cat([z.real, z.imag], dim=-1)


def independent_forward(cfg, w, ids, mistake=None, pos_offset=0):
    """Last-position logits [B, vocab] of a causal forward over ids [B, S],
    float64, from library routines only.  `mistake` plants one error;
    pos_offset shifts every position (which RoPE, depending only on
    position differences, must not notice)."""
    wt = {k: v.double() for k, v in w.items()}
    b, s = ids.shape
    hid, hq, hkv, d = (cfg["hidden_size"], cfg["num_attention_heads"],
                       cfg["num_key_value_heads"], cfg["head_dim"])
    eps, theta = cfg["rms_norm_eps"], cfg["rope_theta"]
    pos = torch.arange(s) + pos_offset
    pos_k = pos + (1 if mistake == "k_pos_off_by_one" else 0)
    inter = mistake == "rope_interleaved"

    def norm(x, name):
        weight = None if mistake == "norm_unweighted" else wt[name]
        return F.rms_norm(x, (hid,), weight=weight, eps=eps)

    x = F.embedding(ids, wt["model.embed_tokens.weight"])
    for l in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{l}"
        n_in, n_post = f"{p}.input_layernorm.weight", f"{p}.post_attention_layernorm.weight"
        if mistake == "norms_swapped":
            n_in, n_post = n_post, n_in
        h = norm(x, n_in)
        q = F.linear(h, wt[f"{p}.self_attn.q_proj.weight"]).view(b, s, hq, d).transpose(1, 2)
        k = F.linear(h, wt[f"{p}.self_attn.k_proj.weight"]).view(b, s, hkv, d).transpose(1, 2)
        v = F.linear(h, wt[f"{p}.self_attn.v_proj.weight"]).view(b, s, hkv, d).transpose(1, 2)
        q = _rope_complex(q, pos, theta, inter)
        if mistake != "no_rope_k":
            k = _rope_complex(k, pos_k, theta, inter)
        if mistake == "rope_on_v":
            v = _rope_complex(v, pos, theta, inter)
        if mistake == "gqa_interleaved":  # query head h on kv head h % Hkv
            idx = torch.arange(hq) % hkv
            k, v = k[:, idx], v[:, idx]
            attn = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        else:
            attn = F.scaled_dot_product_attention(q, k, v, is_causal=mistake != "not_causal",
                                                  enable_gqa=True)
        o = F.linear(attn.transpose(1, 2).reshape(b, s, hq * d),
                     wt[f"{p}.self_attn.o_proj.weight"])
        x = o if mistake == "drop_attn_residual" else x + o
        h = norm(x, n_post)
        gate = F.linear(h, wt[f"{p}.mlp.gate_proj.weight"])
        up = F.linear(h, wt[f"{p}.mlp.up_proj.weight"])
        if mistake == "gate_up_swapped":
            gate, up = up, gate
        m = F.linear(F.silu(gate) * up, wt[f"{p}.mlp.down_proj.weight"])
        x = m if mistake == "drop_mlp_residual" else x + m
    head = wt.get("lm_head.weight", wt["model.embed_tokens.weight"])
    return F.linear(norm(x[:, -1], "model.norm.weight"), head)


def _weights(seed=21, tied=False):
    return random_llama_weights(CFG, seed=seed, std=0.2, tied=tied, norm_std=0.3)


def _ids(seed=22, b=2, s=9):
    return torch.randint(0, CFG["vocab_size"], (b, s), generator=torch.Generator().manual_seed(seed))


def test_zero_projection_weights_make_every_layer_the_identity():
    w = random_llama_weights(CFG, seed=23, std=0.2, tied=True, norm_std=0.3)
    for k in w:
        if k.endswith("proj.weight"):
            w[k] = torch.zeros_like(w[k])
    ids = _ids(24)
    emb = w["model.embed_tokens.weight"].double()
    wn = w["model.norm.weight"].double()

    def closed_form(tok):
        x = emb[tok]
        return F.rms_norm(x, (CFG["hidden_size"],), weight=wn, eps=CFG["rms_norm_eps"]) @ emb.T

    got = LlamaRef(CFG, w).prefill(ids, [0, 1]).double()
    assert torch.allclose(got, closed_form(ids[:, -1]), atol=1e-5, rtol=1e-5)
    ref = LlamaRef(CFG, w)
    ref.prefill(ids[:, :5], [0, 1])
    step = ref.decode(ids[:, 5:6], [5, 5], [0, 1]).double()
    assert torch.allclose(step, closed_form(ids[:, 5]), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("tied", [False, True])
def test_llamaref_prefill_equals_library_composition(tied):
    w = _weights(tied=tied)
    ids = _ids()
    got = LlamaRef(CFG, w).prefill(ids, [0, 1]).double()
    want = independent_forward(CFG, w, ids)
    assert (got - want).abs().max().item() <= TOL * max(1.0, want.abs().max().item())


def test_llamaref_decode_equals_library_composition():
    """Prefill of S-1 tokens then decode steps: each step's logits equal the
    library forward over the whole prefix (the decode path's cache handling
    and positions, not only the prefill's)."""
    w = _weights(seed=25)
    ids = _ids(26, b=2, s=12)
    ref = LlamaRef(CFG, w)
    ref.prefill(ids[:, :8], [3, 7])
    for t in range(8, 12):
        got = ref.decode(ids[:, t:t + 1], [t, t], [3, 7]).double()
        want = independent_forward(CFG, w, ids[:, :t + 1])
        assert (got - want).abs().max().item() <= TOL * max(1.0, want.abs().max().item()), t


def test_rope_is_relative_uniform_position_shift_changes_nothing():
    """Shifting every position by the same amount rotates q and k alike, so
    scores and logits stay the same: a uniform offset is not a detectable
    mistake, an offset between q and k is (k_pos_off_by_one below)."""
    w = _weights()
    ids = _ids()
    got = LlamaRef(CFG, w).prefill(ids, [0, 1]).double()
    want = independent_forward(CFG, w, ids, pos_offset=37)
    assert (got - want).abs().max().item() <= TOL * max(1.0, want.abs().max().item())


MISTAKES = ["drop_attn_residual", "drop_mlp_residual", "gate_up_swapped", "rope_on_v",
            "no_rope_k", "rope_interleaved", "k_pos_off_by_one", "norms_swapped",
            "norm_unweighted", "gqa_interleaved", "not_causal"]


@pytest.mark.parametrize("mistake", MISTAKES)
def test_planted_mistake_is_caught(mistake):
    """Negative control: a forward with the mistake differs from LlamaRef by
    at least 100x the tolerance the two tests above allow."""
    w = _weights()
    ids = _ids()
    got = LlamaRef(CFG, w).prefill(ids, [0, 1]).double()
    bad = independent_forward(CFG, w, ids, mistake=mistake)
    assert (got - bad).abs().max().item() > 100 * TOL * max(1.0, got.abs().max().item())
