"""CPU fp32 reference of the Llama decode step and prefill -- test
infrastructure only.

Composition of the oracle ops with fp32 GEMMs, restating
engine/models/llama.py:59-174 (decode_step) and
benchmarks/benchmark_engine.py:12-129 (prefill_step, without its defects:
per-position KV-store loop, transposed attention output, unused GQA
expansion).  The KV cache is a plain dict of per-(layer, sequence) K/V
lists, so the reference shares no paging code with the engine.
"""
from __future__ import annotations

import math

import torch

from .ops_ref import rmsnorm_ref, rope_ref, rope_tables, swiglu_ref


class LlamaRef:
    def __init__(self, cfg: dict, weights: dict):
        self.c = cfg
        self.w = {k: v.detach().float().cpu() for k, v in weights.items()}
        self.cos, self.sin = rope_tables(4096, cfg["head_dim"], cfg["rope_theta"])
        self.kv = {}  # (layer, seq) -> (K [t, Hkv, D], V [t, Hkv, D])

    def _layer(self, l, x, pos, seqs):
        """x [N, hidden] for N tokens; pos [N] positions; seqs [N] sequence ids.
        Appends each token's K/V to its sequence, then attends causally over
        that sequence's K/V up to the token's position."""
        c, w = self.c, self.w
        hq, hkv, d = c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"]
        p = f"model.layers.{l}"
        xn = rmsnorm_ref(x, w[f"{p}.input_layernorm.weight"], c["rms_norm_eps"])
        q = xn @ w[f"{p}.self_attn.q_proj.weight"].T
        k = xn @ w[f"{p}.self_attn.k_proj.weight"].T
        v = xn @ w[f"{p}.self_attn.v_proj.weight"].T
        n = x.shape[0]
        q = rope_ref(q.view(n, 1, hq, d), self.cos, self.sin, pos.view(n, 1)).view(n, hq, d)
        k = rope_ref(k.view(n, 1, hkv, d), self.cos, self.sin, pos.view(n, 1)).view(n, hkv, d)
        v = v.view(n, hkv, d)
        for i in range(n):
            key = (l, int(seqs[i]))
            kk, vv = self.kv.get(key, (torch.zeros(0, hkv, d), torch.zeros(0, hkv, d)))
            t = int(pos[i])
            if kk.shape[0] <= t:
                pad = t + 1 - kk.shape[0]
                kk = torch.cat([kk, torch.zeros(pad, hkv, d)])
                vv = torch.cat([vv, torch.zeros(pad, hkv, d)])
            kk[t], vv[t] = k[i], v[i]
            self.kv[key] = (kk, vv)
        out = torch.zeros(n, hq, d)
        grp = hq // hkv
        scale = 1.0 / math.sqrt(d)
        for i in range(n):
            kk, vv = self.kv[(l, int(seqs[i]))]
            t = int(pos[i]) + 1
            ks = kk[:t].repeat_interleave(grp, dim=1)  # [t, Hq, D]
            vs = vv[:t].repeat_interleave(grp, dim=1)
            s = torch.einsum("hd,thd->ht", q[i], ks) * scale
            out[i] = torch.einsum("ht,thd->hd", torch.softmax(s, dim=-1), vs)
        x = x + out.view(n, hq * d) @ w[f"{p}.self_attn.o_proj.weight"].T
        xn = rmsnorm_ref(x, w[f"{p}.post_attention_layernorm.weight"], c["rms_norm_eps"])
        gu = torch.cat([xn @ w[f"{p}.mlp.gate_proj.weight"].T,
                        xn @ w[f"{p}.mlp.up_proj.weight"].T], dim=-1)
        return x + swiglu_ref(gu) @ w[f"{p}.mlp.down_proj.weight"].T

    def _logits(self, x):
        xn = rmsnorm_ref(x, self.w["model.norm.weight"], self.c["rms_norm_eps"])
        head = self.w.get("lm_head.weight", self.w["model.embed_tokens.weight"])
        return xn @ head.T

    def prefill(self, input_ids: torch.Tensor, seq_ids) -> torch.Tensor:
        """input_ids [B, S]; returns last-token logits [B, vocab]."""
        b, s = input_ids.shape
        x = self.w["model.embed_tokens.weight"][input_ids.reshape(-1).cpu()]
        pos = torch.arange(s).repeat(b)
        seqs = torch.tensor(seq_ids).repeat_interleave(s)
        for l in range(self.c["num_hidden_layers"]):
            x = self._layer(l, x, pos, seqs)
        return self._logits(x.view(b, s, -1)[:, -1])

    def decode(self, input_ids: torch.Tensor, positions, seq_ids) -> torch.Tensor:
        """input_ids [B, 1]; positions [B] (the new token's position)."""
        x = self.w["model.embed_tokens.weight"][input_ids.reshape(-1).cpu()]
        pos = torch.as_tensor(positions).reshape(-1).cpu()
        seqs = torch.tensor(seq_ids)
        for l in range(self.c["num_hidden_layers"]):
            x = self._layer(l, x, pos, seqs)
        return self._logits(x)


def random_llama_weights(cfg: dict, seed: int, device="cpu", std: float = 0.02,
                         tied: bool = True, norm_std: float = 0.0) -> dict:
    """Random-init Llama weights ~ N(0, std), keyed by the Hugging Face names;
    lm_head tied to the embedding unless tied=False.  RMSNorm weights are 1
    (as in every reference harness, benchmarks/benchmark_engine.py:180-181)
    unless norm_std > 0: then 1 + N(0, norm_std), drawn from a second
    generator so the other tensors keep the values a given seed gives them."""
    g = torch.Generator().manual_seed(seed)
    gn = torch.Generator().manual_seed(seed + 1_000_003)
    hid, inter = cfg["hidden_size"], cfg["intermediate_size"]
    hq, hkv, d = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]

    def rnd(*shape):
        return (torch.randn(*shape, generator=g) * std).to(torch.float16).to(device)

    def norm():
        w = torch.ones(hid)
        if norm_std > 0:
            w = w + torch.randn(hid, generator=gn) * norm_std
        return w.to(torch.float16).to(device)

    w = {"model.embed_tokens.weight": rnd(cfg["vocab_size"], hid),
         "model.norm.weight": norm()}
    if not tied:
        w["lm_head.weight"] = rnd(cfg["vocab_size"], hid)
    for l in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{l}"
        w[f"{p}.input_layernorm.weight"] = norm()
        w[f"{p}.post_attention_layernorm.weight"] = norm()
        w[f"{p}.self_attn.q_proj.weight"] = rnd(hq * d, hid)
        w[f"{p}.self_attn.k_proj.weight"] = rnd(hkv * d, hid)
        w[f"{p}.self_attn.v_proj.weight"] = rnd(hkv * d, hid)
        w[f"{p}.self_attn.o_proj.weight"] = rnd(hid, hq * d)
        w[f"{p}.mlp.gate_proj.weight"] = rnd(inter, hid)
        w[f"{p}.mlp.up_proj.weight"] = rnd(inter, hid)
        w[f"{p}.mlp.down_proj.weight"] = rnd(hid, inter)
    return w
