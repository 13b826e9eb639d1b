"""Safetensors weight loader (reference: engine/weight_loader.py:9-46).

Reads config.json and every *.safetensors shard of a local model directory
(sorted by name), casting each tensor to fp16 on the target device, keyed by
the Hugging Face names (model.layers.{l}.self_attn.q_proj.weight, ...).
Missing config.json or shards raise FileNotFoundError, as in the reference.
Loading happens shard by shard through the CPU, so peak host memory is one
shard.
"""
from __future__ import annotations

import gc
import glob
import json
import os
from typing import Any, Dict

import torch


class WeightLoader:
    def __init__(self, model_dir: str, device: str = "cuda", dtype: torch.dtype = torch.float16):
        self.model_dir = model_dir
        self.device = device
        self.dtype = dtype
        self.config = self._load_config()

    def _load_config(self) -> Dict[str, Any]:
        path = os.path.join(self.model_dir, "config.json")
        if not os.path.exists(path):
            raise FileNotFoundError(f"config.json not found in {self.model_dir}")
        with open(path, "r") as f:
            return json.load(f)

    def shard_files(self):
        files = sorted(glob.glob(os.path.join(self.model_dir, "*.safetensors")))
        if not files:
            raise FileNotFoundError(f"No .safetensors files found in {self.model_dir}")
        return files

    def load_weights(self) -> Dict[str, torch.Tensor]:
        from safetensors.torch import load_file
        weights: Dict[str, torch.Tensor] = {}
        for path in self.shard_files():
            shard = load_file(path, device="cpu")
            for name, tensor in shard.items():
                weights[name] = tensor.to(dtype=self.dtype, device=self.device)
            del shard
            gc.collect()
        return weights
