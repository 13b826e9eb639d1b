"""Drop-in engine around the my_cuda_engine_cpp ops: paged KV block allocator
(cache), graph-replayed decode runner (runner), safetensors loader
(weight_loader), Llama-3.2-3B wrapper (models.llama) and batched prefill
(prefill).  Mirrors the reference's engine/ package (engine/cache.py,
engine/runner.py, engine/weight_loader.py, engine/models/llama.py) and its
prefill driver (benchmarks/benchmark_engine.py:12-129)."""
from .cache import KVCacheManager
from .models.llama import Llama3BConfig, Llama3BEngineModel
from .prefill import prefill_step
from .runner import CUDAGraphRunner
from .weight_loader import WeightLoader

__all__ = ["KVCacheManager", "Llama3BConfig", "Llama3BEngineModel", "CUDAGraphRunner",
           "WeightLoader", "prefill_step"]
