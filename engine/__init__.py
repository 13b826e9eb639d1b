"""The reference's `engine` package path (engine/cache.py, engine/runner.py,
engine/weight_loader.py, engine/models/llama.py), so callers written against
the reference -- `from engine.cache import KVCacheManager`,
`from engine.models.llama import Llama3BEngineModel` (benchmarks/
benchmark_engine.py:7-9, engine/runner.py:5) -- import the MI355X engine
unchanged.  Every name is re-exported from mycustomcudaengine_amd.engine."""
