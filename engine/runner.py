"""engine.runner (reference: engine/runner.py:8-178) -> the hipGraph decode runner."""
from mycustomcudaengine_amd.engine.runner import CUDAGraphRunner  # noqa: F401

__all__ = ["CUDAGraphRunner"]
