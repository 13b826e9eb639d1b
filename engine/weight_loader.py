"""engine.weight_loader (reference: engine/weight_loader.py:9-46) -> the safetensors loader."""
from mycustomcudaengine_amd.engine.weight_loader import WeightLoader  # noqa: F401

__all__ = ["WeightLoader"]
