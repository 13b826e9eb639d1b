"""engine.models.llama (reference: engine/models/llama.py:10-174) -> Llama3BConfig and
Llama3BEngineModel over the paged KV cache."""
from mycustomcudaengine_amd.engine.models.llama import (  # noqa: F401
    Llama3BConfig,
    Llama3BEngineModel,
    rope_tables,
)

__all__ = ["Llama3BConfig", "Llama3BEngineModel", "rope_tables"]
