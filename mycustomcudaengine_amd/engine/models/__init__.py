from .llama import Llama3BConfig, Llama3BEngineModel

__all__ = ["Llama3BConfig", "Llama3BEngineModel"]
