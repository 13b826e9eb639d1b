"""engine.models (reference: engine/models/) -> the Llama-3.2-3B wrapper."""
