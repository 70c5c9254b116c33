"""Import path of the reference (src/coda_gqa_l/llama_adapter.py); the class lives in
coda_gqa_l.adapters."""

from .adapters import LlamaCoDAAdapter

__all__ = ["LlamaCoDAAdapter"]
