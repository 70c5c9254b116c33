"""Import path of the reference (src/coda_gqa_l/qwen3_adapter.py); the class lives in
coda_gqa_l.adapters."""

from .adapters import Qwen3CoDAAdapter

__all__ = ["Qwen3CoDAAdapter"]
