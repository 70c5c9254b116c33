"""Import path of the reference (src/coda_gqa_l/eve_adapter.py); the class lives in
coda_gqa_l.adapters."""

from .adapters import EveCoDAAdapter

__all__ = ["EveCoDAAdapter"]
