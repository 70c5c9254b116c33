"""CoDA-GQA-L bounded differential attention for AMD Instinct MI355X (gfx950).

Drop-in for the reference package's hot path (same import name, classes,
state dataclass and operator seams); compute runs in the hand-written HIP
kernels of libcoda_mi355x.so (C ABI: include/coda_mi355x.h).
"""

from .adapters import EveCoDAAdapter, LlamaCoDAAdapter, Qwen3CoDAAdapter
from .attention import CoDAGQALandmarkPerf2
from .baseline import CoDAGQA
from .memory_banks import MemoryBankMixin
from .ops import diff_epilogue, diff_flash_attn, diff_sub_only, is_available
from .primitives import HeadwiseRMSNorm, RotaryEmbedding, apply_rope, compute_lf_start, repeat_kv
from .state import CoDAGQALandmarkStatePerf2

__all__ = [
    "CoDAGQALandmarkPerf2",
    "CoDAGQALandmarkStatePerf2",
    "CoDAGQA",
    "LlamaCoDAAdapter",
    "Qwen3CoDAAdapter",
    "EveCoDAAdapter",
    "MemoryBankMixin",
    "HeadwiseRMSNorm",
    "RotaryEmbedding",
    "apply_rope",
    "repeat_kv",
    "compute_lf_start",
    "diff_flash_attn",
    "diff_epilogue",
    "diff_sub_only",
    "is_available",
]
