"""CPU oracle for the bounded differential-attention hot path.

TEST INFRASTRUCTURE ONLY. This package restates, on torch CPU, the eager
(non-Triton, non-CUDA) path of anthony-maio/CoDA-GQA-L:
  - src/coda_gqa_l/attention.py      -> layer.OracleLayer
  - src/coda_gqa_l/memory_banks.py   -> banks.*
  - src/coda_gqa_l/primitives.py     -> prims.*
  - src/coda_gqa_l/baseline.py       -> ops.OracleUnbounded
  - operator seams (diff_flash_attn, coda_kernels epilogue, bank routing)
                                     -> ops.*
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
it, as the checker; the product package never does.

Pinning (what proves this restatement equals the reference):
  - tests/golden/*.npz, written by tests/golden/make_golden.py from the
    reference itself in the build container: full prefill+decode trajectories
    (outputs, states, per-chunk slot decisions) are compared bit-exactly.
  - closed forms in tests/test_oracle_*.py (fp64 brute-force attention,
    RMSNorm, RoPE, W>=L bounded==unbounded, zero-init summary routing,
    torch.topk tie orders).
"""

from .layer import METRIC_KEYS, OracleLayer, OracleState
from .ops import (OracleUnbounded, diff_attention, diff_epilogue, diff_sub_only, exact_route,
                  lower_right_mask, summary_update)
from . import banks, prims

__all__ = ["OracleLayer", "OracleState", "OracleUnbounded", "METRIC_KEYS", "banks", "prims",
           "diff_attention", "diff_epilogue", "diff_sub_only", "exact_route", "summary_update",
           "lower_right_mask"]
