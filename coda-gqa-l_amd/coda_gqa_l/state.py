"""Mutable inference state of one bounded layer.

Same dataclass name, module path (coda_gqa_l.state), field names, field
order and defaults as the reference (src/coda_gqa_l/state.py:12-54), so
states pickled with torch.save by either implementation load in the other.

Buffer layout: [recent ring W | exact bank Me | summary bank Ms] along the
slot axis.  Keys in k_buf carry RoPE.  Exact bank routes on values, the
summary bank on the low-frequency key band; summary keys keep a zero
high-frequency band.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, Optional

import torch


@dataclass
class CoDAGQALandmarkStatePerf2:
    k_buf: torch.Tensor            # (B, Hkv, Lbuf, Dh)
    v_buf: torch.Tensor            # (B, Hkv, Lbuf, Dh)
    allowed: torch.Tensor          # (B, Lbuf) bool, True = slot valid

    g_recent: torch.Tensor         # (B, W) float32 write gate per ring slot
    recent_idx: int                # next eviction slot when the ring is full
    recent_filled: int             # ring occupancy, <= W

    mem_last_exact: torch.Tensor   # (B, Me) int64 LRU stamps

    pos: int                       # absolute position of the next token

    active_exact: int = 0          # active exact slots (dynamic expansion)
    active_summary: int = 0        # active summary slots

    _exact_v_norm: Optional[torch.Tensor] = field(default=None, repr=False)    # (B, Hkv, Me, Dh)
    _sum_lf_k_norm: Optional[torch.Tensor] = field(default=None, repr=False)   # (B, Hkv, Ms, Dh - lf)

    metrics: Optional[Dict[str, Any]] = field(default=None, repr=False)
