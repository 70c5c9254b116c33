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

from dataclasses import dataclass, field, fields
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

    def __getstate__(self):
        # the dataclass fields only, active sizes folded in from the device
        # (the reference's pickled layout; the device words stay behind)
        _fold_active(self)
        d = self.__dict__
        return {k: d[k] for k in _FIELD_NAMES if k in d}


_FIELD_NAMES = tuple(f.name for f in fields(CoDAGQALandmarkStatePerf2))


# Dynamic bank expansion runs on the device: after a bank update the layer
# leaves the grown active sizes in the state's device words
# (__dict__["_active_dev"], int32 [exact, summary]) and marks the host ints
# stale.  Reading active_exact / active_summary folds them in (one host
# sync, the first read after an update only); assigning either one makes the
# host ints authoritative again (the layer re-makes the device words from
# them at its next bank update).
def _fold_active(st) -> None:
    d = st.__dict__
    if d.get("_active_stale"):
        a, b = d["_active_dev"].tolist()
        d["active_exact"], d["active_summary"] = int(a), int(b)
        d["_active_stale"] = False


def _active_property(name: str) -> property:
    def get(self):
        if self.__dict__.get("_active_stale"):
            _fold_active(self)
        return self.__dict__[name]

    def set(self, value):
        d = self.__dict__
        if d.get("_active_stale"):
            _fold_active(self)  # the other size stays current
        d[name] = value
        d.pop("_active_dev", None)

    return property(get, set, doc=f"{name} (folded in from the device after a dynamic expansion)")


CoDAGQALandmarkStatePerf2.active_exact = _active_property("active_exact")
CoDAGQALandmarkStatePerf2.active_summary = _active_property("active_summary")
