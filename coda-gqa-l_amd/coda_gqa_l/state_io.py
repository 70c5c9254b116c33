"""Saving, loading and moving bounded-layer states.

The on-disk format is the reference's (src/coda_gqa_l/neural_db.py:285-308):
one ``torch.save`` of ``{"states": {layer_index: CoDAGQALandmarkStatePerf2
with CPU tensors}, "metadata": {...}}``.  The state dataclass keeps the
reference's module path and field order (coda_gqa_l.state), so files written
by either implementation load in the other.

Differences from the reference, on purpose:
- ``load_state`` unpickles with ``weights_only=True`` (only the state
  dataclass is allowed besides tensors and plain containers), where the
  reference uses ``weights_only=False``.
- ``state_to_device`` keeps the norm caches in the model dtype.  The
  reference casts ``_exact_v_norm`` / ``_sum_lf_k_norm`` to float32 on restore
  (neural_db.py:61-64) although ``init_state`` creates them in the model dtype
  (attention.py:306-316); the HIP kernels read them in the dtype of the K/V
  buffers, so they are cast back to it here.

A restored state starts its next decode step with a fresh routing record
(the module recognises the new tensors), so save -> load -> step gives the
same results as stepping the original state.
"""

from __future__ import annotations

import os
from typing import Any, Dict, Union

import torch

from .state import CoDAGQALandmarkStatePerf2

__all__ = ["state_to_cpu", "state_to_device", "deep_copy_state", "save_state", "load_state"]


def _map_tensors(state: CoDAGQALandmarkStatePerf2, fn) -> CoDAGQALandmarkStatePerf2:
    return CoDAGQALandmarkStatePerf2(
        k_buf=fn(state.k_buf),
        v_buf=fn(state.v_buf),
        allowed=fn(state.allowed),
        g_recent=fn(state.g_recent),
        recent_idx=int(state.recent_idx),
        recent_filled=int(state.recent_filled),
        mem_last_exact=fn(state.mem_last_exact),
        pos=int(state.pos),
        active_exact=int(state.active_exact),
        active_summary=int(state.active_summary),
        _exact_v_norm=fn(state._exact_v_norm) if state._exact_v_norm is not None else None,
        _sum_lf_k_norm=fn(state._sum_lf_k_norm) if state._sum_lf_k_norm is not None else None,
        metrics=dict(state.metrics) if state.metrics is not None else None,
    )


def state_to_cpu(state: CoDAGQALandmarkStatePerf2) -> CoDAGQALandmarkStatePerf2:
    """A copy of ``state`` with every tensor on the CPU (neural_db.py:30-46)."""
    return _map_tensors(state, lambda t: t.detach().cpu())


def deep_copy_state(state: CoDAGQALandmarkStatePerf2) -> CoDAGQALandmarkStatePerf2:
    """A copy of ``state`` with every tensor cloned in place (neural_db.py:67-83)."""
    return _map_tensors(state, lambda t: t.clone())


def state_to_device(state: CoDAGQALandmarkStatePerf2, device: Union[str, torch.device],
                    dtype: torch.dtype) -> CoDAGQALandmarkStatePerf2:
    """Move ``state``'s tensors to ``device`` in place and return it
    (neural_db.py:49-64): K/V and the norm caches in ``dtype``, the ring gates
    in float32, ``allowed`` bool, LRU stamps int64."""
    state.k_buf = state.k_buf.to(device=device, dtype=dtype)
    state.v_buf = state.v_buf.to(device=device, dtype=dtype)
    state.allowed = state.allowed.to(device=device, dtype=torch.bool)
    state.g_recent = state.g_recent.to(device=device, dtype=torch.float32)
    state.mem_last_exact = state.mem_last_exact.to(device=device, dtype=torch.int64)
    if state._exact_v_norm is not None:
        state._exact_v_norm = state._exact_v_norm.to(device=device, dtype=dtype)
    if state._sum_lf_k_norm is not None:
        state._sum_lf_k_norm = state._sum_lf_k_norm.to(device=device, dtype=dtype)
    return state


def save_state(ingested: Dict[str, Any], path: Union[str, os.PathLike]) -> int:
    """Write ``{"states": {i: state}, "metadata": ...}`` with CPU copies of the
    states; returns the file size in bytes (neural_db.py:285-295)."""
    data = {
        "states": {k: state_to_cpu(v) for k, v in ingested["states"].items()},
        "metadata": ingested.get("metadata", {}),
    }
    torch.save(data, path)
    return os.path.getsize(path)


def load_state(path: Union[str, os.PathLike]) -> Dict[str, Any]:
    """Read a file written by ``save_state`` (or by the reference's
    ``NeuralDatabase.save_state``) onto the CPU, unpickling nothing but
    tensors, plain containers and the state dataclass."""
    with torch.serialization.safe_globals([CoDAGQALandmarkStatePerf2]):
        return torch.load(path, map_location="cpu", weights_only=True)
