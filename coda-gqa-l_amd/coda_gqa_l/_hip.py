"""ctypes binding of libcoda_mi355x.so (the C ABI in include/coda_mi355x.h).

The library is the only compute path of this package: when it is missing,
or a tensor is not on a HIP device, the calls raise instead of falling back
to anything else.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

from ._srchash import source_hash

LIB_NAME = "libcoda_mi355x.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
_DEFAULT_LIB_PATH = LIB_PATH

CODA_F32, CODA_BF16, CODA_F16 = 0, 1, 2
CODA_OK, CODA_EUNSUP = 0, 2
DTYPE_CODE = {torch.float32: CODA_F32, torch.bfloat16: CODA_BF16, torch.float16: CODA_F16}
NUM_COUNTERS = 8
(CNT_EXACT_HITS, CNT_EXACT_INSERTS, CNT_EXACT_OVERWRITES, CNT_SUMMARY_UPDATES, CNT_SUMMARY_INSERTS,
 CNT_TOKENS_GATED_OUT, CNT_EXACT_FRUSTRATED, CNT_SUMMARY_FRUSTRATED) = range(8)

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float


class AttnDesc(ctypes.Structure):
    """coda_attn_desc."""

    _fields_ = [
        ("dtype", _i32), ("B", _i32), ("H", _i32), ("Hkv", _i32), ("Lq", _i32), ("Dh", _i32),
        ("q", _vp), ("q_sb", _i64), ("q_sh", _i64), ("q_sl", _i64),
        ("q_noise", _vp), ("qn_sb", _i64), ("qn_sh", _i64), ("qn_sl", _i64),
        ("theta_cos", _vp), ("theta_sin", _vp),
        ("rope_cos", _vp), ("rope_sin", _vp), ("rope_interleaved", _i32),
        ("kp", _vp), ("vp", _vp), ("Lp", _i32), ("p_sb", _i64), ("p_sh", _i64), ("p_sl", _i64),
        ("allowed", _vp), ("al_sb", _i64),
        ("kb", _vp), ("vb", _vp), ("Lb", _i32), ("b_sb", _i64), ("b_sh", _i64), ("b_sl", _i64),
        ("causal", _i32),
        ("lam", _vp), ("lam_sb", _i64), ("lam_sh", _i64), ("lam_sl", _i64),
        ("rms_w", _vp), ("eps", _f32), ("sm_scale", _f32),
        ("out", _vp), ("o_sb", _i64), ("o_sh", _i64), ("o_sl", _i64),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
    ]


class BankDesc(ctypes.Structure):
    """coda_bank_desc."""

    _fields_ = [
        ("dtype", _i32), ("B", _i32), ("Hkv", _i32), ("Dh", _i32), ("W", _i32), ("Me", _i32), ("Ms", _i32),
        ("lf", _i32), ("active_exact", _i32), ("active_summary", _i32),
        ("k_buf", _vp), ("v_buf", _vp), ("allowed", _vp), ("g_recent", _vp), ("mem_last", _vp),
        ("exact_v_norm", _vp), ("sum_lf_k_norm", _vp), ("eta", _vp),
        ("gated", _i32), ("tau_exact", _f32), ("tau_summary", _f32), ("tau_match", _f32), ("tau_novel", _f32),
        ("refresh_on_hit", _i32), ("overwrite_on_insert", _i32), ("energy_scale", _f32),
        ("metrics", _vp), ("frustrated", _vp), ("trace", _vp), ("active", _vp),
    ]


class ProjDesc(ctypes.Structure):
    """coda_proj_desc (include/coda_mi355x.h)."""

    _fields_ = [
        ("dtype", _i32), ("M", _i32), ("D", _i32), ("L", _i32), ("H", _i32), ("Hkv", _i32), ("Dh", _i32),
        ("rope_interleaved", _i32), ("gate", _i32), ("w_layout", _i32),
        ("x", _vp), ("x_sm", _i64), ("w", _vp), ("bias", _vp), ("rope_cos", _vp), ("rope_sin", _vp),
        ("q", _vp), ("q_sm", _i64), ("k", _vp), ("k_sm", _i64), ("v", _vp), ("v_sm", _i64),
        ("lam", _vp), ("lam_sm", _i64), ("g", _vp), ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
    ]


_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None

_SIGS = {
    "coda_abi_version": (_i32, []),
    "coda_last_error": (ctypes.c_char_p, []),
    "coda_source_hash": (ctypes.c_char_p, []),
    "coda_device_count": (_i32, []),
    "coda_attn_workspace_bytes": (_i32, [ctypes.POINTER(AttnDesc), ctypes.POINTER(ctypes.c_size_t)]),
    "coda_diff_attn_fwd": (_i32, [ctypes.POINTER(AttnDesc), _vp]),
    "coda_prefill_attn_chunks": (_i32, [ctypes.POINTER(AttnDesc), _i32, _i32, _i32, _i32, _i32, _i64, _i64, _vp]),
    "coda_diff_epilogue_fwd": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _f32, _vp]),
    "coda_diff_sub_only_fwd": (_i32, [_i32, _vp, _vp, _vp, _vp, _i32, _i32, _vp]),
    "coda_rope_fwd": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _vp, _i32, _i32, _i32,
                             _i32, _i32, _vp]),
    "coda_decode_write": (_i32, [ctypes.POINTER(BankDesc), _vp, _vp, _i64, _i64, _vp, _i32, _i32, _i64, _vp]),
    "coda_decode_step_workspace_bytes": (_i32, [ctypes.POINTER(BankDesc), ctypes.POINTER(AttnDesc),
                                                 ctypes.POINTER(ctypes.c_size_t)]),
    "coda_decode_step": (_i32, [ctypes.POINTER(BankDesc), ctypes.POINTER(AttnDesc), _vp, _vp, _i64, _i64, _vp, _i32,
                                _i32, _i64, _vp, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int), _vp]),
    "coda_decode_step_raw_k": (_i32, [ctypes.POINTER(BankDesc), ctypes.POINTER(AttnDesc), _vp, _vp, _i64, _i64, _vp, _i32,
                                _i32, _i64, _vp, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int), _vp]),
    "coda_block_plan": (_i32, [_vp, _i32, _i32, _i32, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp,
                               _i32, _vp]),
    "coda_block_write": (_i32, [ctypes.POINTER(BankDesc), _vp, _vp, _i64, _i64, _i64, _vp, _i64, _i32, _i32,
                                _i32, _i64, _vp, _i32, _i32, _i32, _vp, ctypes.c_size_t, _vp]),
    "coda_block_write_snapshot": (_i32, [ctypes.POINTER(BankDesc), _vp, _vp, _i64, _i64, _i64, _vp, _i64, _i32, _i32,
                                         _i32, _i64, _vp, _i32, _i32, _i32, _vp, ctypes.c_size_t, _vp, _vp, _vp, _vp]),
    "coda_project_pack": (_i32, [_vp, _i32, _i32, _i64, _vp, _vp]),
    "coda_block_write_chain": (_i32, [ctypes.POINTER(BankDesc), _vp, _vp, _i64, _i64, _i64, _vp, _i64, _i32, _i32, _i32,
                                      _i32, _i32, _i32, _i64, _vp, _i32, _i32, _i32, _vp, ctypes.c_size_t, _vp, _vp, _vp,
                                      _i64, _i64, ctypes.POINTER(ctypes.c_int), _vp]),
    "coda_block_workspace_bytes": (_i32, [ctypes.POINTER(BankDesc), _i32, ctypes.POINTER(ctypes.c_size_t)]),
    "coda_block_write_check": (_i32, [ctypes.POINTER(BankDesc), _i32, _i32]),
    "coda_block_sync_timeouts": (_i32, [ctypes.POINTER(ctypes.c_uint)]),
    "coda_bank_expand": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp]),
    "coda_block_sync_spin_limit": (_i32, [_i32]),
    "coda_block_write_noalloc": (_i32, [ctypes.POINTER(BankDesc), _vp, _vp, _i64, _i64, _i64, _vp, _i64, _i32, _i32,
                                        _i32, _i64, _vp, _i32, _i32, _i32, _vp]),
    "coda_block_write_noalloc_max_bytes": (ctypes.c_size_t, []),
    "coda_ring_rotate": (_i32, [ctypes.POINTER(BankDesc), _i32, _vp, ctypes.c_size_t, _vp]),
    "coda_unit_rows": (_i32, [_i32, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i32, _i32, _vp]),
    "coda_project": (_i32, [ctypes.POINTER(ProjDesc), _vp]),
    "coda_project_workspace_bytes": (_i32, [ctypes.POINTER(ProjDesc), ctypes.POINTER(ctypes.c_size_t)]),
    "coda_topk_order_host": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp]),
    # the reference's typed epilogue symbols (void, errors in coda_last_error)
    **{"diff_epilogue_forward_" + t: (None, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _f32, _vp])
       for t in ("bf16", "fp16", "fp32")},
    **{"diff_sub_only_forward_" + t: (None, [_vp, _vp, _vp, _vp, _i32, _i32, _vp]) for t in ("bf16", "fp16", "fp32")},
    "coda_topk_order_host_i64": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp]),
}


def _check_fresh(L: ctypes.CDLL) -> None:
    """The in-tree library must be built from the sources beside it (a
    library loaded from another path, LIB_PATH changed, is not checked)."""
    if os.path.abspath(LIB_PATH) != _DEFAULT_LIB_PATH:
        return
    want = source_hash()
    if want is None:
        return
    have = L.coda_source_hash().decode(errors="replace")
    if have != want:
        raise RuntimeError(f"{LIB_NAME} was built from other sources (hash {have}) than the ones beside it "
                           f"(hash {want}); rebuild it: `python coda-gqa-l_amd/csrc/build.py`")


def available() -> bool:
    """Whether the library is built in place (no load, no HIP call)."""
    return os.path.exists(LIB_PATH)


def lib() -> ctypes.CDLL:
    """Load the library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(f"{LIB_NAME} is not built ({LIB_PATH}); run "
                                   "`python coda-gqa-l_amd/csrc/build.py` (needs hipcc for gfx950)")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGS.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _check_fresh(L)
            _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        msg = lib().coda_last_error().decode(errors="replace")
        raise RuntimeError(f"coda_mi355x error {rc}: {msg}")


def dtype_code(dt: torch.dtype) -> int:
    if dt not in DTYPE_CODE:
        raise TypeError(f"unsupported dtype {dt}")
    return DTYPE_CODE[dt]


def require_device(*tensors: Optional[torch.Tensor]) -> None:
    """Every tensor must live on a HIP device: there is no host path."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("coda_gqa_l (MI355X build) runs on HIP devices only; got a tensor on "
                               f"{t.device}. Move the module and inputs to a GPU.")


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()
