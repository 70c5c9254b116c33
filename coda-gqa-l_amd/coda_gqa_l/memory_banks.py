"""Host orchestration of the bank kernels (ring FIFO, exact bank, summary bank).

The reference implements bank maintenance as ~100 eager torch ops per
prefill chunk and ~40 per decode token with several host syncs each
(src/coda_gqa_l/memory_banks.py:183-950).  Here a decode token is one
kernel (coda_decode_write) and a prefill chunk is one (coda_block_write;
four where a chunk's working set does not fit one CU's LDS);
the candidate choice of every chunk of a prefill call is planned up front
by one kernel (coda_block_plan), since the evicted gates depend only on the
token stream.  Within a prefill call the ring stays circular (head =
oldest slot); the call ends with the reference's layout (time order at
slots 0..filled-1, recent_idx = 0).

Host syncs happen only where the reference's semantics need host ints that
depend on device data: dynamic bank expansion (min < max capacities) and
the optional metrics dict.
"""

from __future__ import annotations

import ctypes
import collections
from typing import Dict, Optional

import torch

from . import _hip, ops
from .state import CoDAGQALandmarkStatePerf2

METRIC_KEYS = ("exact_hits", "exact_inserts", "exact_overwrites", "exact_fill_ratio", "summary_updates",
               "summary_inserts", "summary_fill_ratio", "tokens_gated_out", "total_evictions", "exact_frustrated",
               "summary_frustrated", "active_exact", "active_summary", "expansions_exact", "expansions_summary")

# device counters after the kernels' own (coda_bank_expand)
_EXPAND_KEYS = ("summary_frustrated", "expansions_exact", "expansions_summary")

_COUNTER_KEYS = {
    _hip.CNT_EXACT_HITS: "exact_hits", _hip.CNT_EXACT_INSERTS: "exact_inserts",
    _hip.CNT_EXACT_OVERWRITES: "exact_overwrites", _hip.CNT_SUMMARY_UPDATES: "summary_updates",
    _hip.CNT_SUMMARY_INSERTS: "summary_inserts", _hip.CNT_TOKENS_GATED_OUT: "tokens_gated_out",
    _hip.CNT_EXACT_FRUSTRATED: "exact_frustrated",
}


class DeviceMetrics(dict):
    """A state's ``metrics`` dict (the reference's keys and value types)
    whose bank-update counters stay on the device: each bank update adds
    into ``pending`` (int64, one slot per kernel counter plus one for
    ``summary_frustrated``) and leaves the latest fill ratios as device
    scalars, with no host sync; the first read of a value folds them in.
    Pickled, it is a mapping of the folded values; save_state writes a
    plain dict, the reference's format."""

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        self.pending: Optional[torch.Tensor] = None
        self.fill: Dict[str, torch.Tensor] = {}

    def accumulator(self, device) -> torch.Tensor:
        """int64 device counters: the kernels' NUM_COUNTERS, then
        summary_frustrated, expansions_exact, expansions_summary
        (coda_bank_expand)."""
        if self.pending is None or self.pending.device != torch.device(device):
            self._fold()
            self.pending = torch.zeros(_hip.NUM_COUNTERS + len(_EXPAND_KEYS), dtype=torch.int64, device=device)
        return self.pending

    def add_host(self, key: str, n: int) -> None:
        """A host-known increment (no fold)."""
        dict.__setitem__(self, key, dict.__getitem__(self, key) + n)

    def _fold(self) -> None:
        p, f = self.pending, self.fill
        if p is None and not f:
            return
        if p is not None:
            c = p.tolist()
            p.zero_()
            # (a key the caller removed comes back only with a new count)
            keys = list(_COUNTER_KEYS.items()) + [(_hip.NUM_COUNTERS + i, k) for i, k in enumerate(_EXPAND_KEYS)]
            for i, key in keys:
                if int(c[i]) or dict.__contains__(self, key):
                    dict.__setitem__(self, key, dict.get(self, key, 0) + int(c[i]))
        for key, v in list(f.items()):
            old = dict.get(self, key)
            val = v.item()
            dict.__setitem__(self, key, int(val) if isinstance(old, int) and not isinstance(old, bool) else float(val))
        f.clear()

    def __getitem__(self, key):
        self._fold()
        return super().__getitem__(key)

    # writes fold first, so a value set directly (a reset to 0, as on the
    # reference's plain dict) is not later raised by counts that were still
    # pending on the device when it was set
    def __setitem__(self, key, value):
        self._fold()
        super().__setitem__(key, value)

    def __delitem__(self, key):
        self._fold()
        super().__delitem__(key)

    def update(self, *args, **kwargs):
        self._fold()
        super().update(*args, **kwargs)

    def pop(self, key, *default):
        self._fold()
        return super().pop(key, *default)

    def popitem(self):
        self._fold()
        return super().popitem()

    def setdefault(self, key, default=None):
        self._fold()
        return super().setdefault(key, default)

    def clear(self):
        self._fold()
        super().clear()

    def get(self, key, default=None):
        self._fold()
        return super().get(key, default)

    def items(self):
        self._fold()
        return super().items()

    def values(self):
        self._fold()
        return super().values()

    def __iter__(self):
        self._fold()
        return super().__iter__()

    def __eq__(self, other):
        self._fold()
        return super().__eq__(other)

    __hash__ = None

    def __repr__(self):
        self._fold()
        return super().__repr__()

    def copy(self):
        self._fold()
        return dict(super().items())

    def __reduce__(self):
        # an OrderedDict of the folded values: loads anywhere, torch.load
        # with weights_only=True included (save_state writes a plain dict)
        self._fold()
        return (collections.OrderedDict, (list(super().items()),))


class MemoryBankMixin:
    """Bank maintenance for CoDAGQALandmarkPerf2 (memory_banks.py:36-950)."""

    # ------------------------------------------------------------ plumbing
    def _expandable(self) -> bool:
        return self.Me_min < self.Me_max or self.Ms_min < self.Ms_max

    def _check_state(self, st: CoDAGQALandmarkStatePerf2) -> None:
        _hip.require_device(st.k_buf, st.v_buf, st.allowed, st.g_recent, st.mem_last_exact)
        B, Hkv, Lbuf, Dh = st.k_buf.shape
        if (Hkv, Lbuf, Dh) != (self.num_kv_heads, self.Lbuf, self.head_dim):
            raise ValueError(f"state k_buf shape {tuple(st.k_buf.shape)} does not match the layer")
        for name in ("k_buf", "v_buf", "allowed", "g_recent", "mem_last_exact"):
            if not getattr(st, name).is_contiguous():
                setattr(st, name, getattr(st, name).contiguous())
        if st.allowed.dtype != torch.bool or st.g_recent.dtype != torch.float32 or \
                st.mem_last_exact.dtype != torch.int64:
            raise ValueError("state metadata dtypes must be allowed=bool, g_recent=float32, mem_last_exact=int64")
        for name in ("_exact_v_norm", "_sum_lf_k_norm"):
            t = getattr(st, name)
            if t is not None:
                if t.dtype != st.k_buf.dtype:
                    # norm caches follow the buffer dtype (a state moved with a
                    # dtype cast of the caches is brought back to it)
                    t = t.to(st.k_buf.dtype)
                setattr(st, name, t.contiguous())

    def _derived(self, name: str, src: torch.Tensor, key, fn) -> torch.Tensor:
        """Tensor derived from a parameter, recomputed only when the parameter
        changes (in-place version counter or storage), so a decode step
        launches no conversion kernels."""
        cache = self.__dict__.setdefault("_derived_cache", {})
        tag = (src._version, src.data_ptr(), src.dtype, src.device)
        hit = cache.get((name, key))
        if hit is not None and hit[0] == tag:
            return hit[1]
        with torch.no_grad():
            val = fn()
        cache[(name, key)] = (tag, val)
        return val

    def _eta_f32(self, device, dtype: torch.dtype) -> torch.Tensor:
        """sigmoid(summary_eta_logit).to(dtype) per KV head, as float32 on the
        device (memory_banks.py:394, :902).  The sigmoid is torch's CPU op on
        the parameter's own dtype, as in the reference's CPU path; it runs
        once per parameter version (an [Hkv] copy to the host and back)."""
        p = self.summary_eta_logit

        def make():
            eta = torch.sigmoid(p.detach().to("cpu")).to(dtype).to(torch.float32)
            return eta.to(device).contiguous()

        return self._derived("eta", p, (device, dtype), make)

    def _block_check(self, B: int, dtype: torch.dtype, Te: int, Ts: int) -> None:
        """coda_block_write_check: a clear error, before anything runs, for
        bank sizes and candidate counts whose chunk update does not fit the
        kernels' LDS (B = 0: any batch)."""
        d = _hip.BankDesc()
        d.dtype, d.B = _hip.dtype_code(dtype), int(B)
        d.Hkv, d.Dh, d.W, d.Me, d.Ms, d.lf = self.num_kv_heads, self.head_dim, self.window, self.Me_max, \
            self.Ms_max, self.lf_start
        d.active_exact, d.active_summary = self.Me_max, self.Ms_max
        _hip.check(_hip.lib().coda_block_write_check(d, int(Te), int(Ts)))

    def _check_bank_sizes(self) -> None:
        """At construction: the bank sizes alone (one candidate of each kind)
        must fit; skipped when the library is not built (every call raises
        then)."""
        if not _hip.available():
            return
        te = 1 if self.Me_max > 0 and self.exact_candidates_per_block > 0 else 0
        ts = 1 if self.Ms_max > 0 and self.summary_candidates_per_block > 0 else 0
        try:
            self._block_check(0, torch.bfloat16, te, ts)
        except RuntimeError as e:
            raise ValueError(f"bank sizes beyond this build's prefill kernels: {e}") from None

    def _bank_desc(self, st: CoDAGQALandmarkStatePerf2, eta: Optional[torch.Tensor],
                   metrics: Optional[torch.Tensor], frustrated: Optional[torch.Tensor],
                   trace: Optional[torch.Tensor] = None) -> _hip.BankDesc:
        d = _hip.BankDesc()
        d.dtype = _hip.dtype_code(st.k_buf.dtype)
        d.B = st.k_buf.shape[0]
        d.Hkv, d.Dh, d.W, d.Me, d.Ms, d.lf = self.num_kv_heads, self.head_dim, self.window, self.Me, self.Ms, \
            self.lf_start
        # the host ints as they stand (no fold: with dynamic expansion the
        # kernels read the device words instead)
        sd = st.__dict__
        d.active_exact = min(max(int(sd["active_exact"]), 0), self.Me)
        d.active_summary = min(max(int(sd["active_summary"]), 0), self.Ms)
        if self._expandable():
            d.active = self._active_words(st).data_ptr()
        d.k_buf, d.v_buf = st.k_buf.data_ptr(), st.v_buf.data_ptr()
        d.allowed, d.g_recent, d.mem_last = st.allowed.data_ptr(), st.g_recent.data_ptr(), \
            st.mem_last_exact.data_ptr()
        d.exact_v_norm = _hip.ptr(st._exact_v_norm)
        d.sum_lf_k_norm = _hip.ptr(st._sum_lf_k_norm)
        d.eta = _hip.ptr(eta)
        d.gated = int(self.write_policy != "none")
        d.tau_exact, d.tau_summary = self.write_gate_threshold_exact, self.write_gate_threshold_summary
        d.tau_match, d.tau_novel = self.exact_match_threshold, self.exact_novelty_threshold
        d.refresh_on_hit, d.overwrite_on_insert = int(self.exact_refresh_on_hit), \
            int(self.summary_overwrite_on_insert)
        d.energy_scale = self.energy_scale
        d.metrics = _hip.ptr(metrics)
        d.frustrated = _hip.ptr(frustrated)
        d.trace = _hip.ptr(trace)
        return d

    # ------------------------------------------------------------ decision trace
    # Setting ``layer.decision_trace = []`` makes every bank update append its
    # slot decisions as device tensors, with the tags and fields of the events
    # the reference path's decisions are usually inspected by:
    #   ("exact_one", idx, overwrite, keep), ("summary_one", idx, keep)   decode
    #   ("select", candidate ids), ("exact_block", idx, overwrite, touch),
    #   ("summary_block", idx)                                            prefill
    # (memory_banks.py:290-337, :364-432, :459-510, :690-742, :866-878).
    # Decode steps then take the general (uncached) launch path.
    def _tracing(self) -> bool:
        return self.__dict__.get("decision_trace") is not None

    def _trace_decode(self, tr: Optional[torch.Tensor]) -> None:
        if tr is None:
            return
        out = self.__dict__["decision_trace"]
        if self.Me > 0:
            out.append(("exact_one", tr[:, 0].long(), (tr[:, 1] & 1).bool(), (tr[:, 1] & 2).bool()))
        if self.Ms > 0:
            out.append(("summary_one", tr[:, 2].long(), (tr[:, 3] & 1).bool()))

    def _trace_block(self, tr: Optional[torch.Tensor], plan_c: torch.Tensor, Te: int, Ts: int) -> None:
        if tr is None:
            return
        out = self.__dict__["decision_trace"]
        out.append(("select", plan_c[:, :max(Te, Ts)].long()))
        if Te > 0:
            out.append(("exact_block", tr[:, :Te].long(), (tr[:, Te:2 * Te] & 1).bool(),
                        (tr[:, Te:2 * Te] & 2).bool()))
        if Ts > 0:
            out.append(("summary_block", tr[:, 2 * Te:2 * Te + Ts].long()))

    @staticmethod
    def _device_metrics(st) -> Optional[DeviceMetrics]:
        mt = st.metrics
        if mt is not None and not isinstance(mt, DeviceMetrics):
            mt = st.metrics = DeviceMetrics(mt)
        return mt

    def _aux_buffers(self, st, device):
        """The kernels' counter array (the state's device accumulator, added
        into by every bank update) and frustration flags."""
        mt = self._device_metrics(st)
        metrics = mt.accumulator(device)[:_hip.NUM_COUNTERS] if mt is not None else None
        need_fr = (self._expandable() and not self.training) or st.metrics is not None
        frustrated = torch.zeros(4, dtype=torch.int64, device=device) if need_fr else None
        return metrics, frustrated

    def _fold_metrics(self, st, counters: Optional[torch.Tensor], evictions: int, exact_ran: bool,
                      summary_ran: bool) -> None:
        """Host-known metrics and the latest fill ratios (device scalars);
        the kernel counters are already in the state's accumulator."""
        mt = st.metrics
        if mt is None or counters is None:
            return
        mt.add_host("total_evictions", int(evictions))
        W, Me = self.window, self.Me
        if exact_ran and Me > 0:
            mt.fill["exact_fill_ratio"] = st.allowed[:, W:W + Me].any(dim=0).float().mean()
        if summary_ran and self.Ms > 0:
            mt.fill["summary_fill_ratio"] = st.allowed[:, W + Me:].any(dim=0).float().mean()

    def _active_words(self, st) -> torch.Tensor:
        """The state's active bank sizes as device words (int32 [exact,
        summary]), made from its host ints when missing or on another device
        (two fill launches, no host sync)."""
        d = st.__dict__
        dev = st.k_buf.device
        w = d.get("_active_dev")
        if w is None or w.device != dev:
            a, b = int(st.active_exact), int(st.active_summary)  # (folds a stale copy from another device)
            w = torch.empty(2, dtype=torch.int32, device=dev)
            w[0:1].fill_(a)
            w[1:2].fill_(b)
            d["_active_dev"] = w
            d["_active_stale"] = False
        return w

    def _expand_from(self, st, fr: Optional[torch.Tensor], exact_count_mode: bool, ran_e: bool, ran_s: bool):
        """Dynamic expansion after a bank update (attention.py:358-390) and
        its metrics, on the device (coda_bank_expand): the active sizes grow
        in the state's device words, which the next update's kernels read;
        the host ints fold in on their next read."""
        if fr is None:
            return
        expand = self._expandable() and not self.training
        mt = st.metrics if isinstance(st.metrics, DeviceMetrics) else None
        counters = mt.accumulator(fr.device)[_hip.NUM_COUNTERS:] if mt is not None else None
        if not expand and counters is None:
            return
        act = self._active_words(st) if expand else None
        ce, cs = self._log_ceiling(int(st.pos))
        _hip.check(_hip.lib().coda_bank_expand(_hip.ptr(act), fr.data_ptr(), int(ce), int(cs), int(exact_count_mode),
                                               int(ran_e), int(ran_s), _hip.ptr(counters), _hip.stream_of(fr)))
        if expand:
            st.__dict__["_active_stale"] = True
            if mt is not None:
                mt.fill["active_exact"] = act[0]
                mt.fill["active_summary"] = act[1]

    # ------------------------------------------------------------ decode
    def _write_one(self, st: CoDAGQALandmarkStatePerf2, *, k_new: torch.Tensor, v_new: torch.Tensor,
                   g_new: torch.Tensor) -> None:
        """One token into the ring; evict into the banks when full
        (memory_banks.py:183-224).  k_new, v_new (B, Hkv, 1, Dh); g_new (B,)."""
        self._check_state(st)
        B = st.k_buf.shape[0]
        dev = st.k_buf.device
        kn = k_new.reshape(B, self.num_kv_heads, self.head_dim)
        vn = v_new.reshape(B, self.num_kv_heads, self.head_dim)
        if kn.stride(-1) != 1 or kn.stride() != vn.stride():
            kn, vn = kn.contiguous(), vn.contiguous()
        g = g_new.reshape(B).to(torch.float32).contiguous()
        evict = st.recent_filled >= self.window
        metrics, fr = self._aux_buffers(st, dev) if evict else (None, None)
        eta = self._eta_f32(dev, st.k_buf.dtype) if self.Ms > 0 else None
        tr = torch.full((B, 4), -1, dtype=torch.int32, device=dev) if evict and self._tracing() else None
        d = self._bank_desc(st, eta, metrics, fr, tr)
        _hip.check(_hip.lib().coda_decode_write(
            d, kn.data_ptr(), vn.data_ptr(), kn.stride(0), kn.stride(1), g.data_ptr(), int(st.recent_idx),
            int(st.recent_filled), int(st.pos), _hip.stream_of(kn)))
        if not evict:
            st.recent_filled += 1
        else:
            j = int(st.recent_idx)
            self._trace_decode(tr)
            self._fold_metrics(st, metrics, 1, self.Me > 0, self.Ms > 0)
            self._expand_from(st, fr, False, self.Me > 0, self.Ms > 0)
            st.recent_idx = (j + 1) % self.window
        st.pos += 1

    def _decode_step(self, st: CoDAGQALandmarkStatePerf2, *, k_new: torch.Tensor, v_new: torch.Tensor,
                     g_new: torch.Tensor, attn_desc, k_roped: bool = True) -> None:
        """Write one token then attend (coda_decode_step): the bank update of
        _write_one and the attention described by attn_desc, in one call.
        k_roped False: k_new is the raw projection, roped by the kernels with
        the query's tables (coda_decode_step_raw_k).

        The library leaves the routing record of the next token in the
        workspace; it is handed back (one launch per token) only while this
        module sees an unbroken sequence of decode steps on the same state:
        same state object, same buffers, no in-place edit of them through
        torch (version counters), position and ring index as the last step
        left them."""
        self._check_state(st)
        B = st.k_buf.shape[0]
        dev = st.k_buf.device
        kn = k_new.reshape(B, self.num_kv_heads, self.head_dim)
        vn = v_new.reshape(B, self.num_kv_heads, self.head_dim)
        if kn.stride(-1) != 1 or kn.stride() != vn.stride():
            kn, vn = kn.contiguous(), vn.contiguous()
        g = g_new.reshape(B).to(torch.float32).contiguous()
        evict = st.recent_filled >= self.window
        metrics, fr = self._aux_buffers(st, dev) if evict else (None, None)
        eta = self._eta_f32(dev, st.k_buf.dtype) if self.Ms > 0 else None
        tr = torch.full((B, 4), -1, dtype=torch.int32, device=dev) if evict and self._tracing() else None
        d = self._bank_desc(st, eta, metrics, fr, tr)
        L = _hip.lib()
        wkey = (B, attn_desc.H, st.k_buf.shape[2], st.k_buf.dtype)
        sizes = self.__dict__.setdefault("_step_ws_bytes", {})
        need = sizes.get(wkey)
        if need is None:
            nb = ctypes.c_size_t(0)
            _hip.check(L.coda_decode_step_workspace_bytes(d, attn_desc, nb))
            need = sizes[wkey] = nb.value
        ws = self._route_workspace(dev, need)
        routed = ctypes.c_int(1 if self.__dict__.get("_route_tag") == self._route_key(st, ws) else 0)
        self.__dict__["_route_tag"] = None
        fn = L.coda_decode_step if k_roped else L.coda_decode_step_raw_k
        _hip.check(fn(
            d, attn_desc, kn.data_ptr(), vn.data_ptr(), kn.stride(0), kn.stride(1), g.data_ptr(),
            int(st.recent_idx), int(st.recent_filled), int(st.pos), _hip.ptr(ws), need, ctypes.byref(routed),
            _hip.stream_of(kn)))
        if not evict:
            st.recent_filled += 1
        else:
            j = int(st.recent_idx)
            self._trace_decode(tr)
            self._fold_metrics(st, metrics, 1, self.Me > 0, self.Ms > 0)
            self._expand_from(st, fr, False, self.Me > 0, self.Ms > 0)
            st.recent_idx = (j + 1) % self.window
        st.pos += 1
        if routed.value:
            self.__dict__["_route_tag"] = self._route_key(st, ws)

    # ------------------------------------------------------------ decode plan
    def _plan_key(self, st: CoDAGQALandmarkStatePerf2, q: torch.Tensor):
        """Everything the cached descriptors of a decode step depend on."""
        w = self.head_norm.weight if self.head_norm_mode == "full" else None
        return (id(st), st.k_buf.data_ptr(), st.v_buf.data_ptr(), st.allowed.data_ptr(), st.g_recent.data_ptr(),
                st.mem_last_exact.data_ptr(), _hip.ptr(st._exact_v_norm), _hip.ptr(st._sum_lf_k_norm),
                st.active_exact, st.active_summary, q.dtype, q.shape[0], q.device, self.theta._version,
                None if w is None else w._version, self.summary_eta_logit._version)

    def _decode_step_planned(self, st: CoDAGQALandmarkStatePerf2, q, k_new, v_new, g_new, lam, rope_cos, rope_sin,
                             out, k_roped: bool = True) -> bool:
        """Steady-state decode step through descriptors cached per state:
        full ring, no metrics dict, fixed bank sizes.  Per call only the
        token's pointers change, so the host side is a few field updates and
        one library call.  Returns False when the general path must run."""
        if st.metrics is not None or st.recent_filled < self.window or self._expandable() or \
                (self.Me == 0 and self.Ms == 0) or self._tracing():
            return False
        plan = self.__dict__.get("_dplan")
        key = self._plan_key(st, q)
        if plan is None or plan["key"] != key:
            self.__dict__["_dplan"] = None
            self._check_state(st)
            key = self._plan_key(st, q)
            dt = q.dtype
            ct, sn = self._theta_tables(dt)
            B, H, Dh = q.shape[0], self.num_heads, self.head_dim
            a, keep = ops.attention_desc(
                q=q, rope_cos=rope_cos, rope_sin=rope_sin, rope_interleaved=self.rope_interleaved, theta_cos=ct,
                theta_sin=sn, k_prefix=st.k_buf, v_prefix=st.v_buf,
                allowed=st.allowed if self.mask_unused_memory else None, k_block=None, v_block=None, lam=lam,
                rms_weight=self._rms_weight(dt), eps=self._eps, out=out.permute(0, 2, 1, 3))
            eta = self._eta_f32(q.device, st.k_buf.dtype) if self.Ms > 0 else None
            d = self._bank_desc(st, eta, None, None)
            nb = ctypes.c_size_t(0)
            _hip.check(_hip.lib().coda_decode_step_workspace_bytes(d, a, nb))
            ws = self._route_workspace(q.device, nb.value)
            plan = {"key": key, "attn": a, "bank": d, "keep": (keep, ct, sn, eta, self._rms_weight(dt)),
                    "ws": ws, "ws_ptr": _hip.ptr(ws), "ws_bytes": nb.value, "routed": ctypes.c_int(0),
                    "fn": _hip.lib().coda_decode_step, "fn_raw_k": _hip.lib().coda_decode_step_raw_k}
            self.__dict__["_dplan"] = plan
        a = plan["attn"]
        a.q = q.data_ptr()
        a.q_sb, a.q_sh, a.q_sl = q.stride()[:3]
        a.rope_cos, a.rope_sin = rope_cos.data_ptr(), rope_sin.data_ptr()
        a.lam = lam.data_ptr()
        a.lam_sb, a.lam_sh, a.lam_sl = lam.stride()
        a.out = out.data_ptr()
        ob, ol, oh = out.stride()[:3]
        a.o_sb, a.o_sh, a.o_sl = ob, oh, ol
        # (B, Hkv, 1, Dh) or (B, Hkv, Dh): sequence / head strides, unit channel stride
        kst, vst = k_new.stride(), v_new.stride()
        if kst[-1] != 1 or kst[:2] != vst[:2] or vst[-1] != 1 or g_new.dtype != torch.float32 or \
                g_new.stride(-1) != 1 or rope_cos.stride(-1) != 1 or rope_sin.stride(-1) != 1:
            return False
        routed = plan["routed"]
        tag = self._route_key(st, plan["ws"])
        routed.value = 1 if self.__dict__.get("_route_tag") == tag else 0
        self.__dict__["_route_tag"] = None
        fn = plan["fn"] if k_roped else plan["fn_raw_k"]
        _hip.check(fn(plan["bank"], a, k_new.data_ptr(), v_new.data_ptr(), kst[0], kst[1], g_new.data_ptr(),
                              int(st.recent_idx), int(st.recent_filled), int(st.pos), plan["ws_ptr"],
                              plan["ws_bytes"], ctypes.byref(routed), _hip.stream_of(q)))
        j = int(st.recent_idx)
        st.recent_idx = 0 if j + 1 == self.window else j + 1
        st.pos += 1
        if routed.value:
            self.__dict__["_route_tag"] = self._route_key(st, plan["ws"])
        return True

    @staticmethod
    def _route_key(st: CoDAGQALandmarkStatePerf2, ws: Optional[torch.Tensor]):
        ts = (st.k_buf, st.v_buf, st.allowed, st.g_recent, st.mem_last_exact, st._exact_v_norm, st._sum_lf_k_norm)
        return (id(st), int(st.pos), int(st.recent_idx), None if ws is None else ws.data_ptr()) + tuple(
            (None, None) if t is None else (t.data_ptr(), t._version) for t in ts)

    def _route_workspace(self, device, nbytes: int) -> Optional[torch.Tensor]:
        """Workspace of the decode step (routing records), kept apart from
        the other scratch buffers so nothing else overwrites a record."""
        if nbytes == 0:
            return None
        cache = self.__dict__.setdefault("_route_ws", {})
        key = str(device)
        buf = cache.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
            cache[key] = buf
        return buf

    def _workspace(self, device, nbytes: int) -> Optional[torch.Tensor]:
        """Device scratch reused across calls (grown on demand); calls on one
        stream run in order, so reuse needs no synchronisation."""
        if nbytes == 0:
            return None
        cache = self.__dict__.setdefault("_ws_cache", {})
        key = str(device)
        buf = cache.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
            cache[key] = buf
        return buf

    # ------------------------------------------------------------ prefill
    def _plan_candidates(self, st, g_seq: torch.Tensor, L: int, block_size: int):
        """Candidate order of every chunk (memory_banks.py:459-510)."""
        do_e = self.Me > 0 and self.exact_candidates_per_block > 0
        do_s = self.Ms > 0 and self.summary_candidates_per_block > 0
        kmax = max(self.exact_candidates_per_block if do_e else 0, self.summary_candidates_per_block if do_s else 0)
        kmax = max(1, min(kmax, block_size))
        n_chunks = (L + block_size - 1) // block_size
        B = g_seq.shape[0]
        plan = torch.empty((n_chunks, B, kmax), dtype=torch.int32, device=g_seq.device)
        if do_e or do_s:
            head = int(st.recent_idx) if st.recent_filled >= self.window else 0
            _hip.check(_hip.lib().coda_block_plan(
                st.g_recent.data_ptr(), head, int(st.recent_filled), self.window, g_seq.data_ptr(),
                g_seq.stride(0), B, L, block_size, self.exact_candidates_per_block,
                self.summary_candidates_per_block, int(do_e), int(do_s), plan.data_ptr(), kmax,
                _hip.stream_of(g_seq)))
        return plan, kmax, do_e, do_s

    def _write_block(self, st, *, k_blk: torch.Tensor, v_blk: torch.Tensor, g_blk: torch.Tensor, pos0: int,
                     ring_head: int, ring_filled: int, plan_c: torch.Tensor, kmax: int, do_e: bool, do_s: bool,
                     workspace: Optional[torch.Tensor], eta: Optional[torch.Tensor], snap=None):
        """Evict / update banks / ring write for one chunk (memory_banks.py:438-564).

        k_blk, v_blk (B, Hkv, blk, Dh) views; g_blk (B, blk) float32 view.
        snap: (K, V, visibility bytes) tensors that receive the bank slots
        as they stand before this chunk's update; the one-launch update
        writes them (coda_block_write_snapshot), any other chunk copies them
        first.  Returns the ring (head, filled) after the chunk, or None when
        snap is given and the one-launch update does not run for this chunk
        (nothing has run then).
        """
        B, Hkv, blk, Dh = k_blk.shape
        W = self.window
        total = ring_filled + blk
        keep_len = min(W, total)
        n_ev = total - keep_len
        Te = min(self.exact_candidates_per_block, n_ev) if do_e else 0
        Ts = min(self.summary_candidates_per_block, n_ev) if do_s else 0
        metrics, fr = self._aux_buffers(st, k_blk.device) if n_ev > 0 else (None, None)
        tr = None
        if n_ev > 0 and (Te > 0 or Ts > 0) and self._tracing():
            tr = torch.full((B, 2 * Te + Ts), -1, dtype=torch.int32, device=k_blk.device)
        d = self._bank_desc(st, eta, metrics, fr, tr)
        ws_ptr, ws_bytes = (workspace.data_ptr(), workspace.numel()) if workspace is not None else (None, 0)
        if k_blk.stride() != v_blk.stride() or k_blk.stride(-1) != 1:
            v_blk = v_blk.contiguous()
            k_blk = k_blk.contiguous()
        args = (d, k_blk.data_ptr(), v_blk.data_ptr(), k_blk.stride(0), k_blk.stride(1), k_blk.stride(2),
                g_blk.data_ptr(), g_blk.stride(0), blk, ring_head, ring_filled, int(pos0), _hip.ptr(plan_c), kmax,
                Te, Ts, ws_ptr, ws_bytes)
        if snap is not None and n_ev > 0 and (Te > 0 or Ts > 0):
            rc = _hip.lib().coda_block_write_snapshot(*args, snap[0].data_ptr(), snap[1].data_ptr(),
                                                      snap[2].data_ptr(), _hip.stream_of(k_blk))
            if rc == _hip.CODA_EUNSUP:
                return None
            _hip.check(rc)
        else:
            if snap is not None:
                W_ = self.window
                snap[0].copy_(st.k_buf[:, :, W_:])
                snap[1].copy_(st.v_buf[:, :, W_:])
                snap[2].copy_(st.allowed[:, W_:].view(torch.uint8))
            _hip.check(_hip.lib().coda_block_write(*args, _hip.stream_of(k_blk)))
        if n_ev > 0:
            self._trace_block(tr, plan_c, Te, Ts)
            self._fold_metrics(st, metrics, n_ev, Te > 0, Ts > 0)
            self._expand_from(st, fr, True, Te > 0, Ts > 0)
        head = ring_head if ring_filled == W else 0
        if keep_len == W:
            head = (head + n_ev) % W
        return head, keep_len

    def _block_workspace(self, st, kmax: int) -> Optional[torch.Tensor]:
        """Scratch of the chunk updates, kept per device and batch and zeroed
        once when made: its tail holds the per-sequence generation words and
        the status word (coda_block_write), which carry over between calls."""
        need = ctypes.c_size_t(0)
        d = self._bank_desc(st, None, None, None)
        _hip.check(_hip.lib().coda_block_workspace_bytes(d, kmax, need))
        if need.value == 0:
            return None
        self.check_bank_status(wait=False)
        cache = self.__dict__.setdefault("_block_ws", {})
        key = (str(st.k_buf.device), st.k_buf.shape[0])
        buf = cache.get(key)
        if buf is None or buf.numel() < need.value:
            # tail words at the end of the buffer: a new size starts them over
            buf = cache[key] = torch.zeros(need.value, dtype=torch.uint8, device=st.k_buf.device)
        return buf

    @staticmethod
    def _status_word(ws: torch.Tensor) -> torch.Tensor:
        n = (ws.numel() // 8) * 8
        return ws[n - 8:n].view(torch.int64)

    def _queue_status_check(self, ws: Optional[torch.Tensor]) -> None:
        """After a prefill call: copy the workspace's status word to pinned
        host memory behind the call's kernels (no host sync); the next entry
        into the layer, or check_bank_status(), reads it."""
        if ws is None:
            return
        host = torch.empty(1, dtype=torch.int64, pin_memory=True)
        host.copy_(self._status_word(ws), non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(ws.device))
        self.__dict__.setdefault("_status_pending", []).append((ev, host, ws))

    def check_bank_status(self, wait: bool = True) -> None:
        """Raise if a chunk update of an earlier prefill call gave up waiting
        for the other heads of its sequence (its bank state is then
        incomplete).  wait=False reads only the status copies that have
        already landed, without a host sync."""
        pend = self.__dict__.get("_status_pending")
        while pend:
            ev, host, ws = pend[0]
            if not ev.query():
                if not wait:
                    return
                ev.synchronize()
            pend.pop(0)
            n = int(host[0])
            if n:
                pend.clear()
                self._status_word(ws).zero_()
                raise RuntimeError(
                    f"coda_block_write: {n} workgroup(s) of a prefill chunk's bank update gave up waiting for the "
                    "other heads of their sequence; that call's bank state is incomplete and must be discarded "
                    "(re-run the prefill from a saved state)")

    def _ring_to_time_order(self, st, head: int, filled: int) -> None:
        """Circular ring -> time order at slots 0..filled-1 (memory_banks.py:152-177)."""
        if filled == self.window and head != 0:
            B = st.k_buf.shape[0]
            e = st.k_buf.element_size()
            need = B * self.num_kv_heads * self.window * self.head_dim * 2 * e + B * self.window * 4
            ws = torch.empty(need, dtype=torch.uint8, device=st.k_buf.device)
            d = self._bank_desc(st, None, None, None)
            _hip.check(_hip.lib().coda_ring_rotate(d, head, ws.data_ptr(), need, _hip.stream_of(st.k_buf)))
        st.recent_idx = 0
        st.recent_filled = int(filled)
