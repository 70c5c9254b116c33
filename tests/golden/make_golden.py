"""Write golden vectors for the bounded-attention hot path from the reference.

Run in the build container only (the reference is not present on the GPU
box):  python tests/golden/make_golden.py [/root/reference]

It imports anthony-maio/CoDA-GQA-L from <reference>/src, runs seeded CPU
prefill + decode trajectories (eval mode, the reference's CPU/PyTorch path),
and records, per case, into tests/golden/<case>.npz:
  - the seeds that generate weights, initial state and inputs, plus
    checksums of each so the test can verify it regenerated them exactly;
  - prefill / decode outputs (full for small cases, strided rows plus a
    sha256 of the whole tensor for large ones);
  - every slot decision, read from the reference's own locals when its bank
    functions return (sys.setprofile): candidate order of the block topk,
    exact idx/overwrite/touch, summary routing idx, decode idx/overwrite;
  - the final state (buffers, masks, LRU stamps, ring ints, norm caches).
Nothing from the reference is pickled: arrays and ints only.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from cases import CASES, make_inputs  # noqa: E402

WATCH = {
    "_write_block_fast": ("select", ("idxs_all", "idxs", "idxs_s")),
    "_exact_update_block_vectorized": ("exact_block", ("idx_tok", "overwrite_tok", "touch_tok")),
    "_summary_update_block_hard": ("summary_block", ("idx_tok",)),
    "_exact_update_one": ("exact_one", ("idx", "overwrite", "keep_b")),
    "_summary_update_one": ("summary_one", ("idx", "keep_b")),
}


class Recorder:
    def __init__(self):
        self.events = []

    def __call__(self, frame, event, arg):
        if event != "return":
            return
        name = frame.f_code.co_name
        if name not in WATCH or "memory_banks" not in frame.f_code.co_filename:
            return
        tag, keys = WATCH[name]
        loc = frame.f_locals
        vals = []
        for k in keys:
            if k in loc and torch.is_tensor(loc[k]):
                vals.append(loc[k].detach().clone())
        if tag == "select":
            if vals:
                self.events.append((tag, vals[0]))
        elif vals:
            self.events.append((tag, *vals))


def to_np(t):
    t = t.detach()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy()  # raw bits
    return t.numpy()


def checksum(t):
    """sha256 of the raw bytes (thread-count independent), as uint8 array."""
    import hashlib
    t = t.detach().contiguous()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return np.frombuffer(hashlib.sha256(t.numpy().tobytes()).digest(), dtype=np.uint8)


def main(ref_root):
    sys.path.insert(0, os.path.join(ref_root, "src"))
    from coda_gqa_l import CoDAGQALandmarkPerf2  # noqa: E402  (reference, read-only)

    torch.set_num_threads(1)
    meta_all = {}
    for name, case in CASES.items():
        dtype = getattr(torch, case["dtype"])
        torch.manual_seed(case["seed_model"])
        ref = CoDAGQALandmarkPerf2(**case["kw"]).to(dtype=dtype).eval()
        x, xs = make_inputs(case)
        torch.manual_seed(case["seed_state"])
        st = ref.init_state(batch_size=case["B"], device=torch.device("cpu"), dtype=dtype,
                            mem_init=case.get("mem_init"))
        rec = Recorder()
        out = {}
        with torch.no_grad():
            sys.setprofile(rec)
            try:
                y, st = ref.prefill_chunked(x, st, block_size=case["block"], write_cache=True,
                                            return_outputs=True)
                n_pref = len(rec.events)
                ys = []
                for xt in xs:
                    yt, st = ref.step(xt, st)
                    ys.append(yt)
            finally:
                sys.setprofile(None)
        out["weights_ck"] = np.array([checksum(p) for _, p in sorted(ref.state_dict().items())])
        out["x_ck"] = np.array(checksum(x))
        rows = case.get("y_rows")
        out["y_prefill"] = to_np(y if rows is None else y[:, ::rows])
        out["y_prefill_ck"] = np.array(checksum(y))
        if ys:
            out["y_decode"] = to_np(torch.cat(ys, dim=1))
        for f in ("k_buf", "v_buf", "allowed", "g_recent", "mem_last_exact", "_exact_v_norm", "_sum_lf_k_norm"):
            v = getattr(st, f)
            if v is not None:
                out["state_" + f] = to_np(v)
        ints = [st.recent_idx, st.recent_filled, st.pos, st.active_exact, st.active_summary]
        out["state_ints"] = np.array(ints, dtype=np.int64)
        if st.metrics is not None:
            out["metrics_json"] = np.frombuffer(json.dumps(st.metrics, sort_keys=True).encode(), dtype=np.uint8)
        tags = []
        for i, ev in enumerate(rec.events):
            tag = ev[0]
            tags.append(tag)
            for j, t in enumerate(ev[1:]):
                out[f"ev{i:05d}_{j}"] = to_np(t)
        out["ev_tags"] = np.frombuffer(json.dumps(tags).encode(), dtype=np.uint8)
        out["n_prefill_events"] = np.array(n_pref)
        out["torch_version"] = np.frombuffer(torch.__version__.encode(), dtype=np.uint8)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **out)
        meta_all[name] = {"events": len(rec.events), "bytes": os.path.getsize(path)}
        print(name, meta_all[name], flush=True)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
