"""Helpers to replay the golden cases (tests/golden/*.npz) on the oracle."""

from __future__ import annotations

import json
import os

import numpy as np
import torch

from cases import CASES, GPU_CASES, make_inputs

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    z = np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)
    return {k: z[k] for k in z.files}


def checksum(t):
    """sha256 of the raw bytes (thread-count independent), as uint8 array."""
    import hashlib
    t = t.detach().contiguous()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return np.frombuffer(hashlib.sha256(t.numpy().tobytes()).digest(), dtype=np.uint8)


def from_np(a, like_dtype):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if like_dtype == torch.bfloat16 and t.dtype == torch.int16:
        return t.view(torch.bfloat16)
    return t


def events(g):
    """Golden events grouped by tag: {tag: [tuple of tensors]} in call order."""
    tags = json.loads(bytes(g["ev_tags"]).decode())
    out = {}
    for i, tag in enumerate(tags):
        vals = []
        j = 0
        while f"ev{i:05d}_{j}" in g:
            vals.append(torch.from_numpy(g[f"ev{i:05d}_{j}"]))
            j += 1
        out.setdefault(tag, []).append(tuple(vals))
    return out


def trace_events(trace):
    out = {}
    for ev in trace:
        out.setdefault(ev[0], []).append(tuple(t.clone() for t in ev[1:]))
    return out


def build_oracle(name):
    from coda_oracle import OracleLayer
    case = CASES[name] if name in CASES else GPU_CASES[name]
    dtype = getattr(torch, case["dtype"])
    torch.manual_seed(case["seed_model"])
    m = OracleLayer(**case["kw"]).to(dtype=dtype).eval()
    return case, dtype, m
