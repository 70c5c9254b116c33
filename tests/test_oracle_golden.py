"""Pin the CPU oracle to the reference: replay every golden case bit-exactly.

The golden vectors were written by tests/golden/make_golden.py from the
reference's own CPU path; nothing here imports the reference.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from cases import CASES, make_inputs
from golden_util import build_oracle, checksum, events, from_np, load, trace_events


def _eq(a, b, what):
    assert a.shape == b.shape, (what, a.shape, b.shape)
    assert torch.equal(a, b), f"{what}: {(a != b).sum().item()} mismatches"


@pytest.mark.parametrize("name", sorted(CASES))
@torch.no_grad()
def test_oracle_matches_reference_trajectory(name):
    g = load(name)
    case, dtype, m = build_oracle(name)
    ck = np.array([checksum(p) for _, p in sorted(m.state_dict().items())])
    np.testing.assert_array_equal(ck, g["weights_ck"], err_msg="weights not regenerated")
    x, xs = make_inputs(case)
    np.testing.assert_array_equal(np.array(checksum(x)), g["x_ck"])
    torch.manual_seed(case["seed_state"])
    st = m.init_state(batch_size=case["B"], dtype=dtype, mem_init=case.get("mem_init"))
    trace = []
    y, st = m.prefill_chunked(x, st, block_size=case["block"], trace=trace)
    ys = []
    for xt in xs:
        yt, st = m.step(xt, st, trace=trace)
        ys.append(yt)

    rows = case.get("y_rows")
    _eq(y if rows is None else y[:, ::rows], from_np(g["y_prefill"], dtype), "prefill y")
    np.testing.assert_array_equal(checksum(y), g["y_prefill_ck"])
    if ys:
        _eq(torch.cat(ys, dim=1), from_np(g["y_decode"], dtype), "decode y")
    for f in ("k_buf", "v_buf", "allowed", "g_recent", "mem_last_exact", "_exact_v_norm", "_sum_lf_k_norm"):
        v = getattr(st, f)
        if v is None:
            assert "state_" + f not in g
        else:
            _eq(v, from_np(g["state_" + f], v.dtype), f)
    ints = [st.recent_idx, st.recent_filled, st.pos, st.active_exact, st.active_summary]
    assert ints == list(g["state_ints"])
    if "metrics_json" in g:
        assert st.metrics == json.loads(bytes(g["metrics_json"]).decode())

    ge, oe = events(g), trace_events(trace)
    assert sorted(ge) == sorted(oe), (sorted(ge), sorted(oe))
    for tag in ge:
        assert len(ge[tag]) == len(oe[tag]), tag
        for i, (a, b) in enumerate(zip(ge[tag], oe[tag])):
            for j, (ta, tb) in enumerate(zip(a, b)):
                _eq(tb.to(ta.dtype), ta, f"{tag}[{i}][{j}]")
