"""The metrics dict of a state with device-side counters: values fold in on
read (host logic, exercised with CPU tensors standing in for the device
accumulator); pickled it is a plain mapping of the folded values, and
save_state writes the reference's plain dict."""

from __future__ import annotations

import io
import os
import pickle
import tempfile

import torch


def _metrics():
    from coda_gqa_l import _hip
    from coda_gqa_l.memory_banks import METRIC_KEYS, DeviceMetrics
    mt = DeviceMetrics({k: (0.0 if k.endswith("ratio") else 0) for k in METRIC_KEYS})
    return mt, _hip


def test_counters_fold_in_on_first_read():
    mt, _hip = _metrics()
    acc = mt.accumulator("cpu")
    acc[_hip.CNT_EXACT_HITS] += 3
    acc[_hip.CNT_SUMMARY_UPDATES] += 5
    acc[_hip.NUM_COUNTERS] += 1                  # summary_frustrated
    mt.add_host("total_evictions", 7)
    mt.fill["exact_fill_ratio"] = torch.tensor(0.25)
    assert dict.__getitem__(mt, "exact_hits") == 0   # nothing folded yet
    assert mt["exact_hits"] == 3
    assert mt["summary_updates"] == 5 and mt["summary_frustrated"] == 1
    assert mt["total_evictions"] == 7 and mt["exact_fill_ratio"] == 0.25
    assert int(acc.sum()) == 0 and not mt.fill    # folded once
    acc[_hip.CNT_EXACT_HITS] += 2
    assert dict(mt)["exact_hits"] == 5               # dict() copies through the fold as well


def test_pickles_as_a_plain_mapping_and_saves_as_a_dict():
    from coda_gqa_l import CoDAGQALandmarkStatePerf2
    from coda_gqa_l.memory_banks import DeviceMetrics
    from coda_gqa_l.state_io import load_state, save_state
    mt, _hip = _metrics()
    mt.accumulator("cpu")[_hip.CNT_EXACT_INSERTS] += 4
    d = pickle.loads(pickle.dumps(mt))
    assert isinstance(d, dict) and not isinstance(d, DeviceMetrics) and d["exact_inserts"] == 4
    buf = io.BytesIO()
    torch.save({"m": mt}, buf)
    buf.seek(0)
    d = torch.load(buf, weights_only=True)["m"]
    assert not isinstance(d, DeviceMetrics) and d == dict(mt)
    z = torch.zeros(1, 1, 4, 2)
    st = CoDAGQALandmarkStatePerf2(k_buf=z, v_buf=z, allowed=torch.ones(1, 4, dtype=torch.bool),
                                   g_recent=torch.zeros(1, 2), recent_idx=0, recent_filled=2,
                                   mem_last_exact=torch.zeros(1, 1, dtype=torch.int64), pos=2, active_exact=1,
                                   active_summary=1, metrics=mt)
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "s.pt")
        save_state({"states": {0: st}}, path)
        got = load_state(path)["states"][0].metrics
    assert type(got) is dict and got["exact_inserts"] == 4


def test_direct_writes_fold_pending_counts_first():
    """A key reset directly (reset_metrics, or metrics[k] = 0 on the
    reference's plain dict) stays reset: counts pending on the device at the
    time of the write are folded in before it, not added on the next read."""
    mt, _hip = _metrics()
    acc = mt.accumulator("cpu")
    acc[_hip.CNT_EXACT_HITS] += 3
    acc[_hip.CNT_EXACT_INSERTS] += 2
    mt["exact_hits"] = 0
    assert mt["exact_hits"] == 0 and mt["exact_inserts"] == 2
    acc[_hip.CNT_EXACT_INSERTS] += 5
    mt.update(exact_inserts=1)
    assert mt["exact_inserts"] == 1
    acc[_hip.CNT_SUMMARY_UPDATES] += 4
    assert mt.setdefault("summary_updates", 99) == 4
    acc[_hip.CNT_SUMMARY_INSERTS] += 6
    assert mt.pop("summary_inserts") == 6
    acc[_hip.CNT_TOKENS_GATED_OUT] += 1
    mt.clear()
    assert len(mt) == 0 and int(acc.sum()) == 0
