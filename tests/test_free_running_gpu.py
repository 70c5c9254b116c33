"""Long free-running streams at configs[0]'s shape, HIP path against the
CPU oracle: each side keeps its own state for the whole stream (no reset
from the oracle between calls), every slot decision of every chunk and
decode step is compared (candidate ids, exact idx / overwrite / touch,
summary routing idx), and the whole state after every call.  The stream
stops at the first decision that differs and reports the oracle's margin
there (the score gap between the two best slots and the distance to the
cosine thresholds)."""

from __future__ import annotations

import pytest
import torch

from parity_util import assert_close, compare_states, compare_traces, product_like, to_product_state

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

C1 = dict(embed_dim=512, num_heads=8, num_kv_heads=2, window=256, num_landmarks_exact=64,
          num_landmarks_summary=64)


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


# (dtype, batch, prefill tokens, tokens per prefill call, decode steps)
STREAMS = {
    "c1_f32_b1": (torch.float32, 1, 8192, 1024, 512),
    "c1_bf16_b1": (torch.bfloat16, 1, 8192, 1024, 512),
    "c1_bf16_b4": (torch.bfloat16, 4, 8192, 2048, 256),
}


@pytest.mark.parametrize("name", list(STREAMS))
@torch.no_grad()
def test_free_running_stream_decisions_match_oracle(name):
    _need_gpu()
    from coda_oracle import OracleLayer, banks, prims
    dtype, B, L, per_call, steps = STREAMS[name]
    print(f"[free-running] {name}: C1 shape, {dtype}, B{B}, {L} prefill tokens in calls of {per_call} "
          f"(block 256), then {steps} decode steps", flush=True)
    torch.manual_seed(0)
    m = OracleLayer(**C1).to(dtype).eval()
    p = product_like(m, {"kw": C1}, dtype, DEV)
    torch.manual_seed(1)
    st_o = m.init_state(batch_size=B, dtype=dtype)
    st_p = to_product_state(st_o, DEV)
    W, Me, H, Hkv, Dh = m.window, m.Me, m.num_heads, m.num_kv_heads, m.head_dim
    g = torch.Generator().manual_seed(2)
    n_events = 0
    for c0 in range(0, L, per_call):
        n = min(per_call, L - c0)
        # post-projection inputs of real token activations: x ~ N(0, 1)
        # through the layer's own projections on the CPU
        x = torch.randn(B, n, C1["embed_dim"], generator=g).to(dtype)
        q, k, v, gate, lam = m.project(x)
        c, s = m.rope_tables(n, st_o.pos, dtype)
        k_r = prims.rope(k, c, s, m.rope_interleaved)
        tr_o = []
        p.decision_trace = []
        heads_o = m.prefill_core(prims.rope(q, c, s, m.rope_interleaved), k_r, v, gate, lam, st_o, block_size=256,
                                 trace=tr_o)
        heads_p = p.prefill_core(q.to(DEV), k_r.to(DEV), v.to(DEV), gate.to(DEV), lam.squeeze(-1).to(DEV),
                                 c.to(DEV), s.to(DEV), st_p, block_size=256)
        torch.cuda.synchronize()
        what = f"{name} prefill tokens [{c0}, {c0 + n})"
        n_events += compare_traces(p.decision_trace, tr_o, m, what)
        assert_close(heads_p.permute(0, 2, 1, 3), heads_o, dtype, f"{what} heads")
        compare_states(st_p, st_o, dtype, W, Me, what)
    p.decision_trace = None
    print(f"[free-running] {name}: prefill of {L} tokens, {n_events} decision events identical", flush=True)
    for t in range(steps):
        x = torch.randn(B, 1, C1["embed_dim"], generator=g).to(dtype)
        qp = int(st_o.pos)
        kn, vn, gn = m._new_kv(x, qp)
        qt = m.q_proj(x).view(B, 1, H, Dh).transpose(1, 2)
        lamt = torch.sigmoid(m.lambda_proj(x)).transpose(1, 2).unsqueeze(-1)
        tr_o = []
        p.decision_trace = []
        banks.write_one(m, st_o, kn, vn, gn, tr_o)
        ho = m.attend_core(qt, lamt, st_o, qp)
        ct, sn = m.rope_tables(1, qp, dtype)
        hp = p.decode_step_core(qt.to(DEV), kn.to(DEV), vn.to(DEV), gn.reshape(B).to(DEV), lamt.squeeze(-1).to(DEV),
                                st_p, ct.to(DEV), sn.to(DEV))
        torch.cuda.synchronize()
        what = f"{name} decode step {t} (position {qp})"
        n_events += compare_traces(p.decision_trace, tr_o, m, what)
        assert_close(hp.permute(0, 2, 1, 3), ho, dtype, f"{what} heads")
        compare_states(st_p, st_o, dtype, W, Me, what)
    p.decision_trace = None
    print(f"[free-running] {name}: {n_events} decision events identical, 0 flips", flush=True)
