"""Oracle evidence for the pieces around the hot path:

- a state file written from an oracle trajectory (the reference's format,
  neural_db.py:285-308), loaded back with weights_only=True, decodes on the
  HIP path exactly as the oracle continues from its own state;
- two bounded Llama-adapter layers (llama_adapter.py:308-383), under
  eviction, give the oracle's outputs and decisions in a multi-layer
  prefill + decode loop (examples/bounded_generate.py:200-300);
- bank metrics accumulate on the device: a prefill and decode steps with
  collect_metrics run with every torch synchronising operation made an
  error, and the metrics read afterwards equal the oracle's
  (memory_banks.py:117-140)."""

from __future__ import annotations

import os
import tempfile

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


def _oracle_prefill(m, st, B, L, dtype, g, block=256):
    from coda_oracle import prims
    x = torch.randn(B, L, m.embed_dim, generator=g).to(dtype)
    q, k, v, gate, lam = m.project(x)
    c, s = m.rope_tables(L, st.pos, dtype)
    m.prefill_core(prims.rope(q, c, s, m.rope_interleaved), prims.rope(k, c, s, m.rope_interleaved), v, gate, lam,
                   st, block_size=block)


@torch.no_grad()
def test_oracle_state_file_decodes_like_the_oracle():
    _need_gpu()
    from coda_oracle import OracleLayer, banks
    from coda_gqa_l import CoDAGQALandmarkStatePerf2
    from coda_gqa_l.state_io import load_state, save_state, state_to_device
    dtype, B = torch.bfloat16, 2
    print("[state file] C1 bf16 B2: oracle prefill 1536 tokens -> file -> HIP decode 64 steps", flush=True)
    torch.manual_seed(0)
    m = OracleLayer(**C1).to(dtype).eval()
    p = product_like(m, {"kw": C1}, dtype, DEV)
    torch.manual_seed(1)
    st_o = m.init_state(batch_size=B, dtype=dtype)
    g = torch.Generator().manual_seed(2)
    _oracle_prefill(m, st_o, B, 1536, dtype, g)
    cpu = lambda t: None if t is None else t.clone()
    st_file = CoDAGQALandmarkStatePerf2(
        k_buf=cpu(st_o.k_buf), v_buf=cpu(st_o.v_buf), allowed=cpu(st_o.allowed), g_recent=cpu(st_o.g_recent),
        recent_idx=st_o.recent_idx, recent_filled=st_o.recent_filled, mem_last_exact=cpu(st_o.mem_last_exact),
        pos=st_o.pos, active_exact=st_o.active_exact, active_summary=st_o.active_summary,
        _exact_v_norm=cpu(st_o._exact_v_norm), _sum_lf_k_norm=cpu(st_o._sum_lf_k_norm), metrics=None)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "state.pt")
        assert save_state({"states": {0: st_file}, "metadata": {"tokens": 1536}}, path) > 0
        loaded = load_state(path)
    assert loaded["metadata"] == {"tokens": 1536}
    st_p = state_to_device(loaded["states"][0], DEV, dtype)
    compare_states(st_p, st_o, dtype, m.window, m.Me, "restored state")
    H, Hkv, Dh = m.num_heads, m.num_kv_heads, m.head_dim
    n_events = 0
    for t in range(64):
        x = torch.randn(B, 1, m.embed_dim, generator=g).to(dtype)
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
        what = f"restored state, decode step {t}"
        n_events += compare_traces(p.decision_trace, tr_o, m, what)
        p.decision_trace = None
        assert_close(hp.permute(0, 2, 1, 3), ho, dtype, f"{what} heads")
        compare_states(st_p, st_o, dtype, m.window, m.Me, what)
    print(f"[state file] {n_events} decision events identical", flush=True)


def _compare_close_states(sp, so, what, tol=1e-4):
    """Decisions exact (visibility bytes, LRU stamps, ring ints, ring gates);
    values within tol (device and CPU GEMMs round differently)."""
    assert torch.equal(sp.allowed.cpu(), so.allowed), f"{what}: allowed differs"
    assert torch.equal(sp.mem_last_exact.cpu(), so.mem_last_exact), f"{what}: LRU stamps differ"
    assert torch.equal(sp.g_recent.cpu(), so.g_recent), f"{what}: ring gates differ"
    assert [sp.recent_idx, sp.recent_filled, sp.pos] == [so.recent_idx, so.recent_filled, so.pos], what
    for f in ("k_buf", "v_buf", "_exact_v_norm", "_sum_lf_k_norm"):
        assert_close(getattr(sp, f), getattr(so, f), torch.float32, f"{what}: {f}", tol)


@torch.no_grad()
def test_two_bounded_llama_adapters_under_eviction_match_the_oracle():
    """A 2-layer residual stack of bounded LlamaCoDAAdapter layers (device
    projections, fp32) against two OracleLayers with the same weights:
    prefill of 3 windows (eviction in every chunk), then 24 decode steps."""
    _need_gpu()
    from coda_oracle import OracleLayer
    from coda_gqa_l.adapters import LlamaCoDAAdapter
    kw = dict(window=64, num_landmarks_exact=16, num_landmarks_summary=16)
    torch.manual_seed(5)
    ads = [LlamaCoDAAdapter(hidden_size=256, num_heads=4, num_kv_heads=2, head_dim=64, bounded=True, block_size=64,
                            **kw).to(DEV).eval() for _ in range(2)]
    ors = []
    for ad in ads:
        o = OracleLayer(embed_dim=256, num_heads=4, num_kv_heads=2, head_norm_mode="identity", rope_interleaved=False,
                        **kw).eval()
        o.load_state_dict({k: v.detach().cpu() for k, v in ad.coda.state_dict().items()})
        ors.append(o)
    B = 2
    torch.manual_seed(6)
    st_o = [o.init_state(batch_size=B, dtype=torch.float32) for o in ors]
    for ad, s in zip(ads, st_o):
        ad.set_state(to_product_state(s, DEV))
    g = torch.Generator().manual_seed(7)
    print("[adapters] 2 bounded layers, fp32, B2: prefill 192 tokens (block 64, W64), 24 decode steps", flush=True)
    x = torch.randn(B, 192, 256, generator=g)
    hp, ho = x.to(DEV), x.clone()
    for li, (ad, o) in enumerate(zip(ads, ors)):
        yp = ad(hp)[0]
        yo, st_o[li] = o.prefill_chunked(ho, st_o[li], block_size=64)
        assert_close(yp, yo, torch.float32, f"layer {li} prefill output")
        _compare_close_states(ad.get_state(), st_o[li], f"layer {li} after prefill")
        hp, ho = hp + yp, ho + yo
    for t in range(24):
        x = torch.randn(B, 1, 256, generator=g)
        hp, ho = x.to(DEV), x.clone()
        for li, (ad, o) in enumerate(zip(ads, ors)):
            yp = ad(hp)[0]
            yo, st_o[li] = o.step(ho, st_o[li])
            assert_close(yp, yo, torch.float32, f"layer {li} step {t} output")
            _compare_close_states(ad.get_state(), st_o[li], f"layer {li} step {t}")
            hp, ho = hp + yp, ho + yo


@torch.no_grad()
def test_two_bounded_eve_adapters_under_eviction_match_the_oracle():
    """A 2-layer residual stack of bounded EveCoDAAdapter layers (Eve-2's
    layout: multi-head, head_dim 64, fused QKV and output projection with
    biases, interleaved RoPE, full head norm; reference eve_adapter.py:30-465,
    343-369) against two OracleLayers with the same weights and biases, fp32:
    prefill of 3 windows (eviction in every chunk), then 24 decode steps."""
    _need_gpu()
    import torch.nn as nn
    from coda_oracle import OracleLayer
    from coda_gqa_l.adapters import EveCoDAAdapter

    class EveAttention(nn.Module):
        def __init__(self):
            super().__init__()
            self.n_embd, self.n_head, self.head_dim = 256, 4, 64
            self.c_attn = nn.Linear(256, 768, bias=True)
            self.c_proj = nn.Linear(256, 256, bias=True)

    kw = dict(window=64, num_landmarks_exact=16, num_landmarks_summary=16)
    torch.manual_seed(15)
    ads = []
    for _ in range(2):
        eve = EveAttention()
        with torch.no_grad():
            for lin in (eve.c_attn, eve.c_proj):
                lin.bias.normal_(0.0, 0.05)
        ads.append(EveCoDAAdapter.from_eve_attention(eve, bounded=True, block_size=64, **kw).to(DEV).eval())
    ors = []
    for ad in ads:
        assert ad.coda.num_kv_heads == ad.coda.num_heads == 4 and ad.coda.rope_interleaved
        assert ad.coda.head_norm_mode == "full" and ad.coda.q_proj.bias is not None
        o = OracleLayer(embed_dim=256, num_heads=4, num_kv_heads=4, **kw).eval()
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            lin = getattr(o, name)
            setattr(o, name, nn.Linear(lin.in_features, lin.out_features, bias=True))
        o.load_state_dict({k: v.detach().cpu() for k, v in ad.coda.state_dict().items()})
        ors.append(o)
    B = 2
    torch.manual_seed(16)
    st_o = [o.init_state(batch_size=B, dtype=torch.float32) for o in ors]
    for ad, s in zip(ads, st_o):
        ad.set_state(to_product_state(s, DEV))
    g = torch.Generator().manual_seed(17)
    print("[adapters] 2 bounded Eve layers, fp32, B2: prefill 192 tokens (block 64, W64), 24 decode steps",
          flush=True)
    x = torch.randn(B, 192, 256, generator=g)
    hp, ho = x.to(DEV), x.clone()
    for li, (ad, o) in enumerate(zip(ads, ors)):
        yp = ad(hp)
        yo, st_o[li] = o.prefill_chunked(ho, st_o[li], block_size=64)
        assert_close(yp, yo, torch.float32, f"Eve layer {li} prefill output")
        _compare_close_states(ad.get_state(), st_o[li], f"Eve layer {li} after prefill")
        hp, ho = hp + yp, ho + yo
    for t in range(24):
        x = torch.randn(B, 1, 256, generator=g)
        hp, ho = x.to(DEV), x.clone()
        for li, (ad, o) in enumerate(zip(ads, ors)):
            yp = ad(hp)
            yo, st_o[li] = o.step(ho, st_o[li])
            assert_close(yp, yo, torch.float32, f"Eve layer {li} step {t} output")
            _compare_close_states(ad.get_state(), st_o[li], f"Eve layer {li} step {t}")
            hp, ho = hp + yp, ho + yo


@torch.no_grad()
def test_metrics_stay_on_the_device_until_read():
    _need_gpu()
    from coda_oracle import OracleLayer, banks, prims
    dtype, B = torch.bfloat16, 2
    kw = dict(C1, collect_metrics=True)
    torch.manual_seed(0)
    m = OracleLayer(**kw).to(dtype).eval()
    p = product_like(m, {"kw": kw}, dtype, DEV)
    torch.manual_seed(1)
    st_o = m.init_state(batch_size=B, dtype=dtype)
    st_p = to_product_state(st_o, DEV)
    g = torch.Generator().manual_seed(3)
    L = 1024
    x = torch.randn(B, L, m.embed_dim, generator=g).to(dtype)
    q, k, v, gate, lam = m.project(x)
    c, s = m.rope_tables(L, 0, dtype)
    k_r = prims.rope(k, c, s, m.rope_interleaved)
    m.prefill_core(prims.rope(q, c, s, m.rope_interleaved), k_r, v, gate, lam, st_o, block_size=256)
    steps = []
    for t in range(16):
        xt = torch.randn(B, 1, m.embed_dim, generator=g).to(dtype)
        qp = int(st_o.pos)
        kn, vn, gn = m._new_kv(xt, qp)
        qt = m.q_proj(xt).view(B, 1, m.num_heads, m.head_dim).transpose(1, 2)
        lamt = torch.sigmoid(m.lambda_proj(xt)).transpose(1, 2).unsqueeze(-1)
        banks.write_one(m, st_o, kn, vn, gn)
        ct, sn = m.rope_tables(1, qp, dtype)
        steps.append([u.to(DEV) for u in (qt, kn, vn, gn.reshape(B), lamt.squeeze(-1), ct, sn)])
    ins = [u.to(DEV) for u in (q, k_r, v, gate, lam.squeeze(-1), c, s)]
    # the one host round trip of a parameter version (sigmoid of the summary
    # eta logits on the CPU, cached per version) before the checked region
    p._eta_f32(torch.device(DEV), dtype)
    torch.cuda.synchronize()
    print("[metrics] C1 bf16 B2: prefill 1024 + 16 decode steps with synchronising ops made errors", flush=True)
    torch.cuda.set_sync_debug_mode("error")
    try:
        p.prefill_core(*ins[:5], ins[5], ins[6], st_p, block_size=256)
        for u in steps:
            p.decode_step_core(*u[:5], st_p, u[5], u[6])
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    assert st_p.metrics == pytest.approx(st_o.metrics)
    assert st_o.metrics["total_evictions"] > 0 and st_o.metrics["summary_updates"] > 0
    compare_states(st_p, st_o, dtype, m.window, m.Me, "metrics run")


@torch.no_grad()
def test_dynamic_expansion_runs_without_host_syncs_and_matches_the_golden():
    """The golden case with dynamic bank expansion (min < max capacities,
    collect_metrics) through the whole module (device projections, fp32):
    prefill_chunked and every decode step run with each torch synchronising
    operation made an error, so the active sizes grow on the device
    (coda_bank_expand) with no host round trip; afterwards outputs,
    decisions, the grown active sizes and every metric equal the reference's
    recorded values (attention.py:344-390, memory_banks.py:333-337,
    418-426, 744-766, 934-946)."""
    _need_gpu()
    import json
    from golden_util import from_np, load
    from test_parity_gpu import _oracle_case
    from parity_util import TOL
    name = "tiny_expand"
    case, dtype, m, x, xs, _ = _oracle_case(name)
    gold = load(name)
    p = product_like(m, case, dtype, DEV)
    assert p._expandable()
    torch.manual_seed(case["seed_state"])
    st = p.init_state(batch_size=case["B"], device=DEV, dtype=dtype, mem_init=case.get("mem_init"))
    xd, xsd = x.to(DEV), [xt.to(DEV) for xt in xs]
    p._eta_f32(torch.device(DEV), dtype)  # the parameter's one host round trip, before the checked region
    torch.cuda.synchronize()
    print(f"[expansion] {name}: prefill {x.shape[1]} + {len(xs)} steps with synchronising ops made errors",
          flush=True)
    torch.cuda.set_sync_debug_mode("error")
    try:
        y, st = p.prefill_chunked(xd, st, block_size=case["block"])
        ys = []
        for xt in xsd:
            yt, st = p.step(xt, st)
            ys.append(yt)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    assert st.__dict__.get("_active_stale"), "the active sizes were expected to grow on the device"
    assert_close(y, from_np(gold["y_prefill"], dtype), dtype, f"{name} prefill y", TOL[dtype])
    assert_close(torch.cat(ys, 1), from_np(gold["y_decode"], dtype), dtype, f"{name} decode y", TOL[dtype])
    assert torch.equal(st.allowed.cpu(), from_np(gold["state_allowed"], torch.bool))
    assert torch.equal(st.mem_last_exact.cpu(), from_np(gold["state_mem_last_exact"], torch.int64))
    assert [st.recent_idx, st.recent_filled, st.pos, st.active_exact, st.active_summary] == \
        list(gold["state_ints"])
    want = json.loads(bytes(gold["metrics_json"]).decode())
    assert want["expansions_exact"] > 0 or want["expansions_summary"] > 0
    assert dict(st.metrics) == pytest.approx(want), f"{name}: metrics differ from the golden"
