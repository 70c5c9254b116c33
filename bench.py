"""Throughput of the bounded differential-attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch 64] [--no-cpu]

Workload: 7B-shaped bounded layer, hidden 4096,
32 query heads, 8 KV heads, head_dim 128, medium cache (W=256, Me=64,
Ms=64), bf16, random-init weights, state pre-filled with 4096 N(0,1) tokens
per sequence (chunked prefill, block 256), then decode at batch 64.

A step is one decode token of the hot path for the whole batch: one launch
of the fused decode step kernel (ring FIFO + exact bank + summary bank
update, and the differential attention over the updated cache), with the
post-projection inputs of every step already resident in HBM.  `value` =
batch * steps / wall time of the K timed steps.

Also reported (extra keys): configs[1] decode at batch 1 and 16; the
chunked-prefill figures of configs[2] (B=4, 32768 tokens, blocks 256 and
128) for the hot path (attention + banks per chunk); configs[3]'s
unbounded attention; configs[4]'s decode (batch 128) and chunked prefill
(batch 8); the whole 7B layer, projections included (decode batch 64,
prefill batch 4); the dominant kernels' rooflines from HIP events on the
launch stream; and the CPU oracle on this host's cores: the configs[1]
decode sample (`cpu_baseline`) and the C1 / C3 / C4 legs
(`cpu_baseline_legs`), each on a bounded sample stated with it.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "coda-gqa-l_amd"))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--prefill-tokens", type=int, default=4096, help="tokens pre-filled before decode")
    ap.add_argument("--prefill-len", type=int, default=32768, help="configs[2] prefill length")
    ap.add_argument("--prefill-batch", type=int, default=4)
    ap.add_argument("--block", type=int, default=256)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-prefill", action="store_true", help="skip the configs[2] prefill figure")
    ap.add_argument("--no-unbounded", action="store_true", help="skip the configs[3] unbounded attention figure")
    ap.add_argument("--no-c5", action="store_true", help="skip the configs[4] 70B-shaped decode / prefill figures")
    ap.add_argument("--no-small-batch", action="store_true", help="skip the configs[1] batch 1 / 16 decode figures")
    ap.add_argument("--no-layer", action="store_true", help="skip the whole-layer (projections included) figures")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="before timing, run 5 device-to-device copies of this many MiB (a plain copy kernel of "
                         "known size that scales the FETCH_SIZE / WRITE_SIZE counters of a --pmc run)")
    return ap.parse_args()


def layer(torch, coda, dtype, dev):
    torch.manual_seed(0)
    m = coda.CoDAGQALandmarkPerf2(embed_dim=4096, num_heads=32, num_kv_heads=8, window=256,
                                  num_landmarks_exact=64, num_landmarks_summary=64, rope_base=1e4)
    return m.to(dtype=dtype).to(dev).eval()


def attention_launcher(torch, coda, d, like):
    """A closure that enqueues coda_diff_attn_fwd for the prepared
    descriptor d, its workspace (if the plan needs one) allocated once."""
    import ctypes
    hip = coda._hip
    L = hip.lib()
    need = ctypes.c_size_t(0)
    hip.check(L.coda_attn_workspace_bytes(d, need))
    ws = None
    if need.value:
        ws = torch.empty(need.value, dtype=torch.uint8, device=like.device)
        d.workspace, d.workspace_bytes = ws.data_ptr(), need.value
    stream = hip.stream_of(like)

    def launch(_ws=ws):
        hip.check(L.coda_diff_attn_fwd(d, stream))
    return launch


def profile_traffic(label):
    """HBM bytes per launch of `label` from the committed rocprofv3 --pmc
    summaries (FETCH_SIZE / WRITE_SIZE scaled by a plain copy of known size),
    or None when no summary covers it."""
    d = os.path.join(ROOT, "profiles")
    if not os.path.isdir(d):
        return None
    for f in sorted(os.listdir(d)):
        if not f.startswith("traffic_"):
            continue
        for line in open(os.path.join(d, f)):
            if line.startswith("traffic_bytes ") and line[len("traffic_bytes "):].rsplit(" ", 1)[0] == label:
                return int(float(line.rsplit(" ", 1)[1]))
    return None


def decode_bytes(m, B, e=2):
    """Algorithmic HBM bytes of one decode step (bank update + attention)."""
    Hkv, H, Dh, Lbuf, Me, Ms, LF = m.num_kv_heads, m.num_heads, m.head_dim, m.Lbuf, m.Me, m.Ms, m.lf_dim
    attn = B * Hkv * 2 * Lbuf * Dh * e + B * Lbuf + 2 * B * H * Dh * e + B * H * e
    bank = (B * Hkv * (Me * Dh * e + Ms * LF * e)          # norm caches read
            + B * Hkv * Dh * e * 2                         # evicted k, v read
            + B * Hkv * Dh * e * 2 * 2                     # new k, v read + ring write
            + B * Hkv * Dh * e * (2 + 1) * 2               # exact slot k, v (r+w) + norm (w)
            + B * Hkv * Dh * e * 2 * 2 + B * Hkv * LF * e  # summary slot k, v (r+w) + norm (w)
            + B * (Lbuf + 8 * Me + 16))                    # allowed, LRU stamps, gates
    return attn, bank


def prefill_chunk_flops(m, B, blk, n_prefix):
    """8*Dh*B*H*(blk*n_prefix + blk*(blk+1)/2): 2 streams x (QK^T + PV)."""
    return 8 * m.head_dim * B * m.num_heads * (blk * n_prefix + blk * (blk + 1) / 2)


def run_decode(torch, coda, m, B, prefill_tokens, prefill_call, steps, warmup, block, copy_calib_mib=0):
    """Decode throughput of ``m`` at batch ``B``: the state pre-filled with
    ``prefill_tokens`` N(0,1) tokens, post-projection inputs of every step
    resident in HBM (k as projected, before RoPE: the step kernel ropes it),
    then ``warmup`` + ``steps`` calls of the decode step (one launch of the
    fused step kernel each).  Returns tok/s, wall ms per
    step, kernel ms per step (one pair of HIP events on the launch stream
    around the timed steps), the state and the step inputs."""
    dev = "cuda:0"
    dt = torch.bfloat16
    H, Dh, E = m.num_heads, m.head_dim, m.num_heads * m.head_dim
    g = torch.Generator(device=dev).manual_seed(1)
    st = m.init_state(batch_size=B, device=dev, dtype=dt)
    with torch.no_grad():
        for t0 in range(0, prefill_tokens, prefill_call):
            n = min(prefill_call, prefill_tokens - t0)
            x = torch.randn(B, n, E, generator=g, device=dev, dtype=dt)
            _, st = m.prefill_chunked(x, st, block_size=block, return_outputs=False)
            del x
    torch.cuda.synchronize()
    n_steps = warmup + steps
    with torch.no_grad():
        q_all, k_all, v_all, g_all, lam_all, cs_all = [], [], [], [], [], []
        p0 = st.pos
        cos, sin = m.rope(seq_len=n_steps, offset=p0, device=dev, dtype=dt)
        for i in range(n_steps):
            x = torch.randn(B, 1, E, generator=g, device=dev, dtype=dt)
            q_all.append(m._project_q(x))
            kr, v = m._project_kv_raw(x)
            k_all.append(kr)
            v_all.append(v)
            g_all.append(m._write_gate(x).reshape(B).contiguous())
            lam_all.append(m._lambda(x))
            cs_all.append((cos[i:i + 1].contiguous(), sin[i:i + 1].contiguous()))
        heads = torch.empty((B, 1, H, Dh), dtype=dt, device=dev)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    if copy_calib_mib > 0:
        src = torch.empty(copy_calib_mib << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    def run_step(i):
        # one library call: one launch of the fused decode step kernel (the
        # routing record is carried from the previous step)
        m.decode_step_core(q_all[i], k_all[i], v_all[i], g_all[i], lam_all[i], st, cs_all[i][0], cs_all[i][1],
                           out=heads, k_roped=False)

    with torch.no_grad():
        for i in range(warmup):
            run_step(i)
        torch.cuda.synchronize()
        # HIP events on the launch stream bracket the timed region: one
        # kernel launch per step, so their span / steps is the average launch
        # duration (plus any launch gaps)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for j in range(steps):
            run_step(warmup + j)
        e1.record(stream)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    wall = t1 - t0
    return (B * steps / wall, wall * 1e3 / steps, e0.elapsed_time(e1) / steps, st, q_all, k_all, v_all, g_all,
            lam_all)


def main():
    a = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: the bounded layer shards by batch with no communication, "
              "and this build runs on a single GPU only (use --gpus 1).", file=sys.stderr)
        sys.exit(2)
    import torch
    import coda_gqa_l as coda

    dev = "cuda:0"
    dt = torch.bfloat16
    B = a.batch
    m = layer(torch, coda, dt, dev)

    (tok_s, ms_step, step_gpu_ms, st, q_all, k_all, v_all, g_all, lam_all) = run_decode(
        torch, coda, m, B, a.prefill_tokens, 2048, a.steps, a.warmup, a.block, a.copy_calib_mib)
    attn_bytes, bank_bytes = decode_bytes(m, B)
    achieved = (attn_bytes + bank_bytes) / (step_gpu_ms * 1e-3) / 1e9

    out = {
        "metric": "decode tok/s/GPU, 7B-shaped bounded layer, medium cache, batch %d (hot path: banks + "
                  "fused diff attention)" % B,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) inputs, random-init weights (seed 0), state pre-filled with %d tokens"
                % a.prefill_tokens,
        "config": {"workload": "configs[1] decode: hidden 4096, H32/Hkv8/Dh128, W256/Me64/Ms64, bf16",
                   "batch": B, "prefilled_tokens": a.prefill_tokens, "Lbuf": m.Lbuf},
        "roofline": {"bound": "hbm", "kernel": "decode_step_bf16<128> (one launch per step: bank update on one wave beside the ring attention, then the bank slots)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profile_traffic("decode_step_b%d decode_step_bf16<128>" % B),
                     "bytes_per_launch": attn_bytes + bank_bytes, "avg_launch_ms": round(step_gpu_ms, 5)},
        "step_bytes": attn_bytes + bank_bytes,
        "step_hbm_frac": round((attn_bytes + bank_bytes) / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
    }

    print(f"# decode: {tok_s:.0f} tok/s, {ms_step * 1e3:.1f} us/step, kernels {step_gpu_ms * 1e3:.1f} us "
          f"({achieved:.0f} GB/s)", file=sys.stderr, flush=True)
    # ---------------------------------------------------------------- decode at batch 1 / 16
    if not a.no_small_batch:
        for bs in (1, 16):
            t_s, ms_s, gms = run_decode(torch, coda, m, bs, a.prefill_tokens, 2048, a.steps, a.warmup, a.block)[:3]
            ab, bb = decode_bytes(m, bs)
            ach = (ab + bb) / (gms * 1e-3) / 1e9
            out["decode_b%d" % bs] = {
                "metric": "decode tok/s, configs[1] layer, batch %d" % bs, "value": round(t_s, 1), "unit": "tok/s",
                "batch": bs, "steps": a.steps, "ms_per_step": round(ms_s, 5),
                "roofline": {"bound": "hbm", "kernel": "decode_step_bf16<128>", "achieved": round(ach, 1),
                             "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                             "bytes_per_launch": ab + bb, "avg_launch_ms": round(gms, 5)}}
            print(f"# decode B{bs}: {t_s:.0f} tok/s, {ms_s * 1e3:.1f} us/step ({ach:.0f} GB/s)", file=sys.stderr,
                  flush=True)
    # ---------------------------------------------------------------- prefill
    if not a.no_prefill:
        out["prefill"] = bench_prefill(torch, coda, m, a, a.block)
        print(f"# prefill: {out['prefill']['value']:.0f} tok/s", file=sys.stderr, flush=True)
        out["prefill_blk128"] = bench_prefill(torch, coda, m, a, 128)
        print(f"# prefill block 128: {out['prefill_blk128']['value']:.0f} tok/s", file=sys.stderr, flush=True)
    # ---------------------------------------------------------------- unbounded
    if not a.no_unbounded:
        out["unbounded"] = bench_unbounded(torch, coda)
        print(f"# unbounded: {out['unbounded']['value']:.0f} tok/s, "
              f"{out['unbounded']['roofline']['achieved']:.0f} TFLOP/s", file=sys.stderr, flush=True)
    # ---------------------------------------------------------------- 70B-shaped decode
    if not a.no_c5:
        out["decode_c5"] = bench_decode_c5(torch, coda, a)
        print(f"# decode configs[4]: {out['decode_c5']['value']:.0f} tok/s, "
              f"{out['decode_c5']['roofline']['achieved']:.0f} GB/s", file=sys.stderr, flush=True)
        out["prefill_c5"] = bench_prefill_c5(torch, coda, a)
        print(f"# prefill configs[4]: {out['prefill_c5']['value']:.0f} tok/s", file=sys.stderr, flush=True)
    # ---------------------------------------------------------------- whole layer, projections included
    if not a.no_layer:
        out["layer"] = bench_layer(torch, coda, m, a)
        print(f"# layer: decode {out['layer']['decode']['value']:.0f} tok/s, prefill "
              f"{out['layer']['prefill']['value']:.0f} tok/s", file=sys.stderr, flush=True)
    # ---------------------------------------------------------------- CPU baseline
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_baseline(torch, m, st, q_all, k_all, v_all, g_all, lam_all, a)
        out["cpu_baseline_legs"] = cpu_legs(torch)
    print(json.dumps(out), flush=True)


# the prefill attention kernels the dispatch (attn.hip launch_f3_qm) runs,
# named as rocprofv3 prints them: queries roped in-kernel with the noise
# rotation (layer path), and given noise queries (the diff_flash_attn seam,
# 4096 eight-wave workgroups' worth, so the 4-wave kernel)
F3_GIVEN_NOISE = "attn_f3_bf16<128, 4, 2, false, 2>"


def f3_roped(torch, G, Lq, B, Hkv, chunks):
    """The roped-query attention kernel of a launch over `chunks` chunks
    (0: one chunk, as the descriptor says) of Lq queries: 4 waves and two
    tile stages for G <= 4, except a one-launch grid whose 8-wave
    workgroups fill the CUs once (at least one a CU, fewer than two): 8
    waves and four stages (attn.hip launch_f3_qm)."""
    rows8 = 16 * (8 // G)
    n8 = -(-Lq // rows8) * B * Hkv * max(chunks, 1)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    small = G <= 4 and (chunks > 1 or n8 < cus or n8 >= 2 * cus)
    return "attn_f3_bf16<128, %d, 0, true, %d>" % ((4, 2) if small else (8, 4))


def prefill_hot_path(coda, m, q, k_raw, v, gate, lam, k_out, st, blk, heads):
    """The timed prefill path after the projections: RoPE tables of the
    positions and the k RoPE (attention.py:598-600), then the chunk loop
    (attention + bank update per chunk, attention.py:611-724)."""
    L = q.shape[2]
    cos, sin = m.rope(seq_len=L, offset=int(st.pos), device=q.device, dtype=q.dtype)
    cos, sin = cos.contiguous(), sin.contiguous()
    coda.apply_rope(k_raw, cos, sin, interleaved=m.rope_interleaved, out=k_out)
    m.prefill_core(q, k_out, v, gate, lam, cos, sin, st, block_size=blk, out=heads)
    return cos, sin


def chunked_attention_timing(torch, coda, m, q, k, v, lam, cos, sin, heads, blk, reps):
    """The prefill attention as the layer runs it after the bank chain of a
    fresh call: the call's last group of chunks (every chunk when the
    snapshot buffers hold them all) in one launch of coda_prefill_attn_chunks
    from the bank snapshots the chain left (the layer's snapshot buffers,
    still holding the timed call's last group), timed over `reps` launches
    with HIP events on the launch stream.  FLOPs per launch: 8 Dh B H per
    (query, visible key) pair, the visible keys of chunk c being its
    snapshot's used bank slots (mean over the batch), its ring window and the
    causal block."""
    B, H, L, Dh = q.shape
    snaps = m.__dict__.get("_snap_cache", {}).get((str(q.device), q.dtype, B, m.num_kv_heads, m.Me + m.Ms, Dh))
    last = m.__dict__.get("_last_chunk_group")
    if not m.pipelined_prefill or snaps is None or last is None or last[2:] != (blk, L):
        return None  # the timed call did not end in a grouped launch
    sk, sv, sa = snaps
    ca, cb = last[0], last[1]
    n = cb - ca
    ct, sn = m._theta_tables(q.dtype)
    d, keep = coda.ops.attention_desc(
        q=q, rope_cos=cos, rope_sin=sin, rope_interleaved=m.rope_interleaved, theta_cos=ct, theta_sin=sn,
        k_prefix=sk[0], v_prefix=sv[0], allowed=sa[0], k_block=k, v_block=v, lam=lam, rms_weight=m._rms_weight(q.dtype),
        eps=m._eps, out=heads.permute(0, 2, 1, 3))
    L_ = coda._hip.lib()
    stream = coda._hip.stream_of(q)

    def launch():
        coda._hip.check(L_.coda_prefill_attn_chunks(d, n, ca, blk, L, m.window, sk[0].numel(), sa[0].numel(), stream))
    launch()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    tstream = torch.cuda.current_stream(q.device)
    e0.record(tstream)
    for _ in range(reps):
        launch()
    e1.record(tstream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    nb = sa[:n].float().sum(dim=-1).mean(dim=1).tolist()
    flops = 0.0
    for y in range(n):
        t0 = (ca + y) * blk
        lq = min(blk, L - t0)
        flops += 8.0 * Dh * B * H * (lq * (nb[y] + min(t0, m.window)) + lq * (lq + 1) / 2)
    return ms, flops, n


def bench_prefill(torch, coda, m, a, blk):
    """chunked prefill of an N(0,1) sequence through the layer's
    projections (outside the timed region), then the hot path (attention +
    bank update per chunk) timed over the whole sequence; the attention
    kernel alone timed on a steady-state chunk (full prefix)."""
    dev = "cuda:0"
    dt = torch.bfloat16
    B, L = a.prefill_batch, a.prefill_len
    g = torch.Generator(device=dev).manual_seed(7)
    st = m.init_state(batch_size=B, device=dev, dtype=dt)
    x = torch.randn(B, L, 4096, generator=g, device=dev, dtype=dt)
    with torch.no_grad():
        q = m._project_q(x)
        kr, v = m._project_kv_raw(x)
        gate = m._write_gate(x)
        lam = m._lambda(x)
        k = torch.empty((B, L, m.num_kv_heads, m.head_dim), dtype=dt, device=dev).permute(0, 2, 1, 3)
        heads = torch.empty((B, L, m.num_heads, m.head_dim), dtype=dt, device=dev)
        # warm-up pass over a short prefix (plan / workspace / kernels loaded)
        st_w = m.init_state(batch_size=B, device=dev, dtype=dt)
        prefill_hot_path(coda, m, q[:, :, :4 * blk], kr[:, :, :4 * blk], v[:, :, :4 * blk], gate[:, :4 * blk],
                         lam[:, :, :4 * blk], k[:, :, :4 * blk], st_w, blk, heads)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        cos, sin = prefill_hot_path(coda, m, q, kr, v, gate, lam, k, st, blk, heads)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        # attention-kernel-only timing of a steady-state chunk (full prefix)
        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 20
        t_s = L - blk
        ct, sn = m._theta_tables(dt)
        w = m._rms_weight(dt)
        # the descriptor is built once, so the timed loop only enqueues the
        # kernel and host work between launches cannot stretch the average
        d, keep = coda.ops.attention_desc(
            q=q[:, :, t_s:], rope_cos=cos[t_s:], rope_sin=sin[t_s:], rope_interleaved=m.rope_interleaved,
            theta_cos=ct, theta_sin=sn, k_prefix=st.k_buf, v_prefix=st.v_buf, allowed=st.allowed,
            k_block=k[:, :, t_s:], v_block=v[:, :, t_s:], lam=lam[:, :, t_s:], rms_weight=w, eps=m._eps,
            out=heads[:, t_s:].permute(0, 2, 1, 3))
        launch = attention_launcher(torch, coda, d, q)
        launch()
        e0.record(stream)
        for _ in range(reps):
            launch()
        e1.record(stream)
        torch.cuda.synchronize()
        attn_ms = e0.elapsed_time(e1) / reps
        n_prefix = int(st.allowed[0].sum().item())
        chunked = chunked_attention_timing(torch, coda, m, q, k, v, lam, cos, sin, heads, blk, 5)
    flops1 = prefill_chunk_flops(m, B, blk, n_prefix)
    tflops1 = flops1 / (attn_ms * 1e-3) / 1e12
    G = m.num_heads // m.num_kv_heads
    k1 = f3_roped(torch, G, blk, B, m.num_kv_heads, 0)
    single = {"kernel": k1, "what": "one chunk at the full 384-slot state prefix (the dispatch of the first "
                                    "chunks of a call that continues a state)",
              "achieved": round(tflops1, 2), "frac": round(tflops1 / BF16_PEAK_TFLOPS, 4), "flops_per_launch": flops1,
              "avg_launch_ms": round(attn_ms, 5), "valid_prefix_slots": n_prefix,
              "traffic": profile_traffic("prefill_chunk_b%d_blk%d %s" % (B, blk, k1))}
    if chunked is not None:
        ms, flops, n = chunked
        tflops = flops / (ms * 1e-3) / 1e12
        kn = f3_roped(torch, G, blk, B, m.num_kv_heads, n)
        roof = {"bound": "mfma", "kernel": kn + " (a group of the call's chunks in one launch, "
                                                "coda_prefill_attn_chunks)",
                "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tflops / BF16_PEAK_TFLOPS, 4), "flops_per_launch": flops, "avg_launch_ms": round(ms, 5),
                "chunks_per_launch": n, "us_per_chunk": round(ms * 1e3 / n, 3),
                "traffic": profile_traffic("prefill_call_b%d_blk%d %s" % (B, blk, kn)),
                "single_chunk": single}
    else:
        roof = dict({"bound": "mfma", "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s"}, **single)
    return {"metric": "chunked-prefill tok/s (configs[2], hot path: attention + banks per chunk)",
            "value": round(B * L / wall, 1), "unit": "tok/s", "batch": B, "seq_len": L, "block": blk,
            "ms_total": round(wall * 1e3, 3),
            "timed": "k RoPE (tables + kernel) of the whole sequence, then the bank update of every chunk and the "
                     "attention of every chunk (reference attention.py:598-724 after the projections)",
            "roofline": roof}


def bench_decode_c5(torch, coda, a, B=128, steps=50, warmup=10):
    """configs[4]'s decode: the 70B-shaped layer (hidden 8192, 64 q heads, 8
    KV heads, head_dim 128, W512 / Me128 / Ms128, Lbuf 768) at its full decode
    batch of 128 on one GPU (the state is 402 MB), pre-filled with 1024
    tokens; same timing as the configs[1] line."""
    dev = "cuda:0"
    torch.manual_seed(0)
    m = coda.CoDAGQALandmarkPerf2(embed_dim=8192, num_heads=64, num_kv_heads=8, window=512,
                                  num_landmarks_exact=128, num_landmarks_summary=128, rope_base=1e4)
    m = m.to(dtype=torch.bfloat16).to(dev).eval()
    tok_s, ms_step, gpu_ms = run_decode(torch, coda, m, B, 1024, 256, steps, warmup, a.block)[:3]
    attn_b, bank_b = decode_bytes(m, B)
    achieved = (attn_b + bank_b) / (gpu_ms * 1e-3) / 1e9
    return {"metric": "decode tok/s, 70B-shaped bounded layer (configs[4]), large cache, batch %d" % B,
            "value": round(tok_s, 1), "unit": "tok/s", "batch": B, "steps": steps, "ms_per_step": round(ms_step, 5),
            "config": "hidden 8192, H64/Hkv8/Dh128, W512/Me128/Ms128 (Lbuf 768), bf16, 1024 tokens pre-filled",
            "roofline": {"bound": "hbm", "kernel": "decode_step_bf16<128>", "achieved": round(achieved, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                         "bytes_per_launch": attn_b + bank_b, "avg_launch_ms": round(gpu_ms, 5)}}


def bench_prefill_c5(torch, coda, a, B=8, L=8192, blk=256):
    """configs[4]'s chunked prefill on a steady-state sample: the 70B-shaped
    layer (hidden 8192, 64 q heads, 8 KV heads, W512 / Me128 / Ms128, Lbuf
    768) at batch 8, block 256, over 8192 N(0,1) tokens (32 chunks; the ring
    fills after 2) through the layer's projections (outside the timed
    region); hot path timed as in the configs[2] figure."""
    dev = "cuda:0"
    dt = torch.bfloat16
    torch.manual_seed(0)
    m = coda.CoDAGQALandmarkPerf2(embed_dim=8192, num_heads=64, num_kv_heads=8, window=512,
                                  num_landmarks_exact=128, num_landmarks_summary=128, rope_base=1e4)
    m = m.to(dtype=dt).to(dev).eval()
    g = torch.Generator(device=dev).manual_seed(9)
    with torch.no_grad():
        x = torch.randn(B, L, 8192, generator=g, device=dev, dtype=dt)
        q = m._project_q(x)
        kr, v = m._project_kv_raw(x)
        gate = m._write_gate(x)
        lam = m._lambda(x)
        del x
        k = torch.empty((B, L, m.num_kv_heads, m.head_dim), dtype=dt, device=dev).permute(0, 2, 1, 3)
        heads = torch.empty((B, L, m.num_heads, m.head_dim), dtype=dt, device=dev)
        st_w = m.init_state(batch_size=B, device=dev, dtype=dt)
        prefill_hot_path(coda, m, q[:, :, :4 * blk], kr[:, :, :4 * blk], v[:, :, :4 * blk], gate[:, :4 * blk],
                         lam[:, :, :4 * blk], k[:, :, :4 * blk], st_w, blk, heads)
        del st_w
        st = m.init_state(batch_size=B, device=dev, dtype=dt)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        cos, sin = prefill_hot_path(coda, m, q, kr, v, gate, lam, k, st, blk, heads)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        del kr
        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 10
        t_s = L - blk
        ct, sn = m._theta_tables(dt)
        w = m._rms_weight(dt)
        # the descriptor is built once, so the timed loop only enqueues the
        # kernel and host work between launches cannot stretch the average
        d, keep = coda.ops.attention_desc(
            q=q[:, :, t_s:], rope_cos=cos[t_s:], rope_sin=sin[t_s:], rope_interleaved=m.rope_interleaved,
            theta_cos=ct, theta_sin=sn, k_prefix=st.k_buf, v_prefix=st.v_buf, allowed=st.allowed,
            k_block=k[:, :, t_s:], v_block=v[:, :, t_s:], lam=lam[:, :, t_s:], rms_weight=w, eps=m._eps,
            out=heads[:, t_s:].permute(0, 2, 1, 3))
        launch = attention_launcher(torch, coda, d, q)
        launch()
        e0.record(stream)
        for _ in range(reps):
            launch()
        e1.record(stream)
        torch.cuda.synchronize()
        attn_ms = e0.elapsed_time(e1) / reps
        n_prefix = int(st.allowed[0].sum().item())
        chunked = chunked_attention_timing(torch, coda, m, q, k, v, lam, cos, sin, heads, blk, 5)
    flops1 = prefill_chunk_flops(m, B, blk, n_prefix)
    tflops1 = flops1 / (attn_ms * 1e-3) / 1e12
    k1 = f3_roped(torch, m.num_heads // m.num_kv_heads, blk, B, m.num_kv_heads, 0)
    single = {"kernel": k1, "what": "one chunk at the full state prefix", "achieved": round(tflops1, 2),
              "frac": round(tflops1 / BF16_PEAK_TFLOPS, 4), "flops_per_launch": flops1,
              "avg_launch_ms": round(attn_ms, 5), "valid_prefix_slots": n_prefix}
    if chunked is not None:
        ms, flops, n = chunked
        tflops = flops / (ms * 1e-3) / 1e12
        kn = f3_roped(torch, m.num_heads // m.num_kv_heads, blk, B, m.num_kv_heads, n)
        roof = {"bound": "mfma", "kernel": kn + " (a group of the call's chunks in one launch, "
                                                "coda_prefill_attn_chunks)",
                "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tflops / BF16_PEAK_TFLOPS, 4), "flops_per_launch": flops, "avg_launch_ms": round(ms, 5),
                "chunks_per_launch": n, "us_per_chunk": round(ms * 1e3 / n, 3), "single_chunk": single}
    else:
        roof = dict({"bound": "mfma", "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s"}, **single)
    return {"metric": "chunked-prefill tok/s (configs[4], 70B-shaped layer, steady-state sample)",
            "value": round(B * L / wall, 1), "unit": "tok/s", "batch": B, "seq_len": L, "block": blk,
            "ms_total": round(wall * 1e3, 3),
            "sample": "8192 of configs[4]'s 131072 tokens per sequence (32 chunks, ring full after 2)",
            "timed": "k RoPE (tables + kernel), then the bank update and the attention of every chunk",
            "roofline": roof}


def bench_layer(torch, coda, m, a, B_dec=64, steps=100, B_pre=4, L_pre=8192):
    """The whole 7B-shaped layer, projections included (q / k / v / lambda /
    gate, RoPE, the hot path, o_proj): `step` at batch 64 from a state
    pre-filled with 4096 tokens, and `prefill_chunked` at batch 4 over 8192
    tokens (block 256).  Per token: 2 x (weights) FLOPs for the projections
    plus the attention; per decode step the weights (80 MiB at 7B) and the
    state traffic cross HBM once."""
    dev = "cuda:0"
    dt = torch.bfloat16
    E = m.num_heads * m.head_dim
    n_w = sum(p.numel() for p in m.parameters())
    w_bytes = n_w * 2
    g = torch.Generator(device=dev).manual_seed(11)
    with torch.no_grad():
        st = m.init_state(batch_size=B_dec, device=dev, dtype=dt)
        for t0 in range(0, a.prefill_tokens, 2048):
            x = torch.randn(B_dec, min(2048, a.prefill_tokens - t0), E, generator=g, device=dev, dtype=dt)
            _, st = m.prefill_chunked(x, st, block_size=a.block, return_outputs=False)
        xs = torch.randn(steps + 10, B_dec, 1, E, generator=g, device=dev, dtype=dt)
        for i in range(10):
            _, st = m.step(xs[i], st)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            _, st = m.step(xs[10 + i], st)
        torch.cuda.synchronize()
        wall_d = time.perf_counter() - t0
        ab, bb = decode_bytes(m, B_dec)
        step_bytes = w_bytes + ab + bb
        # prefill
        x = torch.randn(B_pre, L_pre, E, generator=g, device=dev, dtype=dt)
        st = m.init_state(batch_size=B_pre, device=dev, dtype=dt)
        m.prefill_chunked(x[:, :4 * a.block], st, block_size=a.block)
        st = m.init_state(batch_size=B_pre, device=dev, dtype=dt)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        m.prefill_chunked(x, st, block_size=a.block)
        torch.cuda.synchronize()
        wall_p = time.perf_counter() - t0
    ms_step = wall_d * 1e3 / steps
    return {"decode": {"metric": "whole-layer decode tok/s (configs[1] layer, projections included)",
                       "value": round(B_dec * steps / wall_d, 1), "unit": "tok/s", "batch": B_dec,
                       "ms_per_step": round(ms_step, 5), "bytes_per_step": step_bytes,
                       "weight_bytes": w_bytes, "flops_per_token": 2 * n_w,
                       "hbm_frac": round(step_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
            "prefill": {"metric": "whole-layer chunked-prefill tok/s (configs[2] layer, projections included)",
                        "value": round(B_pre * L_pre / wall_p, 1), "unit": "tok/s", "batch": B_pre,
                        "seq_len": L_pre, "block": a.block, "ms_total": round(wall_p * 1e3, 3),
                        "flops_per_token_projections": 2 * n_w}}


def bench_unbounded(torch, coda, B=2, L=8192, H=32, Hkv=8, Dh=128, reps=5):
    """unbounded causal differential attention (CoDAGQA,
    reference baseline.py:95-147) through the diff_flash_attn seam: q, k, v ~
    N(0,1), lambda ~ U(0.1, 0.9), q_noise = q R with R a random orthogonal
    128x128 rotation per head, bf16.  Attention kernel only (the projections
    are outside the path); FLOPs over the visible (query, key) pairs."""
    dev = "cuda:0"
    dt = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(3)
    with torch.no_grad():
        q = torch.randn(B, H, L, Dh, generator=g, device=dev, dtype=torch.float32)
        rot = torch.linalg.qr(torch.randn(H, Dh, Dh, generator=g, device=dev, dtype=torch.float32))[0]
        q_noise = torch.matmul(q, rot.unsqueeze(0)).to(dt)
        q = q.to(dt)
        k = torch.randn(B, Hkv, L, Dh, generator=g, device=dev, dtype=dt)
        v = torch.randn(B, Hkv, L, Dh, generator=g, device=dev, dtype=dt)
        lam = (0.1 + 0.8 * torch.rand(B, H, L, 1, generator=g, device=dev, dtype=torch.float32)).to(dt)
        w = torch.ones(Dh, dtype=dt, device=dev)
        for _ in range(2):
            coda.ops.diff_flash_attn(q, q_noise, k, v, lam, rms_weight=w, is_causal=True)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            coda.ops.diff_flash_attn(q, q_noise, k, v, lam, rms_weight=w, is_causal=True)
        e1.record(stream)
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    flops = 8.0 * Dh * B * H * L * (L + 1) / 2
    tflops = flops / (ms * 1e-3) / 1e12
    return {"metric": "unbounded causal diff-attention tok/s (configs[3])", "value": round(B * L / (ms * 1e-3), 1),
            "unit": "tok/s", "batch": B, "seq_len": L, "ms": round(ms, 4),
            "roofline": {"bound": "mfma", "kernel": F3_GIVEN_NOISE + " (causal)", "achieved": round(tflops, 2),
                         "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                         "flops_per_launch": flops, "avg_launch_ms": round(ms, 5)}}


def cpu_baseline(torch, m, st, q_all, k_all, v_all, g_all, lam_all, a):
    """The CPU oracle (a restatement of the reference's CPU eager path) on a
    bounded sample of the same decode workload, on this host's cores."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from coda_oracle import OracleLayer, OracleState, banks, prims
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    dt = torch.bfloat16
    o = OracleLayer(embed_dim=4096, num_heads=32, num_kv_heads=8, window=256, num_landmarks_exact=64,
                    num_landmarks_summary=64, rope_base=1e4).to(dt).eval()
    o.load_state_dict({k: v.cpu() for k, v in m.state_dict().items()})
    so = OracleState(k_buf=st.k_buf.cpu(), v_buf=st.v_buf.cpu(), allowed=st.allowed.cpu(),
                     g_recent=st.g_recent.cpu(), recent_idx=st.recent_idx, recent_filled=st.recent_filled,
                     mem_last_exact=st.mem_last_exact.cpu(), pos=st.pos, active_exact=st.active_exact,
                     active_summary=st.active_summary, _exact_v_norm=st._exact_v_norm.cpu(),
                     _sum_lf_k_norm=st._sum_lf_k_norm.cpu())
    B = q_all[0].shape[0]
    n_done = 0
    t0 = time.perf_counter()
    with torch.no_grad():
        while True:
            i = n_done % len(q_all)
            qp = so.pos
            # the step's k RoPE (k_all holds the raw projections)
            c, s_ = o.rope_tables(1, qp, dt)
            k_new = prims.rope(k_all[i].cpu(), c, s_, o.rope_interleaved)
            banks.write_one(o, so, k_new, v_all[i].cpu(), g_all[i].cpu().view(B, 1))
            o.attend_core(q_all[i].cpu(), lam_all[i].cpu().unsqueeze(-1), so, qp)
            n_done += 1
            if time.perf_counter() - t0 > a.cpu_seconds or n_done >= 2000:
                break
    wall = time.perf_counter() - t0
    return {"value": round(B * n_done / wall, 2), "unit": "tok/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"{n_done} decode steps at batch {B} of the same state "
                                      f"(k RoPE + banks + attention, post-projection inputs), {wall:.1f} s"}


def cpu_legs(torch):
    """The CPU oracle on the other configs' bounded samples (post-projection
    inputs where the GPU figure excludes the projections), on this host's
    cores, in the same run:
      C1  configs[0] in full: D512 layer, fp32, batch 1, prefill_chunked of
          2048 tokens (block 256), then 1000 decode steps (step, projections
          included);
      C3  configs[2]: 16 steady-state chunks (block 256, batch 4, bf16) after
          two chunks that fill the ring, attention + bank update;
      C4  configs[3]: one full causal forward at L 8192, batch 2, bf16,
          computed in blocks of 512 query rows (each against its visible
          keys)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from coda_oracle import OracleLayer, ops
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    legs = {}
    g = torch.Generator().manual_seed(21)
    with torch.no_grad():
        # C1
        torch.manual_seed(0)
        m = OracleLayer(embed_dim=512, num_heads=8, num_kv_heads=2, window=256, num_landmarks_exact=64,
                        num_landmarks_summary=64).eval()
        st = m.init_state(batch_size=1, dtype=torch.float32)
        x = torch.randn(1, 2048, 512, generator=g)
        xs = torch.randn(1000, 1, 1, 512, generator=g)
        t0 = time.perf_counter()
        m.prefill_chunked(x, st, block_size=256)
        t1 = time.perf_counter()
        for i in range(1000):
            m.step(xs[i], st)
        t2 = time.perf_counter()
        legs["C1"] = {"value": round(2048 / (t1 - t0), 1), "unit": "tok/s (prefill)",
                      "decode_value": round(1000 / (t2 - t1), 1), "decode_unit": "tok/s",
                      "cores": torch.get_num_threads(), "kind": "port",
                      "sample": f"configs[0] in full: 2048-token prefill {t1 - t0:.2f} s, 1000 decode steps "
                                f"{t2 - t1:.2f} s"}
        # C3
        dt = torch.bfloat16
        torch.manual_seed(0)
        m = OracleLayer(embed_dim=4096, num_heads=32, num_kv_heads=8, window=256, num_landmarks_exact=64,
                        num_landmarks_summary=64, rope_base=1e4).to(dt).eval()
        B, blk, n_warm, n_chunks = 4, 256, 2, 16
        L = blk * (n_warm + n_chunks)
        q = torch.randn(B, 32, L, 128, generator=g).to(dt)
        k = torch.randn(B, 8, L, 128, generator=g).to(dt)
        v = torch.randn(B, 8, L, 128, generator=g).to(dt)
        gs = torch.sigmoid(torch.randn(B, L, generator=g) - 2.0)
        lam = torch.sigmoid(torch.randn(B, 32, L, 1, generator=g) - 1.0).to(dt)
        st = m.init_state(batch_size=B, dtype=dt)
        w = blk * n_warm
        m.prefill_core(q[:, :, :w], k[:, :, :w], v[:, :, :w], gs[:, :w], lam[:, :, :w], st, block_size=blk)
        t0 = time.perf_counter()
        m.prefill_core(q[:, :, w:], k[:, :, w:], v[:, :, w:], gs[:, w:], lam[:, :, w:], st, block_size=blk)
        t1 = time.perf_counter()
        legs["C3"] = {"value": round(B * blk * n_chunks / (t1 - t0), 1), "unit": "tok/s",
                      "cores": torch.get_num_threads(), "kind": "port",
                      "sample": f"{n_chunks} steady-state chunks of block {blk} at batch {B} (post-projection "
                                f"N(0,1) inputs), {t1 - t0:.2f} s"}
        # C4
        B, L, H, Hkv, Dh, rb = 2, 8192, 32, 8, 128, 512
        wgt = torch.ones(Dh, dtype=dt)
        t_tot = 0.0
        for b in range(B):
            qb = torch.randn(1, H, L, Dh, generator=g).to(dt)
            qn = torch.randn(1, H, L, Dh, generator=g).to(dt)
            kb = torch.randn(1, Hkv, L, Dh, generator=g).to(dt)
            vb = torch.randn(1, Hkv, L, Dh, generator=g).to(dt)
            lb = (0.1 + 0.8 * torch.rand(1, H, L, 1, generator=g)).to(dt)
            t0 = time.perf_counter()
            for r0 in range(0, L, rb):
                r1 = r0 + rb
                ops.diff_attention(qb[:, :, r0:r1], qn[:, :, r0:r1], kb[:, :, :r1], vb[:, :, :r1], lb[:, :, r0:r1],
                                   rms_weight=wgt, is_causal=True)
            t_tot += time.perf_counter() - t0
        legs["C4"] = {"value": round(B * L / t_tot, 1), "unit": "tok/s", "cores": torch.get_num_threads(),
                      "kind": "port", "sample": f"one full causal forward, L {L}, batch {B}, in blocks of {rb} "
                                                f"query rows, {t_tot:.2f} s"}
    return legs


if __name__ == "__main__":
    main()
