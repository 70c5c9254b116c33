"""Golden-vector cases: layer config, seeds, shapes. Shared by the generator
(make_golden.py) and the tests that replay them against the oracle and the
HIP path. Inputs are regenerated from seeds with the torch CPU generator and
checked against the checksums stored in each .npz.
"""

from __future__ import annotations

import torch

TINY = dict(embed_dim=128, num_heads=4, num_kv_heads=2, window=32,
            num_landmarks_exact=16, num_landmarks_summary=16)
C1 = dict(embed_dim=512, num_heads=8, num_kv_heads=2, window=256,
          num_landmarks_exact=64, num_landmarks_summary=64)


def _case(kw, dtype="float32", B=1, L=256, block=64, steps=40, seed=0, **extra):
    c = dict(kw=dict(kw), dtype=dtype, B=B, L=L, block=block, steps=steps,
             seed_model=seed, seed_state=seed + 1, seed_x=seed + 2, seed_steps=1000 + seed)
    for k, v in extra.items():
        if k in ("mem_init", "y_rows"):
            c[k] = v
        else:
            c["kw"][k] = v
    return c


CASES = {
    # small cases: every row of every output stored
    "tiny_f32": _case(TINY),
    "tiny_bf16": _case(TINY, dtype="bfloat16", seed=10),
    "tiny_b2_f32": _case(TINY, B=2, L=200, block=48, seed=20),
    "tiny_b3_bf16": _case(TINY, dtype="bfloat16", B=3, L=160, block=40, seed=30),
    "tiny_policy_none": _case(TINY, seed=40, write_policy="none"),
    "tiny_refresh": _case(TINY, B=2, seed=50, exact_refresh_on_hit=True, exact_match_threshold=0.0,
                          exact_novelty_threshold=-0.5),
    "tiny_no_overwrite": _case(TINY, seed=60, summary_overwrite_on_insert=False),
    "tiny_zeros": _case(TINY, B=2, seed=70, mem_init="zeros"),
    "tiny_nomask": _case(TINY, B=2, seed=80, mask_unused_memory=False),
    "tiny_me0": _case(TINY, seed=90, num_landmarks_exact=0),
    "tiny_ms0": _case(TINY, L=700, block=700, steps=10, seed=100, num_landmarks_summary=0),
    "tiny_w1": _case(TINY, L=40, block=8, steps=12, seed=110, window=1),
    "tiny_llama": _case(TINY, dtype="bfloat16", B=2, seed=120, rope_interleaved=False,
                        head_norm_mode="identity"),
    "tiny_mha": _case(dict(TINY, num_heads=2, num_kv_heads=2, embed_dim=128), seed=130),
    "tiny_expand": _case(TINY, L=512, block=32, steps=60, seed=140, min_landmarks_exact=4,
                         max_landmarks_exact=16, min_landmarks_summary=4, max_landmarks_summary=16,
                         expansion_t_max=1000, collect_metrics=True),
    "tiny_metrics_bf16": _case(TINY, dtype="bfloat16", B=2, seed=150, collect_metrics=True),
    "tiny_bigblock": _case(TINY, L=300, block=1024, steps=10, seed=160),
    "tiny_cand": _case(TINY, B=2, L=256, block=64, seed=170, exact_candidates_per_block=24,
                       summary_candidates_per_block=3),
    # config C1 of BASELINE.json (D512/H8/Hkv2, W256/Me64/Ms64), fewer decode steps
    "c1_f32": _case(C1, L=2048, block=256, steps=50, seed=0, y_rows=16),
    "c1_bf16": _case(C1, dtype="bfloat16", L=2048, block=256, steps=50, seed=200, y_rows=16),
}


# Cases checked only as HIP path vs oracle on the GPU (no reference
# fixture): more than 64 exact candidates per block, so the chunk's exact
# decisions span several 64-candidate passes.
GPU_CASES = {
    "tiny_cand_many": _case(TINY, B=2, L=512, block=128, seed=180, exact_candidates_per_block=80,
                            summary_candidates_per_block=70),
}


def make_inputs(case):
    """(x_prefill (B,L,D), [x_t (B,1,D)] * steps) in the case dtype."""
    dtype = getattr(torch, case["dtype"])
    B, L, D = case["B"], case["L"], case["kw"]["embed_dim"]
    g = torch.Generator().manual_seed(case["seed_x"])
    x = torch.randn(B, L, D, generator=g).to(dtype)
    xs = []
    for t in range(case["steps"]):
        gt = torch.Generator().manual_seed(case["seed_steps"] + t)
        xs.append(torch.randn(B, 1, D, generator=gt).to(dtype))
    return x, xs
