"""Build libcoda_mi355x.so (gfx950) from the HIP sources in this directory.

    python coda-gqa-l_amd/csrc/build.py [--jobs N]

Each .hip file compiles to an object with hipcc for gfx950 (cross-compiles
on a host without a GPU), then one shared library is linked next to the
Python package: coda-gqa-l_amd/coda_gqa_l/libcoda_mi355x.so.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(os.path.dirname(HERE), "coda_gqa_l")
sys.path.insert(0, PKG)
from _srchash import source_hash  # noqa: E402  (no torch import)
sys.path.pop(0)
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(PKG, "libcoda_mi355x.so")
SOURCES = ["abi.hip", "attn.hip", "epilogue.hip", "rope.hip", "banks.hip", "proj.hip"]
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
         # packed fp32 instructions are kept out of every kernel
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         # no implicit multiply-add fusion: the reference rounds every product
         # before the add; accumulations that want FMA call fmaf explicitly
         "-ffp-contract=off",
         # MFMA accumulators in ordinary VGPRs: the online-softmax rescale and
         # the epilogue read them with VALU instructions, which cannot address
         # AGPRs (every access would be a copy)
         "-mllvm", "-amdgpu-mfma-vgpr-form",
         "-Wno-unused-result"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build the MI355X kernels)")


def _compile(src: str, tag: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *FLAGS, f'-DCODA_SOURCE_HASH="{tag}"', "-c", os.path.join(HERE, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    return obj


def build(jobs: int = 0) -> str:
    os.makedirs(OBJ, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1, 8)
    # the loader compares this with the sources it finds (coda_source_hash)
    tag = source_hash() or "unknown"
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda src: _compile(src, tag), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=0)
    a = ap.parse_args()
    print(build(a.jobs))
    sys.exit(0)
