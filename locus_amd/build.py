"""In-tree build of the native libraries (no JIT cache; the .so files travel
with the tree to the GPU box).

* liblocus_sampler.so - HIP kernels for gfx950 + the C ABI
  (include/locus_sampler.h), compiled with hipcc.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
INCLUDE = os.path.join(ROOT, "include")

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
# Packed FP32 math is disabled for every HIP translation unit; contraction is
# off so float expressions round exactly like the reference's. Logits are
# finite (the reference's own precondition for a meaningful argmax / sort), so
# NaN operands need no handling: min/max skip the IEEE quieting step.
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
             "-fno-honor-nans", "-mno-amdgpu-ieee",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-I" + INCLUDE]
HIP_SOURCES = ["lcs_api.hip", "lcs_sample.hip", "lcs_verify.hip"]
SAMPLER_SO = os.path.join(HERE, "liblocus_sampler.so")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        noise = "packed-fp32-ops"
        err = "\n".join(l for l in (r.stderr + r.stdout).splitlines() if noise not in l)
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")


def build_sampler(jobs: int = 4) -> str:
    os.makedirs(BUILD, exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    tmp = SAMPLER_SO + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-o", tmp, *objs])
    os.replace(tmp, SAMPLER_SO)
    return SAMPLER_SO


def build_all() -> None:
    build_sampler()


if __name__ == "__main__":
    build_all()
    print("built", SAMPLER_SO)
