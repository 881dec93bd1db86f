"""In-tree build of the native libraries (no JIT cache; the .so files travel
with the tree to the GPU box).

* liblocus_sampler.so - HIP kernels for gfx950 + the C ABI
  (include/locus_sampler.h), compiled with hipcc.
* liblocus_host.so - the C++ host layer (include/locus/...: the reference's
  sampling API over the C ABI, JSON grammar and mask builder, n-gram draft,
  backend registry) and its C ABI (include/locus_host.h).
* tests/cpp/test_host - the host layer's C++ test program.

build_sanitized() (called by the CPU tests, not by build_all) compiles the
host layer, its test program and a driver of the CPU oracle with g++ under
AddressSanitizer and UndefinedBehaviorSanitizer, into _build/asan/. It builds
no device code: the host layer's HIP calls go to the unmodified runtime.
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
HIP_SOURCES = ["lcs_api.hip", "lcs_sample.hip", "lcs_slice.hip", "lcs_windows.hip", "lcs_nucleus.hip", "lcs_verify.hip", "lcs_draft.hip",
               "lcs_lmhead.hip"]
# the leading scalar arguments (8) of slice_stats and the nucleus kernels
# arrive preloaded in SGPRs; the code object keeps a prologue that loads them
# where the firmware does not
HIP_EXTRA = {"lcs_slice.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=8"],
             "lcs_nucleus.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=8"]}
SAMPLER_SO = os.path.join(HERE, "liblocus_sampler.so")
HOST_SO = os.path.join(HERE, "liblocus_host.so")
HOST_SOURCES = ["grammar.cpp", "speculative.cpp", "sampler_registry.cpp", "host_capi.cpp", "sampling.cpp",
                "batch_sampler.cpp"]
HOST_FLAGS = ["-std=c++20", "-O2", "-fPIC", "-Wall", "-I" + INCLUDE]
TEST_HOST = os.path.join(ROOT, "tests", "cpp", "test_host")
BATCH_BENCH = os.path.join(HERE, "batch_bench")   # bench.py --batch-sampler


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        noise = "packed-fp32-ops"
        err = "\n".join(l for l in (r.stderr + r.stdout).splitlines() if noise not in l)
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")


# the same library with the sliced path's phase clocks (LCS_PROFILE:
# s_memrealtime stamps per workgroup phase, read by bench.py --phase-clocks)
PROFILE_SO = os.path.join(HERE, "_prof", "liblocus_sampler.so")


def build_sampler(jobs: int = 4, profile: bool = False) -> str:
    out_so = PROFILE_SO if profile else SAMPLER_SO
    bdir = os.path.join(BUILD, "prof") if profile else BUILD
    os.makedirs(bdir, exist_ok=True)
    os.makedirs(os.path.dirname(out_so), exist_ok=True)
    defs = ["-DLCS_PROFILE"] if profile else []
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(bdir, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, *HIP_EXTRA.get(src, []), *defs, "-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    tmp = out_so + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-o", tmp, *objs])
    os.replace(tmp, out_so)
    return out_so


def build_host(jobs: int = 4) -> str:
    """The C++ host layer, linked against liblocus_sampler.so (found next to
    it at run time), and its test program."""
    os.makedirs(BUILD, exist_ok=True)
    objs, cmds = [], []
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD, "host_" + src.replace(".cpp", ".o"))
        objs.append(obj)
        cmds.append([HIPCC, *HOST_FLAGS, "-c", os.path.join(HERE, "host", src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    tmp = HOST_SO + ".tmp"
    _run([HIPCC, "-shared", "-o", tmp, *objs, "-L" + HERE, "-llocus_sampler", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, HOST_SO)
    tobj = os.path.join(BUILD, "test_host.o")
    _run([HIPCC, *HOST_FLAGS, "-c", os.path.join(ROOT, "tests", "cpp", "test_host.cpp"), "-o", tobj])
    _run([HIPCC, "-o", TEST_HOST + ".tmp", tobj, "-L" + HERE, "-llocus_host", "-llocus_sampler",
          "-Wl,-rpath," + os.path.relpath(HERE, os.path.dirname(TEST_HOST)).join(["$ORIGIN/", ""])])
    os.replace(TEST_HOST + ".tmp", TEST_HOST)
    bobj = os.path.join(BUILD, "batch_bench.o")
    _run([HIPCC, *HOST_FLAGS, "-c", os.path.join(HERE, "host", "batch_bench.cpp"), "-o", bobj])
    _run([HIPCC, "-o", BATCH_BENCH + ".tmp", bobj, "-L" + HERE, "-llocus_host", "-llocus_sampler",
          "-Wl,-rpath,$ORIGIN"])
    os.replace(BATCH_BENCH + ".tmp", BATCH_BENCH)
    return HOST_SO


ASAN_DIR = os.path.join(BUILD, "asan")
SAN_FLAGS = ["-std=c++20", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
             "-fno-sanitize-recover=undefined"]
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def build_sanitized(jobs: int = 4) -> dict:
    """Host layer + tests/cpp/test_host, and tests/cpp/oracle_asan over
    oracle/oracle.cpp, built with g++ -fsanitize=address,undefined. Returns
    the two programs' paths."""
    os.makedirs(ASAN_DIR, exist_ok=True)
    hip = ["-D__HIP_PLATFORM_AMD__", "-I" + os.path.join(ROCM, "include"), "-I" + INCLUDE]
    objs, cmds = [], []
    for src in HOST_SOURCES:
        obj = os.path.join(ASAN_DIR, src.replace(".cpp", ".o"))
        objs.append(obj)
        cmds.append(["g++", *SAN_FLAGS, "-fPIC", "-Wall", *hip, "-c", os.path.join(HERE, "host", src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    so = os.path.join(ASAN_DIR, "liblocus_host_asan.so")
    rocm_lib = os.path.join(ROCM, "lib")
    links = ["-L" + HERE, "-llocus_sampler", "-L" + rocm_lib, "-lamdhip64",
             "-Wl,-rpath," + HERE, "-Wl,-rpath," + rocm_lib]
    _run(["g++", "-shared", "-fsanitize=address,undefined", "-o", so, *objs, *links])
    test_host = os.path.join(ASAN_DIR, "test_host_asan")
    _run(["g++", *SAN_FLAGS, *hip, os.path.join(ROOT, "tests", "cpp", "test_host.cpp"), "-o", test_host,
          "-L" + ASAN_DIR, "-llocus_host_asan", "-Wl,-rpath," + ASAN_DIR, *links])
    oracle = os.path.join(ASAN_DIR, "oracle_asan")
    _run(["g++", *SAN_FLAGS, "-ffp-contract=off", os.path.join(ROOT, "tests", "cpp", "oracle_asan.cpp"),
          os.path.join(ROOT, "oracle", "oracle.cpp"), "-o", oracle, "-lpthread"])
    return {"test_host": test_host, "oracle": oracle}


def build_all() -> None:
    build_sampler()
    build_host()
    build_sampler(profile=True)


if __name__ == "__main__":
    build_all()
    print("built", SAMPLER_SO)
