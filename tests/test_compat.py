"""The drop-in boundary against the reference's own code (oracle/Makefile's
`compat` target, built in place from /root/reference into oracle/_ref/):

* the reference's tests/test_sampling.cpp, test_grammar.cpp and
  test_speculative.cpp, unchanged, linked against include/ +
  liblocus_host.so (grammar and n-gram cases on the CPU, every case on the
  GPU);
* the reference's engine.hpp and include/locus/engine/batch_sampler.hpp in
  one translation unit, with sample_step bound to the engine's Request;
* the reference's sampling.cpp registered as the "scalar" sampler backend:
  best_sampler_backend() never throws (registry.cpp:105-111), and on the GPU
  the hip and scalar entries agree row for row.

The binaries are built here (where /root/reference exists) and travel with
the tree; without them and without the reference sources these tests skip."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_DIR = os.path.join(ROOT, "oracle", "_ref")
REF_SRC = "/root/reference/src/locus/model"
BINS = ("ref_tests", "registry_fallback", "engine_compat.o")


def _have_or_build():
    if all(os.path.exists(os.path.join(REF_DIR, b)) for b in BINS):
        return True
    if not os.path.isdir(REF_SRC):
        return False
    from locus_amd import build
    if not os.path.exists(build.HOST_SO):
        build.build_all()
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "ref", "compat"], check=True)
    return True


def _run(args, timeout=300):
    r = subprocess.run(args, capture_output=True, text=True, timeout=timeout)
    print(r.stdout[-3000:], r.stderr[-3000:])
    return r


def test_reference_tests_and_engine_header_cpu():
    if not _have_or_build():
        pytest.skip("neither the compat binaries nor the reference sources are present")
    r = _run([os.path.join(REF_DIR, "ref_tests"), "[grammar],[spec]"])
    assert r.returncode == 0
    assert "All tests passed" in r.stdout
    assert os.path.getsize(os.path.join(REF_DIR, "engine_compat.o")) > 0
    r = _run([os.path.join(REF_DIR, "registry_fallback"), "cpu"])
    assert r.returncode == 0
    assert "best=scalar" in r.stdout


@pytest.mark.gpu
def test_reference_tests_gpu():
    if not all(os.path.exists(os.path.join(REF_DIR, b)) for b in BINS[:2]):
        pytest.skip("compat binaries not built (they are built where the reference sources exist)")
    r = _run([os.path.join(REF_DIR, "ref_tests")])
    assert r.returncode == 0
    assert "All tests passed" in r.stdout
    r = _run([os.path.join(REF_DIR, "registry_fallback"), "gpu"])
    assert r.returncode == 0
    assert "best=hip, 300 rows compared, 0 failures" in r.stdout
