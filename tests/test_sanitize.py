"""The host layer and the CPU oracle under AddressSanitizer and
UndefinedBehaviorSanitizer (g++ builds of locus_amd/build.py:build_sanitized):
the host program's CPU checks (grammar, mask builder against per-token
allows(), n-gram draft, registry) and a driver of every oracle entry point on
random and edge-case inputs must run without a sanitizer report."""
import os
import subprocess

from locus_amd import build

ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=23",
           UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")


def _run(path, *args):
    r = subprocess.run([path, *args], capture_output=True, text=True, timeout=300, env=ENV)
    print(r.stdout[-2000:], r.stderr[-4000:])
    assert r.returncode == 0, r.stderr[-4000:]
    assert "ERROR: AddressSanitizer" not in r.stderr
    assert "runtime error:" not in r.stderr
    return r


def test_host_layer_and_oracle_under_sanitizers():
    if not os.path.exists(build.SAMPLER_SO):
        build.build_all()
    progs = build.build_sanitized()
    r = _run(progs["test_host"], "cpu")
    assert ", 0 failed" in r.stdout
    r = _run(progs["oracle"])
    assert "0 failures" in r.stdout
