"""The C++ host layer: JSON grammar, allow-mask builder and n-gram draft
against the compiled reference's golden vectors (tests/golden/grammar.json,
ngram.json) and the pinned oracle; backend resolution; the C++ test program
(the reference's own KATs, restated)."""
import os
import subprocess

import numpy as np
import pytest

from locus_amd import host_lib as H
from oracle import pyoracle as O
from tests.util import load

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TEST_HOST = os.path.join(ROOT, "tests", "cpp", "test_host")


def _test_host(mode):
    if not os.path.exists(TEST_HOST):
        from locus_amd import build
        build.build_all()
    r = subprocess.run([TEST_HOST, mode], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr


def test_cpp_host_program_cpu():
    _test_host("cpu")


def test_grammar_matches_reference_strings():
    fx = load("grammar.json")
    for s in fx["strings"]:
        g = H.JsonGrammar()
        n = 0
        for b in s["bytes"]:
            if not g.feed(b):
                break
            n += 1
        assert n == s["accepted"], bytes(s["bytes"])
        assert int(g.complete()) == s["complete"], bytes(s["bytes"])


def test_mask_matches_reference_masks():
    fx = load("grammar.json")
    pieces = [bytes(p) for p in fx["pieces"]]
    mb = H.MaskBuilder(pieces)
    for m in fx["masks"]:
        g = H.JsonGrammar()
        ok = all(g.feed(b) for b in m["prefix"])
        assert ok == (m["rc"] == 0)
        if ok:
            got = mb.build(g, fx["vocab"])
            assert got.tolist() == m["mask"], bytes(m["prefix"])
            assert mb.build(g, fx["vocab"]).tolist() == m["mask"]   # cached


def test_mask_matches_oracle_on_random_states():
    rng = np.random.default_rng(3)
    alphabet = list(b'{}[]",:0123456789.-+eEtrufalsn \\/u\n')
    pieces = [bytes([b]) for b in range(256)]
    for _ in range(800):
        n = int(rng.integers(0, 10))
        pieces.append(bytes(int(alphabet[i]) for i in rng.integers(0, len(alphabet), n)))
    V = len(pieces) + 9
    mb = H.MaskBuilder(pieces, cache_entries=8)
    docs = [b'{"k": [1, {"a": "b\\u00e9"}, true, null], "n": -1.5e+3}', b'[[[], {}], "x\\n", 0, false]']
    checked = 0
    for d in docs:
        g, o = H.JsonGrammar(), O.OracleJson()
        for i in range(len(d) + 1):
            assert mb.build(g, V).tolist() == o.mask(pieces, V).tolist(), d[:i]
            checked += 1
            if i < len(d):
                assert g.feed(d[i]) and o.feed(d[i])
    assert checked > 80
    hits, misses = mb.cache_stats()
    assert hits + misses == checked


def test_ngram_matches_reference():
    for c in load("ngram.json"):
        assert H.ngram_draft(c["ctx"], c["ngram"], c["max_draft"]) == c["draft"], c


def test_backend_resolution_without_device():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a device is present: covered by test_cpp_host_program_gpu")
    assert H.resolve_sampler_backend("")[0] == -2
    assert H.resolve_sampler_backend("hip")[0] == -1
    assert H.resolve_sampler_backend("scalar")[0] == -1


@pytest.mark.gpu
def test_cpp_host_program_gpu():
    _test_host("gpu")
    assert H.resolve_sampler_backend("") == (0, "hip")
