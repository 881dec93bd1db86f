"""On-device n-gram drafts (lcs_ngram_draft, lcs_draft.hip) against the
compiled reference's ngram_draft (tests/golden/ngram.json, from
speculative.cpp:7-28), the reference's KATs (tests/test_speculative.cpp:9-32)
and the pinned oracle on random and long contexts."""
import numpy as np
import pytest

from oracle import pyoracle as O
from tests.util import load


@pytest.fixture(scope="module")
def sampler():
    from locus_amd.sampler import Sampler
    s = Sampler(device=0, max_rows=4096, max_vocab=1024, max_hist=64, max_top=4)
    yield s
    s.close()


@pytest.mark.gpu
def test_draft_golden(sampler):
    fx = load("ngram.json")
    by = {}
    for c in fx:   # one batched call per (ngram, max_draft)
        by.setdefault((c["ngram"], c["max_draft"]), []).append(c)
    for (ng, md), cases in by.items():
        got, _ = sampler.ngram_draft([c["ctx"] for c in cases], ng, md)
        for c, g in zip(cases, got):
            assert g == c["draft"], c


@pytest.mark.gpu
def test_draft_reference_kats(sampler):
    got, raw = sampler.ngram_draft([[1, 2, 3, 4, 1, 2, 3], [5, 6, 7], [1, 2], [1, 2, 3, 1, 2]], 2, 3)
    assert got == [[4, 1, 2], [], [], [3, 1, 2]]
    assert raw[1].tolist() == [-1, -1, -1]   # entries past the draft are -1
    got, raw = sampler.ngram_draft([[9, 9, 5, 9, 9, 7, 9, 9]], 2, 2)
    assert got == [[7, 9]]
    got, _ = sampler.ngram_draft([[5, 6, 7]], 0, 3)
    assert got == [[]]
    got, raw = sampler.ngram_draft([[1, 2, 1, 2]], 1, 0)
    assert got == [[]] and raw.shape == (1, 0)


@pytest.mark.gpu
def test_draft_random_and_long_contexts(sampler):
    rng = np.random.default_rng(11)
    ctxs, params = [], []
    for i in range(600):
        n = int(rng.integers(0, 40)) if i % 3 else int(rng.integers(200, 3000))
        alpha = int(rng.integers(2, 6)) if i % 4 else 1000
        ctxs.append(rng.integers(0, alpha, n).astype(np.int32).tolist())
    # the match far back: a unique trailing n-gram that occurs once near the start
    long_ctx = list(range(100000, 100005)) + rng.integers(0, 50, 100000).tolist() + list(range(100002, 100005))
    ctxs.append(long_ctx)
    for ng, md in [(1, 4), (2, 8), (3, 5), (4, 16), (8, 256), (64, 7)]:
        got, _ = sampler.ngram_draft(ctxs, ng, md)
        for c, g in zip(ctxs, got):
            assert g == O.ngram_draft(c, ng, md), (len(c), ng, md)
    # the trailing 3-gram 100002..100004 occurs only at position 2: the draft is
    # the four tokens after it, 100000 positions back
    got, _ = sampler.ngram_draft([long_ctx], 3, 4)
    assert got == [long_ctx[5:9]] == [O.ngram_draft(long_ctx, 3, 4)]


@pytest.mark.gpu
def test_draft_matches_at_round_boundaries(sampler):
    """Contexts whose only earlier occurrence of the trailing n-gram starts at,
    just before or just after a boundary between the kernel's rounds of 4096
    candidate starts (the n-gram then straddles two rounds' token ranges), and
    at the very first position."""
    rng = np.random.default_rng(29)
    chunk = 4096
    for ng in (1, 2, 3, 7, 64):
        ctxs = []
        for n in (chunk + ng + 1, 2 * chunk + ng + 5, 3 * chunk + 2 * ng + 3):
            last = n - ng - 1                     # the most recent candidate start
            for j in (1, 2):
                b = last + 1 - j * chunk          # a round boundary (first start of round j)
                for s in (b - ng, b - 1, b, b + 1, 0):
                    if not 0 <= s <= last:
                        continue
                    ctx = rng.integers(0, 1 << 20, n).astype(np.int32)
                    pat = np.arange(7_000_000, 7_000_000 + ng, dtype=np.int32)
                    ctx[n - ng:] = pat
                    ctx[s:s + ng] = pat
                    ctxs.append(ctx.tolist())
        for md in (5, 256):
            got, _ = sampler.ngram_draft(ctxs, ng, md)
            for c, g in zip(ctxs, got):
                want = O.ngram_draft(c, ng, md)
                assert g == want, (len(c), ng, md)
                assert len(want) > 0


@pytest.mark.gpu
def test_draft_rejects_bad_arguments(sampler):
    from locus_amd.sampler import SamplerError
    with pytest.raises(SamplerError):
        sampler.ngram_draft([[1, 2, 3]], 65, 4)
    with pytest.raises(SamplerError):
        sampler.ngram_draft([[1, 2, 3]], 2, 257)
