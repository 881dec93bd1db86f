"""The lm-head feeding the sampler: lcs_lmhead writes the logits and each
row's raw statistics (lcs_lmhead_out.stats), and lcs_sample takes them
through lcs_batch.raw_stats, so the sliced path's slices skip their raw sums
and row_fin takes the lm-head's log-normaliser (llama.cpp:512-513 produces
the logits that Engine::sample_from samples, engine.cpp:423-450;
logprobs_from's normaliser is sampling.cpp:155-163).

The sampled ids, survivor counts and logprobs are checked against the CPU
oracle on the lm-head's own written logits (the same gate as every sampling
test), and against the same lcs_sample call without the statistics: ids and
survivor counts bit-exact, logprobs within 1e-5.
"""
import numpy as np
import pytest

from locus_amd import workloads as W
from oracle import pyoracle as O
from tests.test_gpu_sampling import compare, say
from tests.util import LOGPROB_TOL

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sampler():
    from locus_amd.sampler import Sampler
    s = Sampler(device=0, max_rows=64, max_vocab=131072, max_hist=4096, max_top=20)
    yield s
    s.close()


def lmhead_logits(sampler, rows, vocab, hidden, seed, scale=3.0):
    """bf16 x (rows, hidden) and w (vocab, hidden) whose product has about
    N(0, scale^2) entries; returns the lm-head's outputs (logits, stats)."""
    torch = sampler.torch
    dev = torch.device("cuda", 0)
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(rows, hidden, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(vocab, hidden, generator=g) * (scale / hidden ** 0.5)).to(torch.bfloat16).to(dev)
    out = sampler.alloc_lmhead_out(rows, vocab, logits=True, stats=True)
    sampler.lmhead_dev(x, w, out)
    torch.cuda.synchronize()
    return out


def check_stats(out):
    """The statistics the lm-head reports against its own logits."""
    lg = out["logits"].cpu().numpy()
    st = out["stats"].cpu().numpy()
    log_z = st[:, 0]
    words = np.ascontiguousarray(st).view(np.uint32).reshape(-1, 4)   # (log_z lo, hi, max, argmax)
    mx, am = words[:, 2].view(np.float32), words[:, 3].view(np.int32)
    l64 = lg.astype(np.float64)
    m = l64.max(axis=1)
    lz = m + np.log(np.exp(l64 - m[:, None]).sum(axis=1))
    assert np.abs(log_z - lz).max() <= 2e-6
    assert np.array_equal(mx, lg.max(axis=1))
    assert np.array_equal(am, np.argmax(lg, axis=1).astype(np.int32))
    return lg


def sample_both(sampler, w, stats):
    """lcs_sample on w's logits with and without the lm-head's statistics."""
    res = []
    for rs in (stats, None):
        d = sampler.upload(w)
        out = sampler.alloc_out(w.rows, w.n_top, w.want_logprobs)
        sampler.sample_dev(d, out, raw_stats=rs)
        sampler.torch.cuda.synchronize()
        assert sampler.status() == 0
        res.append(sampler.fetch(out, w.n_top))
    return res


def test_c2_batch_through_the_lmhead(sampler):
    """C2's chain (penalties, T 0.7, min-p 0.05, top-p 0.9, top-5 logprobs)
    on 64 rows of lm-head logits at V=128256."""
    base = W.make("c2")
    out = lmhead_logits(sampler, base.rows, base.vocab, 512, seed=11)
    lg = check_stats(out)
    w = W.Workload("c2-lmhead", base.rows, base.vocab, "f32", lg, base.params, base.seeds, base.u,
                   base.hist_off, base.hist_ids, None, 5, True)
    g, g0 = sample_both(sampler, w, out["stats"])
    say("lmhead chain c2", int((g["ids"] == g0["ids"]).sum()), "of", w.rows, "ids equal")
    assert np.array_equal(g["ids"], g0["ids"])
    assert np.array_equal(g["diag"]["keep"], g0["diag"]["keep"])
    assert np.abs(g["chosen_lp"] - g0["chosen_lp"]).max() <= LOGPROB_TOL
    assert np.array_equal(g["top_ids"], g0["top_ids"])
    assert np.abs(g["top_lp"] - g0["top_lp"]).max() <= LOGPROB_TOL
    compare(w, g, O.sample_batch(w, threads=16), "lmhead-c2", expect_paths={2, 3})


def test_mixed_rows_through_the_lmhead(sampler):
    """Greedy, min-p window, top-k (sliced), top-p-only (nucleus: computes
    its own normaliser) and plain-temperature rows in one batch."""
    base = W.make("c2", rows=16, set_index=5)
    out = lmhead_logits(sampler, base.rows, base.vocab, 256, seed=12, scale=2.0)
    lg = check_stats(out)
    p = base.params.copy()
    p["temperature"][0:3] = 0.0
    p["min_p"][3:6], p["top_k"][3:6] = 0.0, 40
    p["temperature"][6:8], p["top_p"][6:8], p["min_p"][6:8] = 1.5, 0.98, 0.0
    p["min_p"][8], p["top_p"][8] = 0.0, 1.0
    w = W.Workload("mixed-lmhead", base.rows, base.vocab, "f32", lg, p, base.seeds, base.u,
                   base.hist_off, base.hist_ids, None, 5, True)
    g, g0 = sample_both(sampler, w, out["stats"])
    assert np.array_equal(g["ids"], g0["ids"])
    assert np.abs(g["chosen_lp"] - g0["chosen_lp"]).max() <= LOGPROB_TOL
    assert np.abs(g["top_lp"] - g0["top_lp"]).max() <= LOGPROB_TOL
    compare(w, g, O.sample_batch(w, threads=16), "lmhead-mixed")


def logprobs_case(sampler, w, chosen, raw_stats=None, label="logprobs"):
    """lcs_logprobs on w's logits against the oracle's logprobs_from per row:
    chosen_lp and top_lp within 1e-5, top ids bit-exact outside exact ties,
    out.ids the first index of the max."""
    torch = sampler.torch
    dev = torch.device("cuda", 0)
    d = sampler.upload(w)
    out = sampler.alloc_out(w.rows, w.n_top, True, diag=False)
    ch = None if chosen is None else torch.from_numpy(np.asarray(chosen, dtype=np.int32)).to(dev)
    sampler.logprobs_dev(d, out, chosen=ch, raw_stats=raw_stats)
    torch.cuda.synchronize()
    assert sampler.status() == 0
    g = sampler.fetch(out, w.n_top)
    lg = W.bf16_to_f32(w.logits) if w.dtype == "bf16" else w.logits
    assert np.array_equal(g["ids"], np.argmax(lg, axis=1).astype(np.int32)), label
    for r in range(w.rows):
        c = int(np.argmax(lg[r])) if chosen is None else int(chosen[r])
        lp, ids, lps, tie = O.logprobs(lg[r], c, w.n_top)
        assert abs(g["chosen_lp"][r] - lp) <= LOGPROB_TOL, (label, r)
        assert np.abs(g["top_lp"][r] - lps).max() <= LOGPROB_TOL, (label, r)
        if not tie:
            assert np.array_equal(g["top_ids"][r], ids), (label, r)
    say(label, "rows", w.rows, "ok")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_logprobs_batch(sampler, dtype):
    """logprobs_from over a batch (the registry's logprobs_batch op), chosen
    ids inside and outside [0, V), and with each row's argmax as chosen; the
    rows' params, history and u play no part."""
    base = W.make("c2", rows=16, set_index=21)
    lg = W.bf16_rne(base.logits) if dtype == "bf16" else base.logits
    w = W.Workload("lp", base.rows, base.vocab, dtype, lg, base.params, base.seeds, base.u,
                   base.hist_off, base.hist_ids, None, 5, True)
    rng = np.random.default_rng(4)
    chosen = rng.integers(0, base.vocab, size=base.rows).astype(np.int32)
    chosen[0], chosen[1], chosen[2] = -1, base.vocab, base.vocab - 1
    logprobs_case(sampler, w, chosen, label=f"logprobs-{dtype}")
    logprobs_case(sampler, w, None, label=f"logprobs-{dtype}-argmax")


def test_logprobs_batch_with_lmhead_stats(sampler):
    """lcs_logprobs taking the lm-head's log-normalisers."""
    base = W.make("c2", rows=32, set_index=22)
    out = lmhead_logits(sampler, base.rows, base.vocab, 256, seed=13)
    lg = check_stats(out)
    w = W.Workload("lp-lmhead", base.rows, base.vocab, "f32", lg, base.params, base.seeds, base.u,
                   None, None, None, 5, True)
    chosen = np.random.default_rng(5).integers(0, base.vocab, size=base.rows).astype(np.int32)
    logprobs_case(sampler, w, chosen, raw_stats=out["stats"], label="logprobs-lmhead")
