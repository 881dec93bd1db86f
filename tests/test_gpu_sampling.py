"""GPU parity of the HIP sampler (through the C ABI) against the CPU oracle
and the reference's golden vectors.

Bar: sampled / greedy ids and survivor counts bit-exact, except rows the
oracle flags as exact ties or near ties (|decision - threshold| < NEAR_TIE,
relative); logprobs within 1e-5 absolute."""
import math
import sys

import numpy as np
import pytest

from locus_amd import workloads as W
from oracle import pyoracle as O
from tests.util import LOGPROB_TOL, excluded_rows, load, near_tie_rows, penalized_value

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sampler():
    from locus_amd.sampler import Sampler
    s = Sampler(device=0, max_rows=4096, max_vocab=262144, max_hist=4096, max_top=20)
    yield s
    s.close()


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def top_tied(raw_row, n):
    """True when the reference's top-n order/membership depends on ties."""
    if n == 0:
        return False
    srt = np.sort(raw_row)[::-1]
    head = srt[:n + 1]
    return len(np.unique(head)) < len(head)


def compare(w, g, o, label, expect_paths=None):
    greedy = w.params["temperature"] <= 0
    excl = excluded_rows(o.diag) & ~greedy
    bad = np.nonzero((g["ids"] != o.ids) & ~excl)[0]
    if len(bad):
        r = bad[0]
        say(label, "mismatch rows", bad[:10].tolist(), "gpu", g["ids"][bad[:10]].tolist(),
            "oracle", o.ids[bad[:10]].tolist(), "diag", g["diag"][r], "odiag", o.diag[r])
    assert len(bad) == 0, f"{label}: {len(bad)} id mismatches"
    stoch = ~greedy & ~excl
    kb = np.nonzero(stoch & (g["diag"]["keep"] != o.diag["keep"]))[0]
    assert len(kb) == 0, f"{label}: survivor counts differ at rows {kb[:10].tolist()} " \
                         f"gpu {g['diag']['keep'][kb[:10]].tolist()} oracle {o.diag['keep'][kb[:10]].tolist()}"
    # exact-tie rows (not near ties): the order among equal logits cannot
    # change the survivor count, the kept mass (equal weights give equal f64
    # sums in any order) or the drawn position, so only which of several
    # equal-logit ids is drawn may differ: its penalised logit must be the
    # reference's id's
    tie = (o.diag["tie_flags"] != 0) & ~near_tie_rows(o.diag) & ~greedy
    for r in np.nonzero(tie)[0]:
        assert g["diag"]["keep"][r] == o.diag["keep"][r], \
            f"{label} tie row {r}: keep {g['diag']['keep'][r]} vs {o.diag['keep'][r]}"
        # (the reference adds the keep weights one by one in f64: recursive
        # summation of n terms carries up to n * 2^-53 of the sum in rounding,
        # and so may a sum in another order; rows of many equal weights reach
        # that bound, e.g. 118747 kept weights of three values differ by
        # 3.2e-12 relative)
        ks, oks = float(g["diag"]["kept_sum"][r]), float(o.diag["kept_sum"][r])
        tol = (1e-12 + float(o.diag["keep"][r]) * 2.0 ** -52) * oks
        assert abs(ks - oks) <= tol, f"{label} tie row {r}: kept_sum {ks!r} vs {oks!r}"
        gv, ov = penalized_value(w, r, int(g["ids"][r])), penalized_value(w, r, int(o.ids[r]))
        assert gv == ov, f"{label} tie row {r}: drew {g['ids'][r]} ({gv!r}), reference {o.ids[r]} ({ov!r})"
    if w.want_logprobs:
        same = g["ids"] == o.ids
        err = np.abs(g["chosen_lp"] - o.chosen_lp)[same]
        assert (err <= LOGPROB_TOL).all(), f"{label}: chosen lp err {err.max()}"
        for r in range(w.rows):
            n = w.n_top
            raw = np.asarray(w.logits[r], dtype=np.float32)
            if not top_tied(raw, n):
                assert g["top_ids"][r].tolist() == o.top_ids[r, :n].tolist(), f"{label} row {r} top ids"
            assert np.allclose(g["top_lp"][r], o.top_lp[r, :n], atol=LOGPROB_TOL, rtol=0)
    if expect_paths is not None:
        assert set(np.unique(g["diag"]["path"]).tolist()) <= set(expect_paths), \
            f"{label}: paths {np.unique(g['diag']['path']).tolist()}"
    say(label, "rows", w.rows, "excluded", int(excl.sum()), "of which exact ties checked", int(tie.sum()),
        "paths", np.unique(g["diag"]["path"]).tolist())
    return excl


def run(sampler, w, **kw):
    g = sampler.sample(w, **kw)
    st = sampler.status()
    assert st == 0, f"device status {st}"
    return g


@pytest.mark.parametrize("idx", range(5))
def test_golden_configs(sampler, idx):
    fx = load("configs.json")["sampling"][idx]
    name = fx["workload"]
    say("golden", name)
    w = W.make(name, rows=fx["rows"] if name not in ("c1g", "c1s") else None)
    assert w.input_checksum() == fx["checksum"]
    g = run(sampler, w)
    o = O.sample_batch(w, threads=16)
    excl = compare(w, g, o, f"golden-{name}")
    ref_ids = np.array(fx["ids"])
    assert ((g["ids"] == ref_ids) | excl).all()
    if w.want_logprobs:
        same = g["ids"] == ref_ids
        assert (np.abs(g["chosen_lp"] - np.array(fx["chosen_lp"]))[same] <= LOGPROB_TOL).all()


@pytest.mark.parametrize("name,rows", [("c2", 64), ("c3", 48), ("c4", 32)])
def test_fresh_inputs(sampler, name, rows):
    say("fresh", name, rows)
    w = W.make(name, rows=rows, set_index=3)
    compare(w, run(sampler, w), O.sample_batch(w, threads=16), f"fresh-{name}")


def test_large_magnitude_logits(sampler):
    """Logits offset by +300: the f32 exp2 sums share an exponent error of up
    to half an ulp of 300 log2(e) unless it is taken out; logprobs must stay
    within 1e-5 (sliced, nucleus and verify paths)."""
    import dataclasses
    off = np.float32(300.0)
    w2 = W.make("c2", rows=32, set_index=5)
    w2 = dataclasses.replace(w2, logits=w2.logits + off)
    compare(w2, run(sampler, w2), O.sample_batch(w2, threads=16), "offset-c2")
    w3 = W.make("c3", rows=16, set_index=5)
    w3 = dataclasses.replace(w3, logits=w3.logits + off, want_logprobs=True, n_top=3)
    compare(w3, run(sampler, w3), O.sample_batch(w3, threads=16), "offset-c3")
    w5 = W.make("c5", rows=64, set_index=5)
    w5 = dataclasses.replace(w5, dtype="f32", logits=W.bf16_to_f32(w5.logits) + off)
    g = sampler.verify(w5)
    am, lp, acc = O.verify(w5, threads=16)
    assert np.array_equal(g["argmax_ids"], am)
    assert np.abs(g["draft_lp"] - lp).max() <= LOGPROB_TOL
    assert np.array_equal(g["accept_len"].astype(np.uint32), acc)


def test_full_size_c2(sampler):
    say("full c2")
    w = W.make("c2")
    g = run(sampler, w)
    compare(w, g, O.sample_batch(w, threads=16), "full-c2")


def test_full_size_c3(sampler):
    say("full c3")
    w = W.make("c3")
    compare(w, run(sampler, w), O.sample_batch(w, threads=16), "full-c3")


def test_edge_cases(sampler):
    from tests.golden.make_golden import edge_workloads
    for w in edge_workloads():
        say("edge", w.name, w.vocab)
        compare(w, run(sampler, w), O.sample_batch(w), f"edge-{w.name}")


def test_edge_cases_padded_stride(sampler):
    from tests.golden.make_golden import edge_workloads
    for w in edge_workloads():
        say("edge-padded", w.name, w.vocab)
        d = sampler.upload(w, stride=((w.vocab + 3) // 4) * 4 + 8)
        out = sampler.alloc_out(w.rows, w.n_top, w.want_logprobs)
        sampler.sample_dev(d, out)
        sampler.torch.cuda.synchronize()
        g = sampler.fetch(out, w.n_top)
        assert sampler.status() == 0
        compare(w, g, O.sample_batch(w), f"edge-padded-{w.name}")


@pytest.mark.parametrize("kind", ["c2", "topk"])
def test_deterministic_and_host_params_optional(sampler, kind):
    """Without params_host the host cannot pick the row modes' launch shapes
    (for top-k rows: the finalize that requests the lists at launch); the
    results must not change."""
    w = W.make("c2", rows=16, set_index=5)
    if kind == "topk":
        p = w.params.copy()
        p["top_k"] = [40, 5, 64, 1, 17, 40, 0, 40, 64, 2, 40, 8, 33, 40, 64, 40]
        w = W.Workload("topk-hp", w.rows, w.vocab, "f32", w.logits, p, w.seeds, w.u, w.hist_off, w.hist_ids,
                       None, w.n_top, w.want_logprobs)
    a = run(sampler, w)
    b = run(sampler, w, use_host_params=False)
    assert np.array_equal(a["ids"], b["ids"])
    assert a["diag"].tobytes() == b["diag"].tobytes()
    assert np.array_equal(a["top_lp"], b["top_lp"])
    if kind == "topk":
        compare(w, a, O.sample_batch(w, threads=8), "topk-hp", expect_paths={2, 3, 4, 5})


def test_missing_u_is_rejected_before_any_launch(sampler):
    # without params_host the row modes are unknown on the host, so u is
    # required; with params_host it is required only by stochastic rows
    from locus_amd.sampler import LCS_ERR_INVALID_ARG, SamplerError
    w = W.make("c2", rows=4, set_index=3)
    d = sampler.upload(w)
    d.pop("u")
    out = sampler.alloc_out(w.rows, w.n_top, w.want_logprobs)
    for host_params in (False, True):
        with pytest.raises(SamplerError, match=f"lcs error {LCS_ERR_INVALID_ARG}"):
            sampler.sample_dev(d, out, use_host_params=host_params)
    sampler.torch.cuda.synchronize()
    assert (out["ids"].cpu().numpy() == -7).all(), "a kernel ran"
    # greedy rows need no u when the host sees their params
    g = W.make("c1g")
    assert (g.params["temperature"] <= 0).all()
    dg = sampler.upload(g)
    dg.pop("u", None)
    og = sampler.alloc_out(g.rows, g.n_top, g.want_logprobs)
    sampler.sample_dev(dg, og)
    sampler.torch.cuda.synchronize()
    assert og["ids"].cpu().numpy()[0] == O.sample_batch(g).ids[0]


def test_mixed_modes_in_one_batch(sampler):
    # one batch mixing greedy, min-p window, top-k and top-p-only rows
    base = W.make("c2", rows=8, set_index=7)
    p = base.params.copy()
    p["temperature"][0] = 0.0
    p["min_p"][1], p["top_k"][1] = 0.0, 40
    p["min_p"][2] = 0.0
    p["temperature"][3], p["top_p"][3], p["min_p"][3] = 1.5, 0.98, 0.0
    p["repeat_penalty"][4] = 1.0
    p["frequency_penalty"][4] = 0.0
    p["presence_penalty"][4] = 0.0
    w = W.Workload("mixed", base.rows, base.vocab, "f32", base.logits, p, base.seeds, base.u,
                   base.hist_off, base.hist_ids, None, 5, True)
    compare(w, run(sampler, w), O.sample_batch(w, threads=8), "mixed")


def test_bf16_logits(sampler):
    base = W.make("c2", rows=16, set_index=9)
    b = W.bf16_rne(base.logits)
    w16 = W.Workload("c2bf16", base.rows, base.vocab, "bf16", b, base.params, base.seeds,
                     base.u, base.hist_off, base.hist_ids, None, 5, True)
    w32 = W.Workload("c2bf16-as-f32", base.rows, base.vocab, "f32", W.bf16_to_f32(b), base.params,
                     base.seeds, base.u, base.hist_off, base.hist_ids, None, 5, True)
    g = run(sampler, w16)
    compare(w32, g, O.sample_batch(w32, threads=8), "bf16")


def test_write_penalized_in_place(sampler):
    w = W.make("c2", rows=4, set_index=11)
    d = sampler.upload(w)
    out = sampler.alloc_out(w.rows, w.n_top, w.want_logprobs)
    from locus_amd.sampler import LCS_WRITE_PENALIZED
    sampler.sample_dev(d, out, flags_extra=LCS_WRITE_PENALIZED)
    sampler.torch.cuda.synchronize()
    g = sampler.fetch(out, w.n_top)
    o = O.sample_batch(w, threads=4)
    compare(w, g, o, "write-penalized")
    after = d["logits"].cpu().numpy()[:, :w.vocab]
    assert np.array_equal(after, o.penalized)


def test_verify_golden(sampler):
    fx = load("configs.json")["verify"]
    w = W.make("c5", rows=fx["rows"])
    assert w.input_checksum() == fx["checksum"]
    say("verify golden")
    g = sampler.verify(w)
    assert g["argmax_ids"].tolist() == fx["argmax"]
    assert np.allclose(g["draft_lp"], np.array(fx["draft_lp"]), atol=LOGPROB_TOL, rtol=0)
    assert g["accept_len"].tolist() == fx["accept_len"]


def test_verify_full_size(sampler):
    say("verify full c5")
    w = W.make("c5")
    g = sampler.verify(w)
    am, lp, acc = O.verify(w, threads=16)
    assert np.array_equal(g["argmax_ids"], am)
    assert np.abs(g["draft_lp"] - lp).max() <= LOGPROB_TOL
    assert np.array_equal(g["accept_len"].astype(np.uint32), acc)


def test_hist_capacity_is_reported(sampler):
    from locus_amd.sampler import Sampler
    small = Sampler(device=0, max_rows=4, max_vocab=1024, max_hist=16, max_top=4)
    try:
        V = 1024
        p = W.default_params(2)
        p["temperature"] = 1.0
        p["top_p"] = 0.9
        p["repeat_penalty"] = 1.2
        p["repeat_last_n"] = 64
        hist = np.arange(2 * 40, dtype=np.int32) % V
        w = W.Workload("cap", 2, V, "f32", np.zeros((2, V), np.float32), p,
                       np.zeros(2, np.uint64), np.full(2, 0.5), np.array([0, 40, 80], np.uint32), hist)
        g = small.sample(w)
        assert (g["ids"] == -1).all()
        assert small.status() & 1
    finally:
        small.close()


def test_logprobs_of_given_ids(sampler):
    """lp_ids: chosen_lp reports logprobs_from(raw, lp_ids[row], n) on both
    paths (sliced: c2 / c1g, exact: c3), ids outside [0, V) giving 0."""
    import torch
    for name, rows in (("c2", 8), ("c3", 6), ("c1g", None)):
        w = W.make(name, rows=rows, set_index=13)
        ids = np.random.default_rng(5).integers(-2, w.vocab + 2, size=w.rows).astype(np.int32)
        ids[0] = -1
        if w.rows > 1:
            ids[1] = w.vocab
        say("lp_ids", name, ids.tolist())
        d = sampler.upload(w)
        out = sampler.alloc_out(w.rows, 3, True)
        lp_ids = torch.from_numpy(ids).cuda()
        sampler.sample_dev(d, out, n_top=3, want_lp=True, lp_ids=lp_ids)
        sampler.torch.cuda.synchronize()
        g = sampler.fetch(out, 3)
        assert sampler.status() == 0
        for r in range(w.rows):
            raw = np.asarray(w.logits[r], dtype=np.float32)
            lp, tid, tlp, _ = O.logprobs(raw, int(ids[r]), 3)
            assert abs(float(g["chosen_lp"][r]) - lp) <= LOGPROB_TOL, (name, r, g["chosen_lp"][r], lp)
            assert np.allclose(g["top_lp"][r], tlp, atol=LOGPROB_TOL, rtol=0)


def test_topk_rows_on_the_sliced_path(sampler):
    """top_k <= 64 rows run on the sliced exact top-k path (path 5), with and
    without penalties, top-p and min-p; top_k 65 takes the nucleus path (6)."""
    base = W.make("c2", rows=12, set_index=17)
    p = base.params.copy()
    ks = [1, 2, 5, 17, 40, 64, 40, 40, 64, 8, 65, 33]
    for r, k in enumerate(ks):
        p["top_k"][r] = k
        p["min_p"][r] = 0.0 if r % 3 else 0.05
        p["top_p"][r] = 1.0 if r % 4 == 1 else 0.9
        p["temperature"][r] = [0.7, 1.0, 1.5][r % 3]
    p["repeat_penalty"][6] = 1.0
    p["frequency_penalty"][6] = 0.0
    p["presence_penalty"][6] = 0.0
    w = W.Workload("topk", base.rows, base.vocab, "f32", base.logits, p, base.seeds, base.u,
                   base.hist_off, base.hist_ids, None, 5, True)
    g = run(sampler, w)
    compare(w, g, O.sample_batch(w, threads=8), "topk", expect_paths={5, 6})
    paths = g["diag"]["path"]
    assert (paths[[i for i, k in enumerate(ks) if k <= 64]] == 5).all(), paths.tolist()
    assert paths[ks.index(65)] == 6


def test_topk_merge_past_the_candidate_window(sampler):
    """Top-k rows whose slice lists leave more than 256 candidates under the
    merge's bound: slice 0 holds one large logit, every other slice 64 large
    ones, so the bound (the largest of the lists' m-th keys) falls in slice
    0's noise and admits every other list whole. Those rows are ranked by the
    count over the lists; top_k 5 stays under the bound's window."""
    g = np.random.default_rng(20261431)
    V, rows = 128256, 6
    S = -(-V // 8192)
    L = -(-V // S)
    logits = g.standard_normal((rows, V)).astype(np.float32)
    for r in range(rows):
        logits[r, int(g.integers(0, L))] = 100.0
        for s in range(1, S):
            lo, hi = s * L, min(V, (s + 1) * L)
            pos = g.choice(hi - lo, 64, replace=False) + lo
            logits[r, pos] = (60.0 + 39.0 * g.random(64)).astype(np.float32)
    p = W.default_params(rows)
    ks = [64, 64, 40, 17, 5, 64]
    for r in range(rows):
        p["top_k"][r] = ks[r]
        p["temperature"][r] = [1.0, 30.0, 10.0][r % 3]
        p["top_p"][r] = [1.0, 0.9][r % 2]
        p["min_p"][r] = 0.0
    seeds = np.array([W.row_seed(20261431, r) for r in range(rows)], dtype=np.uint64)
    hoff = np.zeros(rows + 1, dtype=np.uint32)
    w = W.Workload("topk-many", rows, V, "f32", logits, p, seeds, W.uniforms(seeds), hoff,
                   np.zeros(0, dtype=np.int32), None, 3, True)
    out = run(sampler, w)
    compare(w, out, O.sample_batch(w, threads=8), "topk-many", expect_paths={5})


def test_nucleus_rows(sampler):
    """Stochastic rows without top_k run on the sliced nucleus path (path 6):
    top-p only, constrained rows (with and without min-p), plain temperature,
    penalties, extreme temperatures, a mask that allows nothing, f32 and bf16.
    Rows whose decisive group is too large finish on the exact path (4)."""
    for name, rows in (("c3", 40), ("c4", 24)):
        w = W.make(name, rows=rows, set_index=21)
        g = run(sampler, w)
        compare(w, g, O.sample_batch(w, threads=16), f"nucleus-{name}", expect_paths={4, 6})
        assert (g["diag"]["path"] == 6).mean() >= 0.9, g["diag"]["path"].tolist()

    base = W.make("c2", rows=16, set_index=23)
    V = base.vocab
    p = base.params.copy()
    p["top_k"] = 0
    p["min_p"] = 0.0
    cfg = [  # temperature, top_p, min_p, penalties on, masked (fraction allowed)
        (0.7, 0.9, 0.0, True, None), (1.0, 1.0, 0.0, True, None), (1.5, 0.5, 0.0, False, None),
        (0.05, 0.9, 0.0, False, None), (4.0, 0.99, 0.0, True, None), (1.0, 0.1, 0.0, False, None),
        (0.7, 0.9, 0.05, True, 0.3), (1.0, 1.0, 0.2, False, 0.02), (0.8, 0.95, 0.0, True, 0.0),
        (1.0, 0.95, 0.0, False, 1e-4), (1.2, 1.0, 0.0, False, 0.5), (0.9, 0.8, 0.01, True, 0.1),
        (2.0, 0.999, 0.0, False, None), (0.3, 0.7, 0.0, True, 0.05), (1.0, 0.9, 0.0, True, None),
        (0.6, 1.0, 0.3, True, 1.0),
    ]
    bits = np.ones((base.rows, V), dtype=bool)
    has = np.zeros(base.rows, dtype=bool)
    rng = np.random.default_rng(31)
    for r, (t, tp, mp, pen, frac) in enumerate(cfg):
        p["temperature"][r], p["top_p"][r], p["min_p"][r] = t, tp, mp
        if not pen:
            p["repeat_penalty"][r], p["frequency_penalty"][r], p["presence_penalty"][r] = 1.0, 0.0, 0.0
        if frac is not None:
            has[r] = True
            bits[r] = rng.random(V) < frac
    masked = W.Workload("nucleus-mix", base.rows, V, "f32", base.logits, p, base.seeds, base.u,
                        base.hist_off, base.hist_ids, W.pack_mask(bits), 5, True)
    hm = has.astype(np.uint8)
    g = run(sampler, masked, has_mask=sampler.torch.from_numpy(hm).cuda())
    compare(masked, g, O.sample_batch(masked, threads=16, has_mask=hm), "nucleus-mix", expect_paths={4, 6})
    assert (g["diag"]["path"] == 6).sum() >= 12, g["diag"]["path"].tolist()

    bf = W.make("c3", rows=8, set_index=25)
    b16 = W.bf16_rne(bf.logits)
    wb = W.Workload("nucleus-bf16", bf.rows, bf.vocab, "bf16", b16, bf.params, bf.seeds, bf.u,
                    n_top=2, want_logprobs=True)
    w32 = W.Workload("nucleus-bf16-as-f32", bf.rows, bf.vocab, "f32", W.bf16_to_f32(b16), bf.params,
                     bf.seeds, bf.u, n_top=2, want_logprobs=True)
    compare(w32, run(sampler, wb), O.sample_batch(w32, threads=16), "nucleus-bf16", expect_paths={4, 6})


def test_nucleus_histogram_extremes(sampler):
    """Nucleus rows at the limits of the histogram pass's packed bin words
    (count in bits 50-63, mass as an integer below 2^48.1 per slice): every
    candidate of a full 8192-logit slice in one bin (all logits equal, also
    masked and bf16; one such slice in a row of distinct values, its bin
    carrying 4% of the mass below the decisions), two values only, the widest bin scale (candidates within
    1e-3 of the max: sx = 2^19), the narrowest (a candidate 1000 below the max:
    x_lo floored at -128, sx = 4, off-grid candidates) and a temperature that
    spreads the row over all 512 bins. The tied rows' decisive groups exceed
    what the finalize ranks, so they finish on the exact path after the
    histogram pass has binned them."""
    V = 3 * 8192 + 5
    rows = 8
    g = np.random.default_rng(47)
    logits = np.empty((rows, V), dtype=np.float32)
    logits[0] = 0.25                                     # all equal
    logits[1] = np.where(g.random(V) < 0.5, 0.0, -1.0)   # two values
    logits[2] = g.random(V) * 1e-3                       # within 1e-3: sx = 2^19
    logits[3] = g.standard_normal(V)
    logits[3, g.integers(0, V, 7)] = -1000.0             # x_lo floored: sx = 4, off-grid candidates
    logits[4] = g.standard_normal(V) * 8.0               # wide spread at T = 0.25
    logits[5] = 0.25                                     # all equal, masked to two full slices
    logits[6] = g.standard_normal(V)
    logits[7] = g.standard_normal(V)                     # one full slice in one bin, 4% of the mass,
    logits[7, 8192:2 * 8192] = -2.0                      # below the decisions
    p = W.default_params(rows)
    p["temperature"][:] = [1.0, 1.0, 0.8, 1.2, 0.25, 1.0, 1.5, 0.7]
    p["top_p"][:] = [0.9, 0.7, 0.95, 0.5, 0.99, 0.6, 0.98, 0.95]
    bits = np.ones((rows, V), dtype=bool)
    bits[5, 2 * 8192:] = False
    has = np.zeros(rows, dtype=np.uint8)
    has[5] = 1
    seeds = np.array([W.row_seed(4747, r) for r in range(rows)], dtype=np.uint64)
    u = W.uniforms(seeds)
    w = W.Workload("nucleus-extremes", rows, V, "f32", logits, p, seeds, u, mask=W.pack_mask(bits),
                   n_top=2, want_logprobs=True)
    gg = run(sampler, w, has_mask=sampler.torch.from_numpy(has).cuda())
    compare(w, gg, O.sample_batch(w, threads=16, has_mask=has), "nucleus-extremes", expect_paths={4, 6})
    # (rows of equal logits have decisive groups far above 256 candidates and
    # finish on the exact path; the others decide on the nucleus path)
    assert (gg["diag"]["path"][[2, 3, 4, 6, 7]] == 6).all(), gg["diag"]["path"].tolist()
    b16 = W.bf16_rne(logits)
    wb = W.Workload("nucleus-extremes-bf16", rows, V, "bf16", b16, p, seeds, u, mask=W.pack_mask(bits),
                    n_top=2, want_logprobs=True)
    w32 = W.Workload("nucleus-extremes-bf16-as-f32", rows, V, "f32", W.bf16_to_f32(b16), p, seeds, u,
                     mask=W.pack_mask(bits), n_top=2, want_logprobs=True)
    compare(w32, run(sampler, wb, has_mask=sampler.torch.from_numpy(has).cuda()),
            O.sample_batch(w32, threads=16, has_mask=has), "nucleus-extremes-bf16", expect_paths={4, 6})


def _all_paths_workload(V, seed, dtype="f32"):
    """Nine rows over vocab V, one per row path and filter mix: greedy (also
    masked), min-p window, sliced top-k, nucleus (top-p, masked, plain
    temperature, masked top-k 100 with top-p and min-p) and the exact path
    (a penalty window of 5000 ids), with penalties on about half."""
    g = np.random.default_rng(seed)
    cfg = [  # temperature, top_k, top_p, min_p, penalties, masked fraction
        (0.0, 0, 1.0, 0.0, True, None), (0.7, 0, 0.9, 0.05, True, None), (0.8, 20, 0.95, 0.0, False, None),
        (1.5, 0, 0.98, 0.0, False, None), (1.0, 0, 0.95, 0.0, True, 0.05), (1.0, 0, 1.0, 0.0, False, None),
        (0.9, 100, 1.0, 0.0, True, None), (0.0, 0, 1.0, 0.0, False, 0.3), (0.9, 100, 0.9, 0.02, True, 0.2),
    ]
    rows = len(cfg)
    logits = (g.standard_normal((rows, V)) * 2.5).astype(np.float32)
    p = W.default_params(rows)
    bits = np.ones((rows, V), dtype=bool)
    has = np.zeros(rows, dtype=np.uint8)
    for r, (t, k, tp, mp, pen, frac) in enumerate(cfg):
        p["temperature"][r], p["top_k"][r], p["top_p"][r], p["min_p"][r] = t, k, tp, mp
        if pen:
            p["repeat_penalty"][r], p["frequency_penalty"][r], p["presence_penalty"][r] = 1.2, 0.3, 0.2
            p["repeat_last_n"][r] = 5000 if r == 6 else 256
        if frac is not None:
            has[r] = 1
            bits[r] = g.random(V) < frac
    hlen = 300
    hist = g.integers(0, V, size=(rows, hlen)).astype(np.int32)
    seeds = np.array([W.row_seed(seed, r) for r in range(rows)], dtype=np.uint64)
    u = W.uniforms(seeds)
    w32 = W.Workload(f"paths-{V}", rows, V, "f32", logits, p, seeds, u,
                     np.arange(rows + 1, dtype=np.uint32) * hlen, hist.reshape(-1), W.pack_mask(bits), 3, True)
    if dtype == "f32":
        return w32, w32, has
    b16 = W.bf16_rne(logits)
    wb = W.Workload(f"paths-{V}-bf16", rows, V, "bf16", b16, p, seeds, u, w32.hist_off, w32.hist_ids,
                    w32.mask, 3, True)
    w32 = W.Workload(f"paths-{V}-bf16-as-f32", rows, V, "f32", W.bf16_to_f32(b16), p, seeds, u,
                     w32.hist_off, w32.hist_ids, w32.mask, 3, True)
    return wb, w32, has


@pytest.mark.parametrize("V,dtype", [(4096, "f32"), (4097, "bf16"), (8192, "f32"), (8193, "f32"),
                                     (16385, "bf16"), (262144, "f32"), (262144, "bf16")])
def test_every_path_at_slice_boundaries_and_max_vocab(sampler, V, dtype):
    """Every row path at vocabularies that end a slice exactly (8192-logit
    slices of the sliced path and of the nucleus passes), one past it, half a
    slice, and the maximum vocabulary (32 slices)."""
    wg, w32, has = _all_paths_workload(V, 20261300 + V, dtype)
    say("paths", V, dtype)
    g = run(sampler, wg, has_mask=sampler.torch.from_numpy(has).cuda())
    compare(w32, g, O.sample_batch(w32, threads=16, has_mask=has), f"paths-{V}-{dtype}",
            expect_paths={1, 2, 3, 4, 5, 6})
    paths = g["diag"]["path"].tolist()
    assert paths[0] == 1 and paths[2] == 5 and paths[6] == 4 and paths[4] == 6 and paths[8] == 6, paths
    # bf16 rows of the largest vocabulary hold so many equal logits that a
    # decisive sub-bin can exceed one wave's ranking (the exact path then)
    assert paths[3] in ((4, 6) if dtype == "bf16" and V > 131072 else (6,)), paths


def _random_batch(seed):
    """A seeded random batch: vocab, dtype, per-row parameters, history,
    masks and logprob counts drawn so that every row path and filter mix
    appears across seeds."""
    g = np.random.default_rng([20261400, seed])
    V = int(g.choice([1, 7, 64, 1000, 8191, 8192, 8193, 20000, 65537, 128256]))
    rows = int(g.integers(1, 13))
    scale = float(g.choice([0.3, 1.0, 3.0, 8.0]))
    logits = (g.standard_normal((rows, V)) * scale).astype(np.float32)
    if g.random() < 0.2:   # integer logits: exact ties
        logits = np.round(logits).astype(np.float32)
    p = W.default_params(rows)
    for r in range(rows):
        p["temperature"][r] = g.choice([0.0, 0.05, 0.5, 0.8, 1.0, 1.5, 3.0])
        p["top_k"][r] = g.choice([0, 0, 1, 5, 40, 64, 65, 200, 5000])
        p["top_p"][r] = g.choice([1.0, 1.0, 0.5, 0.9, 0.95, 0.99])
        p["min_p"][r] = g.choice([0.0, 0.0, 0.01, 0.05, 0.3])
        if g.random() < 0.5:
            p["repeat_penalty"][r] = g.choice([0.8, 1.1, 1.5])
            p["frequency_penalty"][r] = g.choice([0.0, 0.5, -0.3])
            p["presence_penalty"][r] = g.choice([0.0, 0.3])
            p["repeat_last_n"][r] = g.choice([0, 16, 64, 2048])
    hlen = int(g.integers(0, 200))
    hist = g.integers(-3, V + 3, size=(rows, hlen)).astype(np.int32)
    mask, has = None, None
    if g.random() < 0.4:
        bits = g.random((rows, V)) < g.choice([0.0, 0.001, 0.05, 0.5, 1.0])
        mask = W.pack_mask(bits)
        has = (g.random(rows) < 0.7).astype(np.uint8)
    n_top = int(g.choice([0, 1, 5, 20])) if g.random() < 0.6 else 0
    seeds = np.array([W.row_seed(20261400 + seed, r) for r in range(rows)], dtype=np.uint64)
    u = W.uniforms(seeds)
    hoff = np.arange(rows + 1, dtype=np.uint32) * hlen
    w32 = W.Workload(f"rand{seed}", rows, V, "f32", logits, p, seeds, u, hoff, hist.reshape(-1), mask,
                     min(n_top, V), n_top > 0)
    if g.random() < 0.3:   # bf16 logits, compared as their f32 values
        b16 = W.bf16_rne(logits)
        wg = W.Workload(f"rand{seed}-bf16", rows, V, "bf16", b16, p, seeds, u, hoff, hist.reshape(-1), mask,
                        min(n_top, V), n_top > 0)
        w32 = W.Workload(f"rand{seed}-bf16-as-f32", rows, V, "f32", W.bf16_to_f32(b16), p, seeds, u, hoff,
                         hist.reshape(-1), mask, min(n_top, V), n_top > 0)
        return wg, w32, has
    return w32, w32, has


def test_random_batches(sampler):
    """100 seeded random batches across every path, against the oracle."""
    seen = set()
    for seed in range(100):
        wg, w32, has = _random_batch(seed)
        say("random", seed, wg.name, wg.rows, wg.vocab)
        kw = {} if has is None else {"has_mask": sampler.torch.from_numpy(has).cuda()}
        g = run(sampler, wg, **kw)
        compare(w32, g, O.sample_batch(w32, threads=16, has_mask=has), f"random-{seed}")
        seen.update(np.unique(g["diag"]["path"]).tolist())
    assert {1, 2, 4, 5, 6} <= seen, seen


def slice_geometry(V):
    """The sliced path's cut of a row: S slices of L logits (the last one
    shorter), L a multiple of 8 and at most 8192 (lcs_api.hip)."""
    S = -(-V // 8192)
    L = (-(-V // S) + 7) // 8 * 8
    return S, L


def test_window_rows_with_many_entries_per_slice(sampler):
    """Min-p window rows whose row window is planted in chosen slices: up to 4
    qualifying entries per slice (row_fin's first fetch round), more (further
    rounds, up to a slice's 64-entry record), a slice past its record (exact
    path) and a row window past 256 entries (exact path), including the short
    last slice."""
    base = W.make("c2", rows=12, set_index=29)
    V = base.vocab
    S, L = slice_geometry(V)
    rng = np.random.default_rng(2029)
    logits = (rng.standard_normal((base.rows, V)) - 20.0).astype(np.float32)
    plant = [  # (slice, entries) per row
        [(0, 3), (7, 2)], [(0, 10)], [(0, 16)], [(0, 17)], [(2, 40), (9, 20)], [(S - 1, 30)],
        [(0, 64)], [(0, 70)], [(s, 17) for s in range(S)], [(s, 6) for s in range(S)] + [(3, 8)],
        [(4, 5), (5, 5), (6, 5)], [(1, 33), (14, 1)],
    ]
    for r, spots in enumerate(plant):
        for s, n in spots:
            lo, hi = s * L, min(V, (s + 1) * L)
            idx = rng.choice(np.arange(lo, hi), size=n, replace=False)
            logits[r, idx] = rng.uniform(9.0, 10.0, size=n).astype(np.float32)
    p = base.params.copy()
    p["temperature"], p["min_p"], p["top_p"], p["top_k"] = 1.0, 0.05, 0.9, 0
    for r in range(0, base.rows, 2):
        p["repeat_penalty"][r], p["frequency_penalty"][r], p["presence_penalty"][r] = 1.0, 0.0, 0.0
    w = W.Workload("window-spots", base.rows, V, "f32", logits, p, base.seeds, base.u,
                   base.hist_off, base.hist_ids, None, 5, True)
    g = run(sampler, w)
    compare(w, g, O.sample_batch(w, threads=8), "window-spots", expect_paths={2, 3, 4})
    paths = g["diag"]["path"]
    window_rows = [0, 1, 2, 3, 4, 5, 6, 9, 10, 11]
    assert np.isin(paths[window_rows], [2, 3]).all(), paths.tolist()
    assert (paths[[7, 8]] == 4).all(), paths.tolist()


def test_wide_min_p_windows(sampler):
    """C2-shaped rows whose min-p windows hold thousands of ids (far past a
    slice's 64-entry record), so row_fin resolves them on the exact path: with
    and without penalties, top-p on and off, f32 and bf16."""
    base = W.make("c2", rows=16, set_index=31)
    rng = np.random.default_rng(2031)
    lg = (base.logits / 3.0).astype(np.float32)       # N(0, 1)
    p = base.params.copy()
    p["temperature"][:8], p["min_p"][:8] = 1.5, 0.01
    p["temperature"][8:], p["min_p"][8:] = 1.0, 0.05
    p["top_p"][::3] = 1.0
    for r in range(1, base.rows, 4):
        p["repeat_penalty"][r], p["frequency_penalty"][r], p["presence_penalty"][r] = 1.0, 0.0, 0.0
    lg[5, rng.choice(base.vocab, 4000, replace=False)] += 2.0   # a denser head
    w = W.Workload("wide-min-p", base.rows, base.vocab, "f32", lg, p, base.seeds, base.u,
                   base.hist_off, base.hist_ids, None, 5, True)
    g = run(sampler, w)
    compare(w, g, O.sample_batch(w, threads=8), "wide-min-p", expect_paths={3, 4})
    assert (g["diag"]["keep"] > 64).all(), g["diag"]["keep"].tolist()
    assert (g["diag"]["path"] == 4).sum() >= 14, g["diag"]["path"].tolist()
    b16 = W.bf16_rne(lg)
    wb = W.Workload("wide-min-p-bf16", w.rows, w.vocab, "bf16", b16, p, w.seeds, w.u,
                    w.hist_off, w.hist_ids, None, 5, True)
    w32 = W.Workload("wide-min-p-bf16-as-f32", w.rows, w.vocab, "f32", W.bf16_to_f32(b16), p, w.seeds, w.u,
                     w.hist_off, w.hist_ids, None, 5, True)
    compare(w32, run(sampler, wb), O.sample_batch(w32, threads=8), "wide-min-p-bf16", expect_paths={3, 4})


def test_top_n_with_clustered_maxima(sampler):
    """Top-n logprobs where many logits near the top share the upper 16 bits
    of their sort keys (the slice's candidate bound is cut to 16 bits): 40
    and 100 such values in one slice, 200 in one slice (past the slice's
    candidate capacity: exact path), spread over slices, and top-20."""
    base = W.make("c2", rows=8, set_index=31)
    V = base.vocab
    S, L = slice_geometry(V)
    rng = np.random.default_rng(2031)
    logits = (rng.standard_normal((base.rows, V)) * 3.0).astype(np.float32)
    f32 = lambda x: np.asarray(x, dtype=np.float32)
    spots = [(0, 40), (3, 100), (5, 200), (None, 60), (15, 40), (0, 7), (8, 128), (None, 300)]
    for r, (s, n) in enumerate(spots):
        # distinct floats in [20, 20.07): one 16-bit key prefix spans 2^16 ulps
        vals = f32(20.0) + f32(np.arange(n) * 2 ** -16 * 3 + rng.integers(0, 2, n) * 2 ** -20)
        if s is None:
            idx = rng.choice(V, size=n, replace=False)
        else:
            lo, hi = s * L, min(V, (s + 1) * L)
            idx = rng.choice(np.arange(lo, hi), size=n, replace=False)
        logits[r, idx] = vals
    for n_top in (5, 20):
        w = W.Workload(f"clustered-top{n_top}", base.rows, V, "f32", logits, base.params, base.seeds, base.u,
                       base.hist_off, base.hist_ids, None, n_top, True)
        g = run(sampler, w)
        compare(w, g, O.sample_batch(w, threads=8), w.name, expect_paths={2, 3, 4})
