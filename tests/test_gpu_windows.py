"""Device-resident penalty windows (lcs_windows_reserve / lcs_windows_load and
the lcs_batch win_* fields) against the CPU oracle.

Each test drives a batch through several engine steps (engine.cpp:423-450:
sample, then append the sampled id to the request's history): the device
windows receive one appended id per step, and the oracle receives the whole
history of that step as hist_off / hist_ids. Ids, survivor counts and
logprobs must match as in the other parity tests (the same near-tie rule)."""
import dataclasses

import numpy as np
import pytest

from locus_amd import workloads as W
from oracle import pyoracle as O
from tests.test_gpu_sampling import compare, say

pytestmark = pytest.mark.gpu

LCS_STATUS_WINDOW = 4


@pytest.fixture(scope="module")
def sampler():
    from locus_amd.sampler import Sampler
    s = Sampler(device=0, max_rows=128, max_vocab=262144, max_hist=4096, max_top=20)
    s.windows_reserve(128, 4096)
    yield s
    s.close()


def with_history(w, hist, params=None):
    """w with per-row histories `hist` (list of int32 arrays) as CSR."""
    off = np.zeros(w.rows + 1, dtype=np.uint32)
    off[1:] = np.cumsum([len(h) for h in hist])
    ids = np.concatenate(hist).astype(np.int32) if off[-1] else np.zeros(0, dtype=np.int32)
    return dataclasses.replace(w, hist_off=off, hist_ids=ids, params=w.params if params is None else params)


def run_steps(sampler, base, hists, window, steps, dtype="f32", push_every=None, label="win"):
    """Loads slot r with hists[r][:-1], then for each step samples fresh
    logits with the slot (the step's appended id: hists[r][-1] at step 0, the
    previous step's sampled id after that) and checks against the oracle."""
    torch = sampler.torch
    dev = torch.device("cuda", 0)
    rows, V = base.rows, base.vocab
    hist = [np.asarray(h, dtype=np.int32) for h in hists]
    for r in range(rows):
        pre = hist[r][:-1]
        sampler.windows_load(r, torch.from_numpy(pre.copy()).to(dev) if len(pre) else None, window, V)
    pushes = np.array([h[-1] for h in hist], dtype=np.int32)
    lens = np.array([len(h) for h in hist], dtype=np.uint32)
    slots = torch.arange(rows, dtype=torch.int32, device=dev)
    for s in range(steps):
        w = W.make("c2", rows=rows, set_index=40 + s) if base.name == "c2" else base
        if dtype == "bf16":
            w = dataclasses.replace(w, dtype="bf16", logits=W.bf16_rne(w.logits))
        if w.vocab != V:
            w = dataclasses.replace(w, vocab=V, logits=w.logits[:, :V].copy())
        w = dataclasses.replace(w, params=base.params, n_top=base.n_top, want_logprobs=base.want_logprobs,
                                u=W.uniforms(w.seeds))
        wo = with_history(w, hist)
        d = sampler.upload(wo)
        out = sampler.alloc_out(rows, wo.n_top, wo.want_logprobs)
        win = {"slot": slots, "push": torch.from_numpy(pushes.copy()).to(dev),
               "len": torch.from_numpy(lens.view(np.int32).copy()).to(dev)}
        sampler.sample_dev(d, out, win=win)
        torch.cuda.synchronize()
        g = sampler.fetch(out, wo.n_top)
        assert sampler.status() == 0
        say(label, "step", s, "hist", int(lens.min()), "..", int(lens.max()))
        w32 = dataclasses.replace(wo, dtype="f32", logits=W.bf16_to_f32(wo.logits)) if dtype == "bf16" else wo
        compare(w32, g, O.sample_batch(w32, threads=16), f"{label}-step{s}", expect_paths={2, 3, 4})
        # the engine appends the sampled id; some steps append nothing
        nxt = g["ids"].astype(np.int32)
        grow = np.ones(rows, dtype=bool) if push_every is None else (np.arange(rows) + s) % push_every != 0
        for r in range(rows):
            if grow[r]:
                hist[r] = np.append(hist[r], nxt[r])
        pushes = np.where(grow, nxt, pushes).astype(np.int32)
        lens = np.array([len(h) for h in hist], dtype=np.uint32)
    return hist


def test_c2_windows_over_engine_steps(sampler):
    """C2 shape: 2048-id Zipf windows (repeat_last_n 2048), full from the
    start, so every step's append pushes an id out."""
    w = W.make("c2", rows=64)
    hists = [w.hist_ids[w.hist_off[r]:w.hist_off[r + 1]] for r in range(w.rows)]
    hists = [np.append(h, h[r % len(h)]) for r, h in enumerate(hists)]
    run_steps(sampler, w, hists, 2048, steps=4, label="win-c2")


def test_windows_short_and_edge_histories(sampler):
    """Short windows filling up and sliding, ids outside [0, V) (counted by
    nobody but still taking a window place), repeated ids, empty histories,
    rows without penalties, and steps that append nothing."""
    rng = np.random.default_rng(77)
    base = W.make("c2", rows=24, set_index=9)
    p = base.params.copy()
    p["repeat_last_n"] = 32
    for r in range(0, base.rows, 6):
        p["repeat_penalty"][r], p["frequency_penalty"][r], p["presence_penalty"][r] = 1.0, 0.0, 0.0
    base = dataclasses.replace(base, params=p)
    V = base.vocab
    hists = []
    for r in range(base.rows):
        n = [1, 5, 31, 32, 33, 60][r % 6]
        h = rng.integers(0, V, size=n).astype(np.int64)
        if r % 4 == 1:
            h[::3] = rng.choice([-1, -7, V, V + 5], size=len(h[::3]))
        if r % 4 == 2:
            h[:] = rng.choice(rng.integers(0, V, size=3), size=n)   # a few ids, many times
        hists.append(h.astype(np.int32))
    run_steps(sampler, base, hists, 32, steps=5, push_every=3, label="win-edge")


@pytest.mark.parametrize("dtype,V", [("bf16", 128256), ("f32", 151936)])
def test_windows_dtype_and_large_vocab(sampler, dtype, V):
    """bf16 logits (two quads per 16-byte group), and the largest vocabulary
    of the configurations (19 slices)."""
    base = W.make("c2", rows=16, set_index=11)
    if V != base.vocab:
        rng = np.random.default_rng(V)
        lg = (rng.standard_normal((base.rows, V)) * 3.0).astype(np.float32)
        base = dataclasses.replace(base, vocab=V, logits=lg)
    rng = np.random.default_rng(5)
    hists = [rng.integers(0, V, size=300).astype(np.int32) for _ in range(base.rows)]
    p = base.params.copy()
    p["repeat_last_n"] = 256
    base = dataclasses.replace(base, params=p, name="custom")
    torch = sampler.torch
    dev = torch.device("cuda", 0)
    hist = [h.copy() for h in hists]
    for r in range(base.rows):
        sampler.windows_load(r, torch.from_numpy(hist[r][:-1].copy()).to(dev), 256, V)
    pushes = np.array([h[-1] for h in hist], dtype=np.int32)
    for s in range(3):
        g_rng = np.random.default_rng(100 + s)
        lg = (g_rng.standard_normal((base.rows, V)) * 3.0).astype(np.float32)
        w = dataclasses.replace(base, logits=W.bf16_rne(lg) if dtype == "bf16" else lg, dtype=dtype)
        wo = with_history(w, hist)
        d = sampler.upload(wo)
        out = sampler.alloc_out(base.rows, wo.n_top, wo.want_logprobs)
        lens = np.array([len(h) for h in hist], dtype=np.int32)
        win = {"slot": torch.arange(base.rows, dtype=torch.int32, device=dev),
               "push": torch.from_numpy(pushes.copy()).to(dev), "len": torch.from_numpy(lens).to(dev)}
        sampler.sample_dev(d, out, win=win)
        torch.cuda.synchronize()
        g = sampler.fetch(out, wo.n_top)
        assert sampler.status() == 0
        # the oracle takes the bf16 logits' float32 values
        w32 = dataclasses.replace(wo, dtype="f32", logits=W.bf16_to_f32(wo.logits)) if dtype == "bf16" else wo
        compare(w32, g, O.sample_batch(w32, threads=16), f"win-{dtype}-{V}-step{s}", expect_paths={2, 3, 4})
        nxt = g["ids"].astype(np.int32)
        hist = [np.append(hist[r], nxt[r]) for r in range(base.rows)]
        pushes = nxt


def test_window_mismatch_reports_the_row(sampler):
    """A history length that skips ahead, or a window that is not the row's
    repeat_last_n: id -1 and LCS_STATUS_WINDOW for that row only, and the
    slot keeps its state (a correct call afterwards matches the oracle)."""
    torch = sampler.torch
    dev = torch.device("cuda", 0)
    base = W.make("c2", rows=8, set_index=13)
    p = base.params.copy()
    p["repeat_last_n"] = 64
    base = dataclasses.replace(base, params=p)
    rng = np.random.default_rng(3)
    hist = [rng.integers(0, base.vocab, size=80).astype(np.int32) for _ in range(base.rows)]
    for r in range(base.rows):
        sampler.windows_load(r, torch.from_numpy(hist[r][:-1].copy()).to(dev), 64 if r != 5 else 32, base.vocab)
    lens = np.array([len(h) for h in hist], dtype=np.int32)
    bad_len = lens.copy()
    bad_len[2] += 1
    pushes = np.array([h[-1] for h in hist], dtype=np.int32)
    wo = with_history(base, hist)
    d = sampler.upload(wo)
    out = sampler.alloc_out(base.rows, wo.n_top, wo.want_logprobs)
    win = {"slot": torch.arange(base.rows, dtype=torch.int32, device=dev),
           "push": torch.from_numpy(pushes).to(dev), "len": torch.from_numpy(bad_len).to(dev)}
    sampler.sample_dev(d, out, win=win)
    torch.cuda.synchronize()
    g = sampler.fetch(out, wo.n_top)
    assert sampler.status() == LCS_STATUS_WINDOW
    assert g["ids"][2] == -1 and g["ids"][5] == -1
    o = O.sample_batch(wo, threads=16)
    good = np.array([r not in (2, 5) for r in range(base.rows)])
    assert np.array_equal(g["ids"][good], o.ids[good])
    # row 2 is unchanged: the correct length now matches the oracle
    sampler.windows_load(5, torch.from_numpy(hist[5][:-1].copy()).to(dev), 64, base.vocab)
    win["len"] = torch.from_numpy(lens).to(dev)
    out = sampler.alloc_out(base.rows, wo.n_top, wo.want_logprobs)
    sampler.sample_dev(d, out, win=win)
    torch.cuda.synchronize()
    g = sampler.fetch(out, wo.n_top)
    assert sampler.status() == 0
    compare(wo, g, o, "win-after-mismatch")


def test_windows_of_rows_without_penalties(sampler):
    """Slots keep their windows up to date for rows whose penalties are off
    (the append still happens): turned on again later, they penalise the
    right ids."""
    torch = sampler.torch
    dev = torch.device("cuda", 0)
    base = W.make("c2", rows=8, set_index=17)
    rng = np.random.default_rng(17)
    hist = [rng.integers(0, base.vocab, size=40).astype(np.int32) for _ in range(base.rows)]
    for r in range(base.rows):
        sampler.windows_load(r, torch.from_numpy(hist[r][:-1].copy()).to(dev), 16, base.vocab)
    on = base.params.copy()
    on["repeat_last_n"] = 16
    off = on.copy()
    off["repeat_penalty"], off["frequency_penalty"], off["presence_penalty"] = 1.0, 0.0, 0.0
    pushes = np.array([h[-1] for h in hist], dtype=np.int32)
    for s, p in enumerate([off, off, on, on]):
        w = dataclasses.replace(W.make("c2", rows=8, set_index=60 + s), params=p)
        wo = with_history(w, hist)
        d = sampler.upload(wo)
        out = sampler.alloc_out(w.rows, w.n_top, w.want_logprobs)
        lens = np.array([len(h) for h in hist], dtype=np.int32)
        win = {"slot": torch.arange(w.rows, dtype=torch.int32, device=dev),
               "push": torch.from_numpy(pushes.copy()).to(dev), "len": torch.from_numpy(lens).to(dev)}
        sampler.sample_dev(d, out, win=win)
        torch.cuda.synchronize()
        g = sampler.fetch(out, w.n_top)
        assert sampler.status() == 0
        compare(wo, g, O.sample_batch(wo, threads=16), f"win-off-on-step{s}")
        hist = [np.append(hist[r], g["ids"][r]) for r in range(w.rows)]
        pushes = g["ids"].astype(np.int32)
