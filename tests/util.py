"""Comparison helpers shared by the parity tests."""
from __future__ import annotations

import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
# Documented near-tie band: a row whose reference decision (top-p cumulative,
# min-p ratio or draw residual) is within this relative distance of its
# threshold may legitimately differ (the reference sums sequentially in
# double; the GPU sums exactly in fixed point). north_star allows 1e-6.
NEAR_TIE = 1e-9
LOGPROB_TOL = 1e-5


def load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def near_tie_rows(diag) -> np.ndarray:
    """Rows whose reference decision lies within NEAR_TIE of its threshold."""
    m = np.minimum(np.minimum(diag["margin_p"], diag["margin_m"]), diag["margin_r"])
    return m < NEAR_TIE


def excluded_rows(diag) -> np.ndarray:
    """Rows whose sampled id the reference leaves tie- or near-tie-dependent."""
    return (diag["tie_flags"] != 0) | near_tie_rows(diag)


def row_logits_f32(w, r) -> np.ndarray:
    """Row r of a workload's logits as float32 (bf16 rows widened exactly)."""
    if w.dtype == "bf16":
        from locus_amd import workloads as W
        return W.bf16_to_f32(np.asarray(w.logits[r]))
    return np.asarray(w.logits[r], dtype=np.float32)


def penalized_value(w, r, t) -> np.float32:
    """Token t's logit in row r after apply_penalties (sampling.cpp:16-41):
    float32 arithmetic, one rounding per operation, no fused multiply-add."""
    f32 = np.float32
    l = row_logits_f32(w, r)[t]
    p = w.params[r]
    active = not (p["repeat_penalty"] == 1.0 and p["frequency_penalty"] == 0.0 and p["presence_penalty"] == 0.0)
    if w.hist_off is None or not active:
        return l
    h = np.asarray(w.hist_ids[int(w.hist_off[r]):int(w.hist_off[r + 1])], dtype=np.int64)
    win = h[max(0, len(h) - int(p["repeat_last_n"])):]
    c = int((win == t).sum())
    if c == 0:
        return l
    rp = f32(p["repeat_penalty"])
    if rp != f32(1.0):
        l = f32(l / rp) if l > f32(0.0) else f32(l * rp)
    sub = f32(f32(f32(p["frequency_penalty"]) * f32(c)) + f32(p["presence_penalty"]))
    return f32(l - sub)
