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


def excluded_rows(diag) -> np.ndarray:
    """Rows whose sampled id the reference leaves tie- or near-tie-dependent."""
    m = np.minimum(np.minimum(diag["margin_p"], diag["margin_m"]), diag["margin_r"])
    return (diag["tie_flags"] != 0) | (m < NEAR_TIE)
