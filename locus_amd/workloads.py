"""Deterministic synthetic inputs for the five benchmark configurations.

Every buffer is built from numpy ``Generator`` streams seeded per
(configuration, input set, row), so any prefix of rows is identical to the
same rows of the full-size batch, and the same image produces the same bytes
on every machine (a checksum travels with each golden fixture).

Configurations (seed base ``S = 20261200 + n`` for configuration n):

* ``c1g`` / ``c1s`` - B=1, V=128256 f32 ~ N(0, 2^2) with 8 seeded ids given
  +12; greedy, then T=0.8 / top_k=40 / top_p=0.95.
* ``c2`` - B=64, V=128256 f32 ~ N(0, 3^2); 2048-id Zipf(1.1) history per row
  through a seeded permutation; repeat 1.1, frequency 0.5, presence 0.3,
  repeat_last_n 2048; T=0.7, min_p 0.05, top_p 0.9; top-5 logprobs.
* ``c2w`` - ``c2`` with N(0, 1) logits, T=1.5 and min_p 0.01: min-p windows
  of thousands of ids, past a slice's window record, so every row takes the
  exact path inside the row finalize (a stress case, not a BASELINE config).
* ``c3`` - B=256, V=151936 f32 ~ N(0, 1); T=1.5, top_p 0.98.
* ``c4`` - B=32, V=128256 f32 ~ N(0, 2.5^2); per-row allow mask of V/32
  words with log-uniform density in [5e-4, 0.3] built from runs of 1..64 ids;
  T=1.0, top_p 0.95; top-1 logprob.
* ``c5`` - 512 sequences x 8 rows, V=163840 bf16 (N(0, 2^2) rounded to
  nearest-even) with one dominant id per row set to bf16(rowmax + 6); a
  draft id per row (the dominant id with probability 0.75).

The per-row uniform ``u`` is the first ``generate_canonical<double, 53>``
draw of ``std::mt19937_64(seed)`` (libstdc++ random.tcc:3348-3380), the
stream the reference's per-request RNG produces (engine.cpp:41-43).
"""
from __future__ import annotations

import dataclasses
import hashlib
import math

import numpy as np

PARAMS_DTYPE = np.dtype([
    ("temperature", "<f4"), ("top_k", "<u4"), ("top_p", "<f4"), ("min_p", "<f4"),
    ("repeat_penalty", "<f4"), ("frequency_penalty", "<f4"),
    ("presence_penalty", "<f4"), ("repeat_last_n", "<u4"),
])

_M64 = (1 << 64) - 1


class MT19937_64:
    """std::mt19937_64 (C++ [rand.predef]); the 10000th output of a
    default-seeded engine is 9981545732273789042."""

    N, M = 312, 156

    def __init__(self, seed: int = 5489):
        mt = [0] * self.N
        mt[0] = seed & _M64
        for i in range(1, self.N):
            mt[i] = (6364136223846793005 * (mt[i - 1] ^ (mt[i - 1] >> 62)) + i) & _M64
        self.mt, self.i = mt, self.N

    def _twist(self):
        mt, N, M = self.mt, self.N, self.M
        upper, lower = 0xFFFFFFFF80000000, 0x7FFFFFFF
        for k in range(N):
            y = (mt[k] & upper) | (mt[(k + 1) % N] & lower)
            mt[k] = mt[(k + M) % N] ^ (y >> 1) ^ (0xB5026F5AA96619E9 if y & 1 else 0)
        self.i = 0

    def __call__(self) -> int:
        if self.i >= self.N:
            self._twist()
        y = self.mt[self.i]
        self.i += 1
        y ^= (y >> 29) & 0x5555555555555555
        y ^= (y << 17) & 0x71D67FFFEDA60000 & _M64
        y ^= (y << 37) & 0xFFF7EEE000000000 & _M64
        y ^= y >> 43
        return y & _M64

    def canonical(self) -> float:
        """generate_canonical<double, 53>: double(x) / 2^64, clamped below 1."""
        u = float(self() & _M64) / 18446744073709551616.0
        return u if u < 1.0 else math.nextafter(1.0, 0.0)


def row_seed(cfg_seed: int, row: int) -> int:
    return (cfg_seed * 1000003 + row) & _M64


def uniforms(seeds) -> np.ndarray:
    return np.array([MT19937_64(int(s)).canonical() for s in seeds], dtype=np.float64)


def bf16_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits (uint16), round to nearest even."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = (b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def default_params(n: int) -> np.ndarray:
    p = np.zeros(n, dtype=PARAMS_DTYPE)
    p["top_p"] = 1.0
    p["repeat_penalty"] = 1.0
    p["repeat_last_n"] = 64
    return p


def checksum(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        if a is None:
            h.update(b"none")
        else:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()[:16]


@dataclasses.dataclass
class Workload:
    name: str
    rows: int
    vocab: int
    dtype: str                      # "f32" or "bf16"
    logits: np.ndarray              # (rows, vocab) float32, or uint16 bf16 bits
    params: np.ndarray | None       # PARAMS_DTYPE (rows,), sampling configs
    seeds: np.ndarray | None        # uint64 per row
    u: np.ndarray | None            # float64 per row
    hist_off: np.ndarray | None = None   # uint32 (rows + 1)
    hist_ids: np.ndarray | None = None   # int32
    mask: np.ndarray | None = None       # uint32 (rows, ceil(V/32))
    n_top: int = 0
    want_logprobs: bool = False
    n_seq: int = 0                  # verify workloads
    rows_per_seq: int = 0
    draft: np.ndarray | None = None

    @property
    def mask_words(self) -> int:
        return (self.vocab + 31) // 32

    def input_checksum(self) -> str:
        return checksum(self.logits, self.params, self.hist_off, self.hist_ids,
                        self.mask, self.draft, self.u)

    def algorithmic_bytes(self) -> int:
        """Compulsory bytes per call: inputs read once, outputs written once."""
        s = 2 if self.dtype == "bf16" else 4
        b = s * self.vocab * self.rows
        if self.n_seq:
            return b + 4 * self.rows + 4 * self.rows + 4 * self.rows + 4 * self.n_seq
        if self.hist_ids is not None:
            b += 4 * len(self.hist_ids)   # history ids (the CSR offsets are not counted)
        if self.mask is not None:
            b += 4 * self.mask.size
        b += 32 * self.rows
        greedy = self.params["temperature"] <= 0
        b += 8 * int((~greedy).sum())
        b += 4 * self.rows  # ids
        if self.want_logprobs:
            b += 4 * self.rows + 8 * self.n_top * self.rows
        return b


CFG_SEED = {"c1": 20261201, "c2": 20261202, "c3": 20261203, "c4": 20261204, "c5": 20261205}
FULL_ROWS = {"c1g": 1, "c1s": 1, "c2": 64, "c3": 256, "c4": 32, "c5": 4096}
VOCAB = {"c1g": 128256, "c1s": 128256, "c2": 128256, "c3": 151936, "c4": 128256, "c5": 163840}


def _row_rng(cfg_seed: int, set_index: int, row: int) -> np.random.Generator:
    return np.random.default_rng([cfg_seed, set_index, row])


def _normal_rows(cfg_seed, set_index, rows, V, sigma):
    out = np.empty((rows, V), dtype=np.float32)
    for r in range(rows):
        g = _row_rng(cfg_seed, set_index, r)
        out[r] = g.standard_normal(V, dtype=np.float32) * np.float32(sigma)
    return out


def _seeds(cfg_seed, set_index, rows):
    base = (cfg_seed + 7919 * set_index) & _M64
    return np.array([row_seed(base, r) for r in range(rows)], dtype=np.uint64)


def make_c1(greedy: bool, set_index: int = 0) -> Workload:
    S, V = CFG_SEED["c1"], VOCAB["c1g"]
    g = _row_rng(S, set_index, 0)
    logits = (g.standard_normal(V, dtype=np.float32) * np.float32(2.0))[None, :].copy()
    spikes = g.choice(V, size=8, replace=False)
    logits[0, spikes] += np.float32(12.0)
    p = default_params(1)
    if not greedy:
        p["temperature"], p["top_k"], p["top_p"] = 0.8, 40, 0.95
    seeds = _seeds(S, set_index, 1)
    u = np.zeros(1) if greedy else uniforms(seeds)
    return Workload("c1g" if greedy else "c1s", 1, V, "f32", logits, p, seeds, u)


def _zipf_cdf(V: int, s: float = 1.1) -> np.ndarray:
    w = np.arange(1, V + 1, dtype=np.float64) ** (-s)
    c = np.cumsum(w)
    return c / c[-1]


def make_c2(rows: int | None = None, set_index: int = 0, hist_len: int = 2048) -> Workload:
    S, V = CFG_SEED["c2"], VOCAB["c2"]
    rows = FULL_ROWS["c2"] if rows is None else rows
    logits = _normal_rows(S, set_index, rows, V, 3.0)
    cdf = _zipf_cdf(V)
    perm = np.random.default_rng([S, set_index, 1 << 20]).permutation(V)
    hist = np.empty((rows, hist_len), dtype=np.int32)
    for r in range(rows):
        g = np.random.default_rng([S, set_index, r, 1])
        ranks = np.searchsorted(cdf, g.random(hist_len), side="right")
        hist[r] = perm[np.minimum(ranks, V - 1)]
    p = default_params(rows)
    p["repeat_penalty"], p["frequency_penalty"], p["presence_penalty"] = 1.1, 0.5, 0.3
    p["repeat_last_n"] = hist_len
    p["temperature"], p["min_p"], p["top_p"] = 0.7, 0.05, 0.9
    seeds = _seeds(S, set_index, rows)
    return Workload("c2", rows, V, "f32", logits, p, seeds, uniforms(seeds),
                    hist_off=np.arange(rows + 1, dtype=np.uint32) * hist_len,
                    hist_ids=hist.reshape(-1), n_top=5, want_logprobs=True)


def make_c2w(rows: int | None = None, set_index: int = 0) -> Workload:
    w = make_c2(rows, set_index)
    p = w.params.copy()
    p["temperature"], p["min_p"] = 1.5, 0.01
    return dataclasses.replace(w, name="c2w", logits=(w.logits / np.float32(3.0)).astype(np.float32),
                               params=p)


def make_c3(rows: int | None = None, set_index: int = 0) -> Workload:
    S, V = CFG_SEED["c3"], VOCAB["c3"]
    rows = FULL_ROWS["c3"] if rows is None else rows
    logits = _normal_rows(S, set_index, rows, V, 1.0)
    p = default_params(rows)
    p["temperature"], p["top_p"] = 1.5, 0.98
    seeds = _seeds(S, set_index, rows)
    return Workload("c3", rows, V, "f32", logits, p, seeds, uniforms(seeds))


def run_mask(g: np.random.Generator, V: int, lo: float = 5e-4, hi: float = 0.30) -> np.ndarray:
    """Allow-mask bits (bool, V) of runs of 1..64 ids until >= f*V are set."""
    f = math.exp(g.uniform(math.log(lo), math.log(hi)))
    target = math.ceil(f * V)
    bits = np.zeros(V, dtype=bool)
    count = 0
    while count < target:
        start = int(g.integers(0, V))
        length = int(g.integers(1, 65))
        seg = bits[start:start + length]
        count += int(seg.size - np.count_nonzero(seg))
        seg[:] = True
    return bits


def pack_mask(bits: np.ndarray) -> np.ndarray:
    V = bits.shape[-1]
    words = (V + 31) // 32
    padded = np.zeros(bits.shape[:-1] + (words * 32,), dtype=bool)
    padded[..., :V] = bits
    return np.packbits(padded, axis=-1, bitorder="little").view("<u4").reshape(
        bits.shape[:-1] + (words,))


def make_c4(rows: int | None = None, set_index: int = 0) -> Workload:
    S, V = CFG_SEED["c4"], VOCAB["c4"]
    rows = FULL_ROWS["c4"] if rows is None else rows
    logits = _normal_rows(S, set_index, rows, V, 2.5)
    bits = np.stack([run_mask(np.random.default_rng([S, set_index, r, 2]), V)
                     for r in range(rows)])
    p = default_params(rows)
    p["temperature"], p["top_p"] = 1.0, 0.95
    seeds = _seeds(S, set_index, rows)
    return Workload("c4", rows, V, "f32", logits, p, seeds, uniforms(seeds),
                    mask=pack_mask(bits), n_top=1, want_logprobs=True)


def make_c5(n_seq: int | None = None, set_index: int = 0, rows_per_seq: int = 8) -> Workload:
    S, V = CFG_SEED["c5"], VOCAB["c5"]
    n_seq = FULL_ROWS["c5"] // rows_per_seq if n_seq is None else n_seq
    rows = n_seq * rows_per_seq
    logits = np.empty((rows, V), dtype=np.uint16)
    draft = np.empty(rows, dtype=np.int32)
    for r in range(rows):
        g = _row_rng(S, set_index, r)
        b = bf16_rne(g.standard_normal(V, dtype=np.float32) * np.float32(2.0))
        dom = int(g.integers(0, V))
        rowmax = bf16_to_f32(b).max()
        b[dom] = bf16_rne(np.array([rowmax + np.float32(6.0)], dtype=np.float32))[0]
        logits[r] = b
        draft[r] = dom if g.random() < 0.75 else int(g.integers(0, V))
    return Workload("c5", rows, V, "bf16", logits, None, None, None,
                    n_seq=n_seq, rows_per_seq=rows_per_seq, draft=draft)


def make(name: str, rows: int | None = None, set_index: int = 0) -> Workload:
    if name == "c1g":
        return make_c1(True, set_index)
    if name == "c1s":
        return make_c1(False, set_index)
    if name == "c2":
        return make_c2(rows, set_index)
    if name == "c2w":
        return make_c2w(rows, set_index)
    if name == "c3":
        return make_c3(rows, set_index)
    if name == "c4":
        return make_c4(rows, set_index)
    if name == "c5":
        return make_c5(None if rows is None else max(1, rows // 8), set_index)
    raise ValueError(f"unknown workload {name!r}")
