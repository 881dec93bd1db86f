"""ctypes front-end of the CPU oracle (liboracle.so) and, when it has been
built, of the reference harness (_ref/libref.so). TEST INFRASTRUCTURE ONLY:
imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
never by the product package."""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref.so")

DIAG_DTYPE = np.dtype([
    ("id", "<i4"), ("n_cand", "<u4"), ("keep_topk", "<u4"), ("keep_p", "<u4"),
    ("keep", "<u4"), ("pos", "<u4"), ("maxl", "<f4"), ("boundary", "<f4"),
    ("sum", "<f8"), ("kept_sum", "<f8"), ("r", "<f8"), ("margin_p", "<f8"),
    ("margin_m", "<f8"), ("margin_r", "<f8"), ("tie_flags", "<u4"), ("greedy", "<u4"),
])

_P = C.c_void_p


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def build(ref: bool = False) -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    if ref:
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            build()
        L = C.CDLL(ORACLE_SO)
        L.orc_sample.restype = C.c_int32
        L.orc_sample.argtypes = [_P, C.c_uint32, _P, _P, C.c_uint32, C.c_double, _P, _P]
        L.orc_logprobs.restype = None
        L.orc_logprobs.argtypes = [_P, C.c_uint32, C.c_int32, C.c_uint32, _P, _P, _P, _P]
        L.orc_argmax.restype = C.c_int32
        L.orc_argmax.argtypes = [_P, C.c_uint32]
        L.orc_sample_batch.restype = None
        L.orc_sample_batch.argtypes = [_P, C.c_uint32, C.c_uint32, C.c_uint64, _P, _P, _P, _P,
                                       _P, _P, C.c_uint32, C.c_int, C.c_uint32, _P, _P, _P, _P,
                                       _P, C.c_uint32]
        L.orc_verify.restype = None
        L.orc_verify.argtypes = [_P, C.c_int, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint64,
                                 _P, _P, _P, _P, C.c_uint32]
        L.orc_mt_u.restype = C.c_double
        L.orc_mt_u.argtypes = [C.c_uint64, C.c_uint64]
        L.orc_mt_raw.restype = C.c_uint64
        L.orc_mt_raw.argtypes = [C.c_uint64, C.c_uint64]
        L.orc_json_new.restype = _P
        L.orc_json_clone.restype = _P
        L.orc_json_clone.argtypes = [_P]
        L.orc_json_free.argtypes = [_P]
        L.orc_json_feed.restype = C.c_int
        L.orc_json_feed.argtypes = [_P, C.c_uint8]
        L.orc_json_complete.restype = C.c_int
        L.orc_json_complete.argtypes = [_P]
        L.orc_json_mask.restype = None
        L.orc_json_mask.argtypes = [_P, _P, _P, C.c_uint32, C.c_uint32, _P]
        L.orc_ngram_draft.restype = C.c_uint32
        L.orc_ngram_draft.argtypes = [_P, C.c_uint32, C.c_uint32, C.c_uint32, _P]
        L.orc_sizeof_diag.restype = C.c_uint32
        assert L.orc_sizeof_diag() == DIAG_DTYPE.itemsize
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref():
    global _ref
    if _ref is None:
        L = C.CDLL(REF_SO)
        L.ref_sample_batch.restype = None
        L.ref_sample_batch.argtypes = [_P, C.c_uint32, C.c_uint32, C.c_uint64, _P, _P, _P, _P, _P,
                                       _P, _P, C.c_uint32, C.c_int, C.c_uint32, _P, _P, _P, _P,
                                       C.c_uint32]
        L.ref_argmax.restype = C.c_int32
        L.ref_argmax.argtypes = [_P, C.c_uint32]
        L.ref_logprobs.restype = None
        L.ref_logprobs.argtypes = [_P, C.c_uint32, C.c_int32, C.c_uint32, _P, _P, _P]
        L.ref_mt_first.restype = C.c_uint64
        L.ref_mt_first.argtypes = [C.c_uint64]
        L.ref_crafted_first.restype = C.c_uint64
        L.ref_crafted_first.argtypes = [C.c_uint64]
        L.ref_json_feed.restype = C.c_uint32
        L.ref_json_feed.argtypes = [_P, C.c_uint32, _P]
        L.ref_json_mask.restype = C.c_int
        L.ref_json_mask.argtypes = [_P, C.c_uint32, _P, _P, C.c_uint32, C.c_uint32, _P]
        L.ref_ngram_draft.restype = C.c_uint32
        L.ref_ngram_draft.argtypes = [_P, C.c_uint32, C.c_uint32, C.c_uint32, _P]
        _ref = L
    return _ref


class SampleResult:
    def __init__(self, rows, n_top):
        self.ids = np.zeros(rows, dtype=np.int32)
        self.chosen_lp = np.zeros(rows, dtype=np.float32)
        self.top_ids = np.zeros((rows, max(n_top, 1)), dtype=np.int32)
        self.top_lp = np.zeros((rows, max(n_top, 1)), dtype=np.float32)
        self.diag = np.zeros(rows, dtype=DIAG_DTYPE)


def _batch_args(w):
    logits = np.ascontiguousarray(w.logits, dtype=np.float32).copy()  # mutated in place
    params = np.ascontiguousarray(w.params)
    hist_off = None if w.hist_off is None else np.ascontiguousarray(w.hist_off, dtype=np.uint32)
    hist_ids = None if w.hist_ids is None else np.ascontiguousarray(w.hist_ids, dtype=np.int32)
    mask = None if w.mask is None else np.ascontiguousarray(w.mask, dtype=np.uint32)
    return logits, params, hist_off, hist_ids, mask


def sample_batch(w, threads: int = 1, u=None, has_mask=None) -> SampleResult:
    """Oracle over a sampling Workload (the engine's per-row flow)."""
    logits, params, hist_off, hist_ids, mask = _batch_args(w)
    u = np.ascontiguousarray(w.u if u is None else u, dtype=np.float64)
    hm = None if has_mask is None else np.ascontiguousarray(has_mask, dtype=np.uint8)
    res = SampleResult(w.rows, w.n_top)
    lib().orc_sample_batch(_ptr(logits), w.rows, w.vocab, w.vocab, _ptr(params),
                           _ptr(hist_off), _ptr(hist_ids), _ptr(u), _ptr(mask), _ptr(hm),
                           w.mask_words, int(w.want_logprobs), w.n_top, _ptr(res.ids),
                           _ptr(res.chosen_lp), _ptr(res.top_ids), _ptr(res.top_lp),
                           _ptr(res.diag), threads)
    res.penalized = logits
    return res


def ref_sample_batch(w, threads: int = 1, first_out=None, has_mask=None) -> SampleResult:
    """The compiled reference over the same Workload (seeds drive each row's
    mt19937_64; first_out, if given, crafts each row's first output)."""
    logits, params, hist_off, hist_ids, mask = _batch_args(w)
    seeds = np.ascontiguousarray(w.seeds, dtype=np.uint64)
    fo = None if first_out is None else np.ascontiguousarray(first_out, dtype=np.uint64)
    hm = None if has_mask is None else np.ascontiguousarray(has_mask, dtype=np.uint8)
    res = SampleResult(w.rows, w.n_top)
    ref().ref_sample_batch(_ptr(logits), w.rows, w.vocab, w.vocab, _ptr(params),
                           _ptr(hist_off), _ptr(hist_ids), _ptr(seeds), _ptr(fo), _ptr(mask),
                           _ptr(hm), w.mask_words, int(w.want_logprobs), w.n_top,
                           _ptr(res.ids), _ptr(res.chosen_lp), _ptr(res.top_ids),
                           _ptr(res.top_lp), threads)
    res.penalized = logits
    return res


def verify(w, threads: int = 1):
    logits = np.ascontiguousarray(w.logits)
    draft = np.ascontiguousarray(w.draft, dtype=np.int32)
    am = np.zeros(w.rows, dtype=np.int32)
    lp = np.zeros(w.rows, dtype=np.float32)
    acc = np.zeros(w.n_seq, dtype=np.uint32)
    lib().orc_verify(_ptr(logits), int(w.dtype == "bf16"), w.n_seq, w.rows_per_seq, w.vocab,
                     w.vocab, _ptr(draft), _ptr(am), _ptr(lp), _ptr(acc), threads)
    return am, lp, acc


def logprobs(logits: np.ndarray, chosen: int, n_top: int):
    l = np.ascontiguousarray(logits, dtype=np.float32)
    lp = np.zeros(1, dtype=np.float32)
    ids = np.zeros(max(n_top, 1), dtype=np.int32)
    lps = np.zeros(max(n_top, 1), dtype=np.float32)
    tie = np.zeros(1, dtype=np.uint32)
    lib().orc_logprobs(_ptr(l), l.size, chosen, n_top, _ptr(lp), _ptr(ids), _ptr(lps), _ptr(tie))
    return float(lp[0]), ids[:n_top].copy(), lps[:n_top].copy(), bool(tie[0])


def sample_row(logits, params, hist=None, u=0.0, mask=None):
    """One reference-style sample() call; returns (id, penalized logits, diag)."""
    l = np.ascontiguousarray(logits, dtype=np.float32).copy()
    p = np.ascontiguousarray(params)
    h = None if hist is None else np.ascontiguousarray(hist, dtype=np.int32)
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint32)
    d = np.zeros(1, dtype=DIAG_DTYPE)
    rid = lib().orc_sample(_ptr(l), l.size, _ptr(p), _ptr(h), 0 if h is None else h.size,
                           float(u), _ptr(m), _ptr(d))
    return int(rid), l, d[0]


class OracleJson:
    """JsonGrammar restatement handle (grammar.cpp)."""

    def __init__(self, handle=None):
        self.h = handle if handle is not None else lib().orc_json_new()

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_json_free(self.h)
            self.h = None

    def clone(self):
        return OracleJson(lib().orc_json_clone(self.h))

    def feed(self, b: int) -> bool:
        return bool(lib().orc_json_feed(self.h, b))

    def feed_all(self, s: bytes) -> bool:
        return all(self.feed(b) for b in s)

    def complete(self) -> bool:
        return bool(lib().orc_json_complete(self.h))

    def mask(self, pieces: list[bytes], V: int) -> np.ndarray:
        blob = np.frombuffer(b"".join(pieces) or b"\0", dtype=np.uint8)
        off = np.zeros(len(pieces) + 1, dtype=np.uint64)
        off[1:] = np.cumsum([len(p) for p in pieces])
        out = np.zeros((V + 31) // 32, dtype=np.uint32)
        lib().orc_json_mask(self.h, _ptr(blob), _ptr(off), len(pieces), V, _ptr(out))
        return out


def ngram_draft(ctx, ngram: int, max_draft: int) -> list[int]:
    c = np.ascontiguousarray(ctx, dtype=np.int32)
    out = np.zeros(max(max_draft, 1), dtype=np.int32)
    n = lib().orc_ngram_draft(_ptr(c), c.size, ngram, max_draft, _ptr(out))
    return out[:n].tolist()
