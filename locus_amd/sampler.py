"""Python binding of the C ABI in include/locus_sampler.h (ctypes).

The product path is liblocus_sampler.so (HIP kernels for gfx950); this module
only marshals device pointers. PyTorch supplies device memory and the HIP
stream. There is no CPU fallback: a missing library or device raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from .workloads import PARAMS_DTYPE

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblocus_sampler.so")

LCS_OK, LCS_ERR_INVALID_ARG, LCS_ERR_NO_DEVICE, LCS_ERR_HIP, LCS_ERR_CAPACITY = 0, -1, -2, -3, -4
LCS_F32, LCS_BF16 = 0, 1
LCS_WANT_LOGPROBS, LCS_WRITE_PENALIZED = 1, 2
PATH_GREEDY, PATH_WINDOW, PATH_WINDOW_EXACT, PATH_GENERAL = 1, 2, 3, 4

DIAG_DTYPE = np.dtype([
    ("n_cand", "<u4"), ("keep", "<u4"), ("maxl", "<f4"), ("boundary", "<f4"),
    ("path", "<u4"), ("reserved", "<u4"), ("sum", "<f8"), ("kept_sum", "<f8"),
])

_P = C.c_void_p


class _Batch(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("vocab", C.c_uint32), ("dtype", C.c_uint32),
                ("flags", C.c_uint32), ("row_stride", C.c_uint64), ("logits", _P),
                ("params", _P), ("params_host", _P), ("hist_off", _P), ("hist_ids", _P),
                ("u", _P), ("mask", _P), ("has_mask", _P), ("mask_words", C.c_uint32),
                ("n_top", C.c_uint32), ("lp_ids", _P), ("win_slot", _P), ("win_push", _P),
                ("win_len", _P), ("raw_stats", _P)]


class _Out(C.Structure):
    _fields_ = [("ids", _P), ("chosen_lp", _P), ("top_ids", _P), ("top_lp", _P), ("diag", _P)]


class _VBatch(C.Structure):
    _fields_ = [("n_seq", C.c_uint32), ("rows_per_seq", C.c_uint32), ("vocab", C.c_uint32),
                ("dtype", C.c_uint32), ("row_stride", C.c_uint64), ("logits", _P), ("draft", _P)]


class _VOut(C.Structure):
    _fields_ = [("argmax_ids", _P), ("draft_lp", _P), ("accept_len", _P)]


class _DBatch(C.Structure):
    _fields_ = [("n_seq", C.c_uint32), ("ngram", C.c_uint32), ("max_draft", C.c_uint32),
                ("ctx_off", _P), ("ctx_ids", _P)]


class _DOut(C.Structure):
    _fields_ = [("draft", _P), ("draft_len", _P)]


class _LBatch(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("vocab", C.c_uint32), ("hidden", C.c_uint32),
                ("rows_per_seq", C.c_uint32), ("x", _P), ("w", _P), ("draft", _P)]


class _LOut(C.Structure):
    _fields_ = [("logits", _P), ("ld_logits", C.c_uint64), ("argmax_ids", _P), ("log_z", _P),
                ("draft_lp", _P), ("accept_len", _P), ("stats", _P)]


class SamplerError(RuntimeError):
    pass


_lib = None


def lib():
    """Loads liblocus_sampler.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise SamplerError(f"{LIB_PATH} is missing: run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        L.lcs_probe.restype = C.c_int
        L.lcs_probe.argtypes = [C.POINTER(C.c_int)]
        L.lcs_create.restype = _P
        L.lcs_create.argtypes = [C.c_int, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]
        L.lcs_destroy.restype = None
        L.lcs_destroy.argtypes = [_P]
        L.lcs_sample.restype = C.c_int
        L.lcs_sample.argtypes = [_P, C.POINTER(_Batch), C.POINTER(_Out), _P]
        L.lcs_sample_noalloc.restype = C.c_int
        L.lcs_sample_noalloc.argtypes = [C.POINTER(_Batch), C.POINTER(_Out), _P]
        L.lcs_verify.restype = C.c_int
        L.lcs_verify.argtypes = [_P, C.POINTER(_VBatch), C.POINTER(_VOut), _P]
        L.lcs_ngram_draft.restype = C.c_int
        L.lcs_ngram_draft.argtypes = [_P, C.POINTER(_DBatch), C.POINTER(_DOut), _P]
        L.lcs_lmhead.restype = C.c_int
        L.lcs_lmhead.argtypes = [_P, C.POINTER(_LBatch), C.POINTER(_LOut), _P]
        L.lcs_last_error.restype = C.c_char_p
        L.lcs_last_error.argtypes = [_P]
        L.lcs_logprobs.restype = C.c_int
        L.lcs_logprobs.argtypes = [_P, C.POINTER(_Batch), _P, C.POINTER(_Out), _P]
        L.lcs_windows_reserve.restype = C.c_int
        L.lcs_windows_reserve.argtypes = [_P, C.c_uint32, C.c_uint32]
        L.lcs_windows_load.restype = C.c_int
        L.lcs_windows_load.argtypes = [_P, C.c_uint32, _P, C.c_uint32, C.c_uint32, C.c_uint32, _P]
        L.lcs_get_status.restype = C.c_int
        L.lcs_get_status.argtypes = [_P, C.POINTER(C.c_uint32), C.c_int]
        _lib = L
    return _lib


def probe() -> int:
    n = C.c_int(0)
    lib().lcs_probe(C.byref(n))
    return n.value


def _dptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream_handle(torch, stream):
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


class Sampler:
    """One lcs_ctx on one device; workspace is allocated here, once."""

    def __init__(self, device: int = 0, max_rows: int = 256, max_vocab: int = 262144,
                 max_hist: int = 4096, max_top: int = 20):
        import torch  # plumbing: device memory and streams
        self.torch = torch
        self.device = device
        L = lib()
        self.ctx = L.lcs_create(device, max_rows, max_vocab, max_hist, max_top)
        if not self.ctx:
            raise SamplerError(L.lcs_last_error(None).decode())
        self.max_rows, self.max_vocab, self.max_top = max_rows, max_vocab, max_top

    def close(self):
        if getattr(self, "ctx", None):
            lib().lcs_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int):
        if rc != LCS_OK:
            raise SamplerError(f"lcs error {rc}: {lib().lcs_last_error(self.ctx).decode()}")

    def status(self, reset: bool = True) -> int:
        s = C.c_uint32(0)
        self._check(lib().lcs_get_status(self.ctx, C.byref(s), int(reset)))
        return s.value

    # ------------------------------------------------- device-resident windows
    def windows_reserve(self, slots: int, max_window: int):
        self._check(lib().lcs_windows_reserve(self.ctx, slots, max_window))

    def windows_load(self, slot: int, ids, window: int, vocab: int, stream=None):
        """Starts `slot` from a history (a device int32 tensor, or None for an
        empty one)."""
        n = 0 if ids is None else int(ids.numel())
        self._check(lib().lcs_windows_load(self.ctx, slot, _dptr(ids) if n else None, n, window, vocab,
                                           _stream_handle(self.torch, stream)))

    # ---------------------------------------------------------------- inputs
    def upload(self, w, stride: int | None = None):
        """Device copies of a workloads.Workload (sampling configs)."""
        torch = self.torch
        dev = torch.device("cuda", self.device)
        V = w.vocab
        G = 8 if w.dtype == "bf16" else 4
        stride = stride or ((V + G - 1) // G * G)
        if w.dtype == "bf16":
            host = np.zeros((w.rows, stride), dtype=np.uint16)
            host[:, :V] = w.logits
            logits = torch.from_numpy(host.view(np.int16)).to(dev).view(torch.bfloat16)
        else:
            host = np.zeros((w.rows, stride), dtype=np.float32)
            host[:, :V] = w.logits
            logits = torch.from_numpy(host).to(dev)
        d = {"logits": logits, "stride": stride, "w": w}
        if w.params is not None:
            d["params"] = torch.from_numpy(np.ascontiguousarray(w.params).view(np.uint8).copy()).to(dev)
            d["params_host"] = np.ascontiguousarray(w.params)
        if w.u is not None:
            d["u"] = torch.from_numpy(np.ascontiguousarray(w.u, dtype=np.float64)).to(dev)
        if w.hist_off is not None:
            d["hist_off"] = torch.from_numpy(w.hist_off.astype(np.int32).view(np.int32)).to(dev)
            ids = np.ascontiguousarray(w.hist_ids, dtype=np.int32)
            if ids.size == 0:  # an empty tensor has no data pointer
                ids = np.zeros(1, dtype=np.int32)
            d["hist_ids"] = torch.from_numpy(ids).to(dev)
        if w.mask is not None:
            d["mask"] = torch.from_numpy(np.ascontiguousarray(w.mask).view(np.int32)).to(dev)
        if w.draft is not None:
            d["draft"] = torch.from_numpy(np.ascontiguousarray(w.draft, dtype=np.int32)).to(dev)
        return d

    def alloc_out(self, rows: int, n_top: int, want_lp: bool, diag: bool = True):
        torch = self.torch
        dev = torch.device("cuda", self.device)
        o = {"ids": torch.full((rows,), -7, dtype=torch.int32, device=dev)}
        if want_lp:
            o["chosen_lp"] = torch.zeros(rows, dtype=torch.float32, device=dev)
            o["top_ids"] = torch.zeros((rows, max(n_top, 1)), dtype=torch.int32, device=dev)
            o["top_lp"] = torch.zeros((rows, max(n_top, 1)), dtype=torch.float32, device=dev)
        if diag:
            o["diag"] = torch.zeros(rows * DIAG_DTYPE.itemsize, dtype=torch.uint8, device=dev)
        return o

    # ---------------------------------------------------------------- calls
    def prepare(self, d, out, n_top: int | None = None, want_lp: bool | None = None,
                has_mask=None, flags_extra: int = 0, use_host_params: bool = True, win=None, raw_stats=None):
        """Builds the C structs of one lcs_sample call once; returns a
        zero-argument launcher (for tight benchmark loops)."""
        w = d["w"]
        want_lp = w.want_logprobs if want_lp is None else want_lp
        n_top = w.n_top if n_top is None else n_top
        b = _Batch()
        b.rows, b.vocab = w.rows, w.vocab
        b.dtype = LCS_BF16 if w.dtype == "bf16" else LCS_F32
        b.flags = (LCS_WANT_LOGPROBS if want_lp else 0) | flags_extra
        b.row_stride = d["stride"]
        b.logits = _dptr(d["logits"])
        b.params = _dptr(d["params"])
        ph = d["params_host"] if use_host_params else None
        b.params_host = None if ph is None else ph.ctypes.data_as(C.c_void_p)
        b.hist_off = _dptr(d.get("hist_off"))
        b.hist_ids = _dptr(d.get("hist_ids"))
        b.u = _dptr(d.get("u"))
        b.mask = _dptr(d.get("mask"))
        b.has_mask = _dptr(has_mask)
        b.mask_words = w.mask_words
        b.n_top = n_top if want_lp else 0
        if win is not None:
            b.win_slot, b.win_push, b.win_len = _dptr(win["slot"]), _dptr(win["push"]), _dptr(win["len"])
            b.hist_off = b.hist_ids = None
        b.raw_stats = _dptr(raw_stats)
        o = _Out()
        o.ids = _dptr(out["ids"])
        o.chosen_lp = _dptr(out.get("chosen_lp"))
        o.top_ids = _dptr(out.get("top_ids"))
        o.top_lp = _dptr(out.get("top_lp"))
        o.diag = _dptr(out.get("diag"))
        fn, ctx, bp, op = lib().lcs_sample, self.ctx, C.byref(b), C.byref(o)
        keep = (ph, b, o, d, out, win, raw_stats)

        def launch(stream_handle):
            _ = keep
            rc = fn(ctx, bp, op, stream_handle)
            if rc != LCS_OK:
                self._check(rc)
        return launch

    def prepare_verify(self, d, out):
        w = d["w"]
        b = _VBatch()
        b.n_seq, b.rows_per_seq, b.vocab = w.n_seq, w.rows_per_seq, w.vocab
        b.dtype = LCS_BF16 if w.dtype == "bf16" else LCS_F32
        b.row_stride = d["stride"]
        b.logits = _dptr(d["logits"])
        b.draft = _dptr(d["draft"])
        o = _VOut()
        o.argmax_ids = _dptr(out["argmax_ids"])
        o.draft_lp = _dptr(out["draft_lp"])
        o.accept_len = _dptr(out["accept_len"])
        fn, ctx, bp, op = lib().lcs_verify, self.ctx, C.byref(b), C.byref(o)
        keep = (b, o, d, out)

        def launch(stream_handle):
            _ = keep
            rc = fn(ctx, bp, op, stream_handle)
            if rc != LCS_OK:
                self._check(rc)
        return launch

    def stream_handle(self, stream=None):
        return _stream_handle(self.torch, stream)

    def sample_dev(self, d, out, n_top: int | None = None, want_lp: bool | None = None,
                   has_mask=None, flags_extra: int = 0, use_host_params: bool = True, stream=None,
                   lp_ids=None, noalloc: bool = False, win=None, raw_stats=None):
        """Enqueues lcs_sample on device buffers from upload()/alloc_out();
        `lp_ids` (device int32 per row) makes chosen_lp report those ids;
        `noalloc` calls lcs_sample_noalloc (no context) instead; `win`
        ({"slot", "push", "len"}: device int32 / int32 / uint32 per row) takes
        the rows' penalty windows from device-resident slots instead of the
        workload's history; `raw_stats` (the "stats" output of lmhead_dev on
        the same logits) gives the rows' raw log-normalisers."""
        w = d["w"]
        want_lp = w.want_logprobs if want_lp is None else want_lp
        n_top = w.n_top if n_top is None else n_top
        b = _Batch()
        b.rows, b.vocab = w.rows, w.vocab
        b.dtype = LCS_BF16 if w.dtype == "bf16" else LCS_F32
        b.flags = (LCS_WANT_LOGPROBS if want_lp else 0) | flags_extra
        b.row_stride = d["stride"]
        b.logits = _dptr(d["logits"])
        b.params = _dptr(d["params"])
        ph = d["params_host"] if use_host_params else None
        b.params_host = None if ph is None else ph.ctypes.data_as(C.c_void_p)
        b.hist_off = _dptr(d.get("hist_off"))
        b.hist_ids = _dptr(d.get("hist_ids"))
        b.u = _dptr(d.get("u"))
        b.mask = _dptr(d.get("mask"))
        b.has_mask = _dptr(has_mask)
        b.mask_words = w.mask_words
        b.n_top = n_top if want_lp else 0
        b.lp_ids = _dptr(lp_ids)
        if win is not None:
            b.win_slot, b.win_push, b.win_len = _dptr(win["slot"]), _dptr(win["push"]), _dptr(win["len"])
            b.hist_off = b.hist_ids = None
        b.raw_stats = _dptr(raw_stats)
        o = _Out()
        o.ids = _dptr(out["ids"])
        o.chosen_lp = _dptr(out.get("chosen_lp"))
        o.top_ids = _dptr(out.get("top_ids"))
        o.top_lp = _dptr(out.get("top_lp"))
        o.diag = _dptr(out.get("diag"))
        self._keep = (ph, b, o, lp_ids, win, raw_stats)
        sh = _stream_handle(self.torch, stream)
        if noalloc:
            rc = lib().lcs_sample_noalloc(C.byref(b), C.byref(o), sh)
            if rc != LCS_OK:
                raise SamplerError(f"lcs error {rc}: {lib().lcs_last_error(None).decode()}")
            return
        self._check(lib().lcs_sample(self.ctx, C.byref(b), C.byref(o), sh))

    def sample(self, w, **kw):
        """Uploads a Workload, samples it, and returns host numpy results."""
        d = self.upload(w)
        out = self.alloc_out(w.rows, w.n_top, w.want_logprobs)
        self.sample_dev(d, out, **kw)
        self.torch.cuda.synchronize()
        return self.fetch(out, w.n_top)

    def logprobs_dev(self, d, out, chosen=None, n_top: int | None = None, raw_stats=None, stream=None):
        """Enqueues lcs_logprobs (logprobs_from over the batch, no draw) on
        device buffers from upload()/alloc_out(): `chosen` (device int32 per
        row, or None for each row's argmax)."""
        w = d["w"]
        b = _Batch()
        b.rows, b.vocab = w.rows, w.vocab
        b.dtype = LCS_BF16 if w.dtype == "bf16" else LCS_F32
        b.row_stride = d["stride"]
        b.logits = _dptr(d["logits"])
        b.n_top = w.n_top if n_top is None else n_top
        b.raw_stats = _dptr(raw_stats)
        o = _Out()
        o.ids = _dptr(out.get("ids"))
        o.chosen_lp = _dptr(out.get("chosen_lp"))
        o.top_ids = _dptr(out.get("top_ids"))
        o.top_lp = _dptr(out.get("top_lp"))
        self._keep = (b, o, chosen, raw_stats)
        self._check(lib().lcs_logprobs(self.ctx, C.byref(b), _dptr(chosen), C.byref(o),
                                       _stream_handle(self.torch, stream)))

    @staticmethod
    def fetch(out, n_top: int):
        r = {"ids": out["ids"].cpu().numpy()}
        if "chosen_lp" in out:
            r["chosen_lp"] = out["chosen_lp"].cpu().numpy()
            r["top_ids"] = out["top_ids"].cpu().numpy()[:, :n_top]
            r["top_lp"] = out["top_lp"].cpu().numpy()[:, :n_top]
        if "diag" in out:
            r["diag"] = out["diag"].cpu().numpy().view(DIAG_DTYPE)
        return r

    def verify_dev(self, d, out, stream=None):
        w = d["w"]
        b = _VBatch()
        b.n_seq, b.rows_per_seq, b.vocab = w.n_seq, w.rows_per_seq, w.vocab
        b.dtype = LCS_BF16 if w.dtype == "bf16" else LCS_F32
        b.row_stride = d["stride"]
        b.logits = _dptr(d["logits"])
        b.draft = _dptr(d["draft"])
        o = _VOut()
        o.argmax_ids = _dptr(out["argmax_ids"])
        o.draft_lp = _dptr(out["draft_lp"])
        o.accept_len = _dptr(out["accept_len"])
        self._keep = (b, o)
        self._check(lib().lcs_verify(self.ctx, C.byref(b), C.byref(o),
                                     _stream_handle(self.torch, stream)))

    def alloc_verify_out(self, w):
        torch = self.torch
        dev = torch.device("cuda", self.device)
        return {"argmax_ids": torch.full((w.rows,), -7, dtype=torch.int32, device=dev),
                "draft_lp": torch.zeros(w.rows, dtype=torch.float32, device=dev),
                "accept_len": torch.full((w.n_seq,), 99, dtype=torch.int32, device=dev)}

    def ngram_draft(self, contexts, ngram: int, max_draft: int):
        """Batched prompt-lookup drafts (lcs_ngram_draft) for a list of token
        sequences; returns (drafts: list of lists, raw (n_seq, max_draft) array)."""
        torch = self.torch
        dev = torch.device("cuda", self.device)
        n = len(contexts)
        off = np.zeros(n + 1, dtype=np.uint32)
        off[1:] = np.cumsum([len(c) for c in contexts])
        ids = np.concatenate([np.asarray(c, dtype=np.int32) for c in contexts]) if off[-1] else np.zeros(1, np.int32)
        off_d = torch.from_numpy(off.view(np.int32)).to(dev)
        ids_d = torch.from_numpy(ids).to(dev)
        dr = torch.full((n, max(max_draft, 1)), -7, dtype=torch.int32, device=dev)
        ln = torch.full((n,), 999, dtype=torch.int32, device=dev)
        b = _DBatch()
        b.n_seq, b.ngram, b.max_draft = n, ngram, max_draft
        b.ctx_off, b.ctx_ids = _dptr(off_d), _dptr(ids_d)
        o = _DOut()
        o.draft, o.draft_len = _dptr(dr), _dptr(ln)
        self._check(lib().lcs_ngram_draft(self.ctx, C.byref(b), C.byref(o), None))
        torch.cuda.synchronize()
        raw = dr.cpu().numpy()[:, :max_draft]
        lens = ln.cpu().numpy()
        return [raw[i, :lens[i]].tolist() for i in range(n)], raw

    def lmhead_dev(self, x, w, out, draft=None, rows_per_seq: int = 0, stream=None):
        """The fused lm-head product (lcs_lmhead) on device tensors: x (rows,
        hidden) and w (vocab, hidden) bf16, contiguous; `out` holds any of
        "logits" (rows, >= vocab) f32, "argmax_ids", "log_z", "draft_lp",
        "accept_len", "stats" (rows x 16 bytes, lcs_row_stats: pass it as
        sample_dev's raw_stats) (missing keys are not written; argmax_ids is
        required)."""
        torch = self.torch
        if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
            raise SamplerError("x and w must be bfloat16")
        if not (x.is_contiguous() and w.is_contiguous()):
            raise SamplerError("x and w must be contiguous")
        b = _LBatch()
        b.rows, b.hidden = x.shape
        b.vocab = w.shape[0]
        if w.shape[1] != b.hidden:
            raise SamplerError("x and w disagree on hidden")
        b.rows_per_seq = rows_per_seq
        b.x, b.w, b.draft = _dptr(x), _dptr(w), _dptr(draft)
        o = _LOut()
        lg = out.get("logits")
        if lg is not None:
            if lg.dtype != torch.float32 or lg.stride(1) != 1:
                raise SamplerError("logits must be f32 with unit column stride")
            o.logits, o.ld_logits = _dptr(lg), lg.stride(0)
        for k in ("argmax_ids", "log_z", "draft_lp", "accept_len", "stats"):
            setattr(o, k, _dptr(out.get(k)))
        self._keep = (b, o)
        self._check(lib().lcs_lmhead(self.ctx, C.byref(b), C.byref(o),
                                     _stream_handle(torch, stream)))

    def alloc_lmhead_out(self, rows: int, vocab: int, logits: bool = True, draft: bool = False,
                         n_seq: int = 0, stats: bool = False):
        torch = self.torch
        dev = torch.device("cuda", self.device)
        out = {"argmax_ids": torch.full((rows,), -7, dtype=torch.int32, device=dev),
               "log_z": torch.full((rows,), -7.0, dtype=torch.float32, device=dev)}
        if logits:
            out["logits"] = torch.full((rows, vocab), -7.0, dtype=torch.float32, device=dev)
        if draft:
            out["draft_lp"] = torch.full((rows,), -7.0, dtype=torch.float32, device=dev)
        if n_seq:
            out["accept_len"] = torch.full((n_seq,), 99, dtype=torch.int32, device=dev)
        if stats:   # lcs_row_stats: (f64 log_z, f32 max, i32 argmax) per row
            out["stats"] = torch.full((rows, 2), -7.0, dtype=torch.float64, device=dev)
        return out

    def verify(self, w):
        d = self.upload(w)
        out = self.alloc_verify_out(w)
        self.verify_dev(d, out)
        self.torch.cuda.synchronize()
        return {k: v.cpu().numpy() for k, v in out.items()}
