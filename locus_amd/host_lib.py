"""ctypes handle on liblocus_host.so (include/locus_host.h): JSON grammar,
allow-mask builder, n-gram draft and sampler-backend resolution."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
HOST_SO = os.path.join(HERE, "liblocus_host.so")
_lib = None


def lib():
    """Loads the built host library (building it first when it is absent)."""
    global _lib
    if _lib is None:
        if not os.path.exists(HOST_SO):
            from locus_amd import build
            build.build_all()
        L = C.CDLL(HOST_SO)
        L.lch_last_error.restype = C.c_char_p
        L.lch_json_new.restype = C.c_void_p
        L.lch_json_clone.restype = C.c_void_p
        L.lch_json_clone.argtypes = [C.c_void_p]
        L.lch_json_free.argtypes = [C.c_void_p]
        L.lch_json_feed.argtypes = [C.c_void_p, C.c_uint8]
        L.lch_json_complete.argtypes = [C.c_void_p]
        L.lch_mask_builder_new.restype = C.c_void_p
        L.lch_mask_builder_new.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32]
        L.lch_mask_builder_free.argtypes = [C.c_void_p]
        L.lch_mask_build.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p]
        L.lch_mask_cache_stats.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
        L.lch_ngram_draft.restype = C.c_uint32
        L.lch_ngram_draft.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p, C.c_uint32]
        L.lch_resolve_sampler_backend.argtypes = [C.c_char_p, C.c_char_p, C.c_uint32]
        _lib = L
    return _lib


class JsonGrammar:
    def __init__(self, handle=None):
        self.h = handle if handle is not None else lib().lch_json_new()

    def __del__(self):
        if getattr(self, "h", None):
            lib().lch_json_free(self.h)
            self.h = None

    def clone(self) -> "JsonGrammar":
        return JsonGrammar(lib().lch_json_clone(self.h))

    def feed(self, b: int) -> bool:
        return bool(lib().lch_json_feed(self.h, b))

    def complete(self) -> bool:
        return bool(lib().lch_json_complete(self.h))


class MaskBuilder:
    """Allow-mask builder over a token piece table (list of bytes)."""

    def __init__(self, pieces: list[bytes], cache_entries: int = 256):
        blob = np.frombuffer(b"".join(pieces) or b"\0", dtype=np.uint8).copy()
        off = np.zeros(len(pieces) + 1, dtype=np.uint64)
        off[1:] = np.cumsum([len(p) for p in pieces])
        self._keep = (blob, off)
        self.h = lib().lch_mask_builder_new(blob.ctypes.data, off.ctypes.data, len(pieces), cache_entries)
        if not self.h:
            raise RuntimeError(lib().lch_last_error().decode())

    def __del__(self):
        if getattr(self, "h", None):
            lib().lch_mask_builder_free(self.h)
            self.h = None

    def build(self, g: JsonGrammar, vocab: int) -> np.ndarray:
        out = np.zeros((vocab + 31) // 32, dtype=np.uint32)
        if lib().lch_mask_build(self.h, g.h, vocab, out.ctypes.data) != 0:
            raise RuntimeError(lib().lch_last_error().decode())
        return out

    def cache_stats(self):
        h, m = C.c_uint64(), C.c_uint64()
        lib().lch_mask_cache_stats(self.h, C.byref(h), C.byref(m))
        return h.value, m.value


def ngram_draft(ctx, ngram: int, max_draft: int) -> list[int]:
    a = np.ascontiguousarray(ctx, dtype=np.int32)
    out = np.zeros(max(max_draft, 1), dtype=np.int32)
    k = lib().lch_ngram_draft(a.ctypes.data if a.size else None, a.size, ngram, max_draft,
                              out.ctypes.data, out.size)
    return out[:k].tolist()


def resolve_sampler_backend(choice: str = "") -> tuple[int, str]:
    buf = C.create_string_buffer(64)
    rc = lib().lch_resolve_sampler_backend(choice.encode(), buf, 64)
    return rc, (buf.value.decode() if rc == 0 else lib().lch_last_error().decode())
