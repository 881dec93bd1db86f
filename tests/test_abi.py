"""The C-ABI library loads and exports every entry point the public headers
declare; without a device it fails loudly (no CPU fallback)."""
import ctypes
import glob
import os
import re

import pytest

from locus_amd import sampler

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions(prefix="lcs_", header="*.h"):
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", header)):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(" + prefix + r"\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return sorted(names)


def test_headers_declare_the_abi():
    names = declared_functions()
    for n in ["lcs_probe", "lcs_create", "lcs_destroy", "lcs_sample", "lcs_verify", "lcs_last_error",
              "lcs_sample_noalloc", "lcs_ngram_draft", "lcs_lmhead"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = sampler.lib()
    for n in declared_functions():
        assert hasattr(lib, n), n


def test_host_library_exports_every_declared_symbol():
    from locus_amd import host_lib
    names = declared_functions("lch_", "locus_host.h")
    assert {"lch_json_new", "lch_json_feed", "lch_mask_build", "lch_ngram_draft",
            "lch_resolve_sampler_backend"} <= set(names)
    lib = host_lib.lib()
    for n in names:
        assert hasattr(lib, n), n


def _gpu_visible():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def test_no_device_fails_loudly():
    if _gpu_visible():
        pytest.skip("a GPU is visible")
    assert sampler.probe() == 0
    with pytest.raises(sampler.SamplerError):
        sampler.Sampler(device=0)
