"""lcs_sample_noalloc (no context, static device workspace) against
lcs_sample on the same inputs: two calls in a row, the second smaller; free
device memory unchanged by further calls; a batch above its row limit
rejected before any launch. The bar for integer work: every output
bit-identical (both entry points run the same kernels)."""
import sys

import numpy as np
import pytest

from locus_amd import workloads as W
from tests.test_gpu_sampling import _all_paths_workload

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def sampler():
    from locus_amd.sampler import Sampler
    s = Sampler(device=0, max_rows=64, max_vocab=262144, max_hist=8192, max_top=20)
    yield s
    s.close()


def _run(sampler, w, noalloc, has_mask=None):
    d = sampler.upload(w)
    out = sampler.alloc_out(w.rows, w.n_top, w.want_logprobs)
    sampler.sample_dev(d, out, has_mask=has_mask, noalloc=noalloc)
    sampler.torch.cuda.synchronize()
    return sampler.fetch(out, w.n_top)


def _same(a, b, label):
    for k in a:
        assert np.array_equal(np.asarray(a[k]).view(np.uint8), np.asarray(b[k]).view(np.uint8)), f"{label}: {k} differs"


def test_noalloc_matches_lcs_sample_on_two_calls(sampler):
    # call 1: the 64 rows of C2 (the largest batch the static workspace
    # takes); call 2, smaller: every row path over a shorter vocabulary
    w1 = W.make("c2", set_index=7)
    _, w2, has = _all_paths_workload(50000, 20261377)
    torch = sampler.torch
    hm = torch.from_numpy(has).cuda()
    say("noalloc call 1", w1.rows, w1.vocab)
    g1 = _run(sampler, w1, True)
    say("noalloc call 2", w2.rows, w2.vocab)
    g2 = _run(sampler, w2, True, has_mask=hm)
    say("context calls")
    r1 = _run(sampler, w1, False)
    r2 = _run(sampler, w2, False, has_mask=hm)
    _same(g1, r1, "call 1")
    _same(g2, r2, "call 2")
    # and again in the other order on the same static workspace
    g2b = _run(sampler, w2, True, has_mask=hm)
    g1b = _run(sampler, w1, True)
    _same(g2b, r2, "call 2 again")
    _same(g1b, r1, "call 1 again")


def test_noalloc_allocates_no_device_memory(sampler):
    # after a first call (kernels loaded, the array's address looked up),
    # further calls of both sizes leave the device's free memory unchanged
    torch = sampler.torch
    w1 = W.make("c2", set_index=9)
    w2 = W.make("c2", rows=8, set_index=10)
    d1, d2 = sampler.upload(w1), sampler.upload(w2)
    o1 = sampler.alloc_out(w1.rows, w1.n_top, w1.want_logprobs)
    o2 = sampler.alloc_out(w2.rows, w2.n_top, w2.want_logprobs)
    say("noalloc first call")
    sampler.sample_dev(d1, o1, noalloc=True)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    say("noalloc calls 2-5")
    for d, o in ((d1, o1), (d2, o2), (d1, o1), (d2, o2)):
        sampler.sample_dev(d, o, noalloc=True)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 == free0, f"free device memory {free0} -> {free1}"
    r = sampler.fetch(o2, w2.n_top)
    assert (r["ids"] >= 0).all()


def test_noalloc_rejects_rows_above_its_limit(sampler):
    from locus_amd.sampler import LCS_ERR_CAPACITY, SamplerError
    w = W.make("c2", rows=65, set_index=8)
    d = sampler.upload(w)
    out = sampler.alloc_out(w.rows, w.n_top, w.want_logprobs)
    out["ids"].fill_(-7)
    with pytest.raises(SamplerError, match=f"lcs error {LCS_ERR_CAPACITY}"):
        sampler.sample_dev(d, out, noalloc=True)
    sampler.torch.cuda.synchronize()
    assert (out["ids"].cpu().numpy() == -7).all()
