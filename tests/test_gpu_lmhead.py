"""The fused lm-head product (lcs_lmhead, lcs_lmhead.hip) through the C ABI.

Two gates, as for every kernel here:
- the logits against the exact product: bit-exact on small-integer operands
  (every bf16 product and every partial sum is then an exactly representable
  f32 integer), and within K * 2^-24 * sum_k |x_k w_k| of the float64 product
  on random operands (f32 accumulation of exact bf16 x bf16 products);
- the epilogue's statistics against the kernel's own written logits: argmax
  bit-exact with the first-index rule (llama.cpp:1237-1245), the draft
  logprob and acceptance length against the oracle's verify
  (sampling.cpp:150-170, engine.cpp:357-383), log_z (returned in f32)
  within 1e-5 plus half an f32 spacing of the float64 log-sum-exp.
"""
import sys
from types import SimpleNamespace

import numpy as np
import pytest

from oracle import pyoracle as O
from tests.util import LOGPROB_TOL

pytestmark = pytest.mark.gpu
U = 2.0 ** -24


@pytest.fixture(scope="module")
def sampler():
    from locus_amd.sampler import Sampler
    s = Sampler(device=0, max_rows=512, max_vocab=262144, max_hist=64, max_top=4)
    yield s
    s.close()


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bf16(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)


def run(sampler, x, w, draft=None, rows_per_seq=0, logits=True):
    """x (rows, hidden), w (vocab, hidden) bf16 on the device."""
    torch = sampler.torch
    rows, vocab = x.shape[0], w.shape[0]
    n_seq = rows // rows_per_seq if (rows_per_seq and draft is not None) else 0
    out = sampler.alloc_lmhead_out(rows, vocab, logits=logits, draft=draft is not None, n_seq=n_seq)
    sampler.lmhead_dev(x, w, out, draft=draft, rows_per_seq=rows_per_seq)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in out.items()}


def logsumexp64(l):
    l = l.astype(np.float64)
    m = l.max(axis=1, keepdims=True)
    return (m + np.log(np.exp(l - m).sum(axis=1, keepdims=True)))[:, 0]


def check_epilogue(g, draft=None, rows_per_seq=0):
    """The fused statistics against the written logits."""
    lg = g["logits"]
    assert np.array_equal(g["argmax_ids"], np.argmax(lg, axis=1).astype(np.int32))
    # log_z is returned in f32: 1e-5 plus half an f32 spacing at its magnitude
    lz = logsumexp64(lg)
    assert (np.abs(g["log_z"] - lz) <= LOGPROB_TOL + 0.5 * np.spacing(np.abs(lz).astype(np.float32))).all()
    if draft is not None:
        rows, vocab = lg.shape
        R = rows_per_seq or 1
        w = SimpleNamespace(logits=lg, draft=draft, dtype="f32", n_seq=rows // R, rows_per_seq=R,
                            vocab=vocab, rows=rows)
        am, lp, acc = O.verify(w, threads=16)
        assert np.array_equal(g["argmax_ids"], am)
        assert np.abs(g["draft_lp"] - lp).max() <= LOGPROB_TOL
        if rows_per_seq:
            assert np.array_equal(g["accept_len"].astype(np.uint32), acc)


def test_integer_operands_are_exact(sampler):
    """Small integers: the product is exact, so the logits are bit-exact and
    ties between columns are frequent (the first index must win)."""
    torch = sampler.torch
    rng = np.random.default_rng(1)
    for rows, vocab, hidden in [(5, 1000, 128), (64, 4096, 64), (67, 300, 192), (1, 1, 64), (130, 257, 256)]:
        say("integer", rows, vocab, hidden)
        xi = rng.integers(-4, 5, (rows, hidden)).astype(np.float32)
        wi = rng.integers(-3, 4, (vocab, hidden)).astype(np.float32)
        ref = (xi.astype(np.int64) @ wi.astype(np.int64).T).astype(np.float32)
        g = run(sampler, bf16(torch, xi).cuda(), bf16(torch, wi).cuda())
        assert np.array_equal(g["logits"], ref)
        check_epilogue(g)
        if vocab > 1:
            ties = sum(int((ref[r] == ref[r].max()).sum() > 1) for r in range(rows))
            say("rows whose maximum is tied:", ties)


# (151936: a vocabulary the kernel serves with 320-column blocks, to fit one
# round of resident workgroups)
@pytest.mark.parametrize("rows,vocab,hidden", [(64, 32000, 1024), (130, 5000, 512), (8, 257, 4096),
                                               (8, 151936, 256)])
def test_random_operands_within_the_f32_bound(sampler, rows, vocab, hidden):
    torch = sampler.torch
    say("random", rows, vocab, hidden)
    rng = np.random.default_rng(rows * 7 + vocab)
    x = bf16(torch, rng.standard_normal((rows, hidden)))
    w = bf16(torch, rng.standard_normal((vocab, hidden)) * 0.05)
    g = run(sampler, x.cuda(), w.cuda())
    x64, w64 = x.double().numpy(), w.double().numpy()
    ref = x64 @ w64.T
    bound = hidden * U * (np.abs(x64) @ np.abs(w64).T)
    assert (np.abs(g["logits"] - ref) <= bound).all()
    check_epilogue(g)


@pytest.mark.parametrize("vocab", [20000, 140000])
def test_drafts_and_acceptance(sampler, vocab):
    """rows_per_seq = 8: each sequence's drafts agree with the argmax on a
    chosen prefix, then differ; the last row carries no draft (-1)."""
    torch = sampler.torch
    rng = np.random.default_rng(5)
    n_seq, R, hidden = 24, 8, 512
    rows = n_seq * R
    x = bf16(torch, rng.standard_normal((rows, hidden))).cuda()
    w = bf16(torch, rng.standard_normal((vocab, hidden)) * 0.05).cuda()
    first = run(sampler, x, w)
    am = first["argmax_ids"].reshape(n_seq, R)
    prefix = rng.integers(0, R, n_seq)
    prefix[:3] = [0, R - 1, 3]
    draft = rng.integers(0, vocab, (n_seq, R)).astype(np.int32)
    for s in range(n_seq):
        draft[s, :prefix[s]] = am[s, :prefix[s]]
        if draft[s, prefix[s]] == am[s, prefix[s]]:
            draft[s, prefix[s]] = (am[s, prefix[s]] + 1) % vocab
    draft[:, R - 1] = -1
    draft[5, 2] = vocab     # out of range: logprob 0
    d = torch.from_numpy(draft.reshape(-1)).cuda()
    g = run(sampler, x, w, draft=d, rows_per_seq=R)
    assert np.array_equal(g["logits"], first["logits"])   # deterministic
    check_epilogue(g, draft.reshape(-1), R)
    assert g["accept_len"].tolist() == [min(int(p), 2) if s == 5 else int(p) for s, p in enumerate(prefix)]
    assert g["draft_lp"][R - 1::R].tolist() == [0.0] * n_seq
    # the fused outputs do not depend on writing the logits
    h = run(sampler, x, w, draft=d, rows_per_seq=R, logits=False)
    for k in ("argmax_ids", "log_z", "draft_lp", "accept_len"):
        assert np.array_equal(h[k], g[k]), k


def test_padded_logits_rows(sampler):
    """ld_logits > vocab: the padding is left as it was."""
    torch = sampler.torch
    rng = np.random.default_rng(9)
    rows, vocab, hidden = 16, 700, 128
    x = bf16(torch, rng.standard_normal((rows, hidden))).cuda()
    w = bf16(torch, rng.standard_normal((vocab, hidden))).cuda()
    big = torch.full((rows, 768), -3.0, dtype=torch.float32, device="cuda")
    out = {"logits": big[:, :vocab], "argmax_ids": torch.zeros(rows, dtype=torch.int32, device="cuda")}
    sampler.lmhead_dev(x, w, out)
    torch.cuda.synchronize()
    b = big.cpu().numpy()
    assert (b[:, vocab:] == -3.0).all()
    assert np.array_equal(out["argmax_ids"].cpu().numpy(), np.argmax(b[:, :vocab], axis=1))


def test_invalid_arguments_are_rejected(sampler):
    from locus_amd.sampler import SamplerError
    torch = sampler.torch
    x = torch.zeros((4, 96), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((100, 96), dtype=torch.bfloat16, device="cuda")
    out = sampler.alloc_lmhead_out(4, 100)
    with pytest.raises(SamplerError, match="multiple of 64"):
        sampler.lmhead_dev(x, w, out)
    x = torch.zeros((6, 64), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((100, 64), dtype=torch.bfloat16, device="cuda")
    d = torch.zeros(6, dtype=torch.int32, device="cuda")
    out = sampler.alloc_lmhead_out(6, 100, draft=True, n_seq=1)
    with pytest.raises(SamplerError, match="divide rows"):
        sampler.lmhead_dev(x, w, out, draft=d, rows_per_seq=4)
    x = torch.zeros((600, 64), dtype=torch.bfloat16, device="cuda")
    out = sampler.alloc_lmhead_out(600, 100)
    with pytest.raises(SamplerError, match="context limits"):
        sampler.lmhead_dev(x, w, out)


def test_decode_shape_full_size(sampler):
    """B = 64, V = 128256, hidden 4096 (the decode batch of the sampling
    workloads): columns checked against float64 on a sample, the epilogue
    against the whole written logits."""
    torch = sampler.torch
    say("full size 64 x 128256 x 4096")
    gen = torch.Generator(device="cuda").manual_seed(3)
    rows, vocab, hidden = 64, 128256, 4096
    x = torch.randn((rows, hidden), generator=gen, device="cuda").to(torch.bfloat16)
    w = (torch.randn((vocab, hidden), generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    g = run(sampler, x, w)
    cols = np.random.default_rng(0).choice(vocab, 2048, replace=False)
    cols[:2] = [0, vocab - 1]
    x64 = x.double().cpu().numpy()
    w64 = w[torch.from_numpy(cols).cuda()].double().cpu().numpy()
    ref = x64 @ w64.T
    bound = hidden * U * (np.abs(x64) @ np.abs(w64).T)
    assert (np.abs(g["logits"][:, cols] - ref) <= bound).all()
    check_epilogue(g)
