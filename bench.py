"""Benchmark of the HIP sampler on one MI355X.

Default workload: BASELINE.json configs[1] ("c2"): B=64, V=128256 f32
logits ~ N(0, 3^2), 2048-id Zipf history, repeat 1.1 / frequency 0.5 /
presence 0.3, T=0.7, min-p 0.05, top-p 0.9, seeded draw, top-5 logprobs.
A step is one lcs_sample call over one batch with inputs already resident in
HBM; the timed loop rotates through enough distinct input sets (> 2x the
256 MB Infinity Cache) that each call reads its logits from HBM.

Prints one JSON line: rows/s (value), HBM roofline of the sampling kernel,
and the reference CPU sampler timed on this host (cpu_baseline).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from locus_amd import workloads as W  # noqa: E402

METRIC = "sampled rows/sec + achieved HBM GB/s (B=64, V=128256, full sampling chain)"
HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20

# the kernels that do a workload's work (the roofline's subject): a name
# pattern (SQL LIKE) matching them, and the stem of their profile summaries
# ("a|b" matches either)
KERNEL = {"c1g": ("slice_stats|row_fin", "sliced"), "c1s": ("slice_stats|row_fin", "sliced"),
          "c2": ("slice_stats|row_fin", "sliced"), "c2w": ("slice_stats|row_fin", "sliced"),
          "c3": ("nuc_", "nucleus"),
          "c4": ("nuc_", "nucleus"), "c5": ("verify_kernel|accept_kernel", "verify")}


def _like(column, kernel):
    """SQL condition and parameters for a name pattern "a|b" (either)."""
    parts = kernel.split("|")
    return "(" + " or ".join(f"{column} like ?" for _ in parts) + ")", tuple(f"%{k}%" for k in parts)

CONFIG_TEXT = {
    "c1g": "B=1 V=128256 f32 greedy",
    "c1s": "B=1 V=128256 f32 T0.8 top-k40 top-p0.95",
    "c2": "B=64 V=128256 f32 pen(1.1,0.5,0.3,last2048) T0.7 min-p0.05 top-p0.9 top-5 logprobs",
    "c2w": "c2 with N(0,1) logits, T1.5, min-p0.01: wide min-p windows, every row on the exact path "
           "inside row_fin (stress case, not a BASELINE config)",
    "c3": "B=256 V=151936 f32 T1.5 top-p0.98",
    "c4": "B=32 V=128256 f32 JSON-mask T1.0 top-p0.95 top-1 logprob",
    "c5": "4096 rows (512x8) V=163840 bf16 verify: argmax + lp(draft) + accept length",
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gpu_bench(name, steps, warmup):
    import torch

    from locus_amd.sampler import Sampler

    w0 = W.make(name)
    set_bytes = w0.logits.nbytes
    nsets = max(1, min(32, -(-2 * MALL_BYTES // set_bytes) + 1)) if set_bytes < MALL_BYTES else 1
    log(f"[bench] {name}: {nsets} input sets of {set_bytes / 1e6:.1f} MB")
    s = Sampler(device=0, max_rows=max(w0.rows, w0.n_seq or 1), max_vocab=w0.vocab,
                max_hist=4096, max_top=20)
    sets = []
    for k in range(nsets):
        w = w0 if k == 0 else W.make(name, set_index=k)
        d = s.upload(w)
        out = s.alloc_verify_out(w) if w.n_seq else s.alloc_out(w.rows, w.n_top, w.want_logprobs, diag=False)
        sets.append((d, out))
    verify = bool(w0.n_seq)
    stream = torch.cuda.current_stream()
    handle = s.stream_handle(stream)
    # C structs are built once per input set; the timed loop only launches
    launchers = [s.prepare_verify(d, out) if verify else s.prepare(d, out) for d, out in sets]

    def call(i):
        launchers[i % nsets](handle)

    for i in range(warmup):
        call(i)
    torch.cuda.synchronize()
    # (1) whole-job timing: events bracket the K calls on the launch stream
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        call(i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = e0.elapsed_time(e1)
    # (2) per-launch duration: events around each launch on the same stream
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    for i in range(steps):
        starts[i].record(stream)
        call(i)
        ends[i].record(stream)
    torch.cuda.synchronize()
    per = np.array([a.elapsed_time(b) for a, b in zip(starts, ends)])
    assert s.status() == 0, "device status set"
    s.close()
    return w0, ev_ms / steps, wall / steps * 1e3, float(np.median(per)), nsets


def copy_ceiling(mib: int = 1024, reps: int = 10) -> float:
    """Measured HBM ceiling: GB/s of a plain device-to-device copy of `mib` MiB
    (bytes read + bytes written over the copy's time), well past the 256 MB
    Infinity Cache."""
    import torch
    n = mib * (1 << 20) // 4
    a = torch.ones(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    for _ in range(2):
        b.copy_(a)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        b.copy_(a)
    e1.record(stream)
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) / reps * 1e-3
    del a, b
    return 2 * n * 4 / sec / 1e9


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the CPU baseline."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_baseline(name, budget_s=10.0, threads=1):
    """The reference sampler (compiled from the reference's own sources,
    oracle/_ref) on this host, rows in order as the reference engine samples
    them (engine.cpp:541-557) on one thread, or spread over `threads`
    threads; the C++ restatement when the reference build is absent."""
    from oracle import pyoracle as O
    kind = "reference" if O.ref_available() else "port"
    w = W.make(name)
    threads = max(1, min(threads, w.rows))
    rows_done = 0
    t0 = time.perf_counter()
    reps = 0
    while True:
        if w.n_seq:
            O.verify(w, threads=threads)
        elif kind == "reference":
            O.ref_sample_batch(w, threads=threads)
        else:
            O.sample_batch(w, threads=threads)
        rows_done += w.rows
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    if w.n_seq:
        kind = "port"  # the reference has no batched verify; the oracle restates its loop
    return {"value": rows_done / el, "unit": "rows/s", "cores": threads, "kind": kind, "cpu": cpu_model(),
            "sample": f"{reps} x {name} batch ({w.rows} rows, V={w.vocab}), "
                      f"{'single thread' if threads == 1 else f'{threads} threads'}, {el:.1f} s"}


def synthetic_pieces(V: int = 128256, seed: int = 20261204) -> list[bytes]:
    """A tokenizer-like piece table of V entries: the 256 single bytes, then
    pieces of 1-10 bytes mixing word fragments (with and without a leading
    space), digits, JSON punctuation, quotes and escapes."""
    rng = np.random.default_rng(seed)
    pieces = [bytes([b]) for b in range(256)]
    letters = np.frombuffer(b"etaoinshrdlucmfwypvbgkjqxz", dtype=np.uint8)
    punct = [b"{", b"}", b"[", b"]", b":", b",", b'"', b'":', b'",', b'{"', b'"}', b"\\n", b"\\\"", b" {", b"},"]
    while len(pieces) < V:
        k = rng.random()
        if k < 0.70:
            n = int(rng.integers(1, 9))
            w = bytes(letters[np.minimum(rng.geometric(0.12, n) - 1, 25)])
            pieces.append((b" " if rng.random() < 0.5 else b"") + w)
        elif k < 0.82:
            pieces.append(str(int(rng.integers(0, 10 ** int(rng.integers(1, 4))))).encode())
        elif k < 0.95:
            pieces.append(punct[int(rng.integers(0, len(punct)))] + (b" " if rng.random() < 0.3 else b""))
        else:
            pieces.append(bytes(rng.integers(32, 127, int(rng.integers(1, 6))).astype(np.uint8)))
    return pieces[:V]


def mask_bench(budget_s: float = 5.0):
    """Host cost of one JSON allow-mask at V=128256 (the per-step host work of a
    constrained row, server.cpp:160-171): the reference's per-token allows()
    loop (a grammar copy fed each piece; the compiled reference when its build
    is present, else the oracle's restatement) against JsonMaskBuilder (trie
    walk), cold (a state not seen before) and cached (a state seen before),
    over the grammar states of a JSON document fed byte by byte."""
    from locus_amd import host_lib as H
    from oracle import pyoracle as O
    V = 128256
    pieces = synthetic_pieces(V)
    doc = b'{"name": "sampler", "ids": [12, 7, 3005], "ok": true, "nested": {"x": -1.5e3, "s": "a\\"b"}}'
    blob = np.frombuffer(b"".join(pieces), dtype=np.uint8).copy()
    off = np.zeros(len(pieces) + 1, dtype=np.uint64)
    off[1:] = np.cumsum([len(p) for p in pieces])
    out = np.zeros((V + 31) // 32, dtype=np.uint32)
    kind = "reference" if O.ref_available() else "port"
    # (1) per-token allows(): one mask per prefix length until the budget ends
    t0, n_ref = time.perf_counter(), 0
    for i in range(len(doc)):
        pre = np.frombuffer(doc[:i], dtype=np.uint8).copy() if i else np.zeros(1, dtype=np.uint8)
        if kind == "reference":
            rc = O.ref().ref_json_mask(pre.ctypes.data, i, blob.ctypes.data, off.ctypes.data, V, V, out.ctypes.data)
            assert rc == 0
        else:
            g = O.OracleJson()
            assert g.feed_all(doc[:i])
            g.mask(pieces, V)
        n_ref += 1
        if time.perf_counter() - t0 > budget_s:
            break
    ref_ms = (time.perf_counter() - t0) / n_ref * 1e3
    # (2) the trie builder: every state of the document, cold, then again cached
    mb = H.MaskBuilder(pieces, cache_entries=4096)
    states = []
    g = H.JsonGrammar()
    for i in range(len(doc) + 1):
        states.append(g.clone())
        if i < len(doc):
            assert g.feed(doc[i])
    cold, warm = [], []
    for st in states:
        _, m0 = mb.cache_stats()
        t0 = time.perf_counter()
        mb.build(st, V)
        dt = time.perf_counter() - t0
        (cold if mb.cache_stats()[1] > m0 else warm).append(dt)
    for st in states:   # every state again: all from the cache
        t0 = time.perf_counter()
        mb.build(st, V)
        warm.append(time.perf_counter() - t0)
    return {"vocab": V, "states": len(states), "distinct_states": len(cold),
            "allows_loop_ms": ref_ms, "allows_loop_kind": kind, "allows_loop_masks": n_ref,
            "trie_cold_ms": float(np.mean(cold)) * 1e3, "trie_cold_max_ms": float(np.max(cold)) * 1e3,
            "trie_cached_ms": float(np.mean(warm)) * 1e3, "cpu": cpu_model()}


def batch_sampler_bench(steps: int, warmup: int):
    """The serving path's step on C2 (locus_amd/host/batch_bench.cpp, a C++
    program over BatchSampler::sample_step: host staging, uploads,
    lcs_sample, read-back, synchronisation and the per-request updates), next
    to lcs_sample alone on resident inputs (the headline's timed call)."""
    import subprocess
    exe = os.path.join(ROOT, "locus_amd", "batch_bench")
    if not os.path.exists(exe):
        raise SystemExit(f"{exe} is missing: run __graft_entry__.build()")
    runs = []
    for mode in ("windows", "uploads"):
        r = subprocess.run([exe, str(steps), str(warmup), mode], capture_output=True, text=True, timeout=600)
        if r.returncode != 0:
            raise SystemExit(f"batch_bench failed ({r.returncode}): {r.stderr.strip()}")
        runs.append(json.loads(r.stdout.strip().splitlines()[-1]))
    line = runs[0]
    line["uploaded_histories"] = {k: runs[1][k] for k in ("us_per_step", "us_median", "us_p90", "rows_per_s")}
    _, ms_step, _, _, _ = gpu_bench("c2", steps, warmup)
    line["kernel_only_us_per_call"] = ms_step * 1e3
    return line


# phase clocks of the sliced path (the LCS_PROFILE build): slot k of a slice
# workgroup, and of a row's finalize (row_fin), with what precedes it
SLICE_PHASES = ["start", "logits decoded", "raw and tempered sums", "history counted (barrier B1)",
                "reductions, penalised groups listed", "penalties applied, top-n bound",
                "barrier B2", "top-n and window entries collected", "barrier B3", "record stored"]
FIN_CHAIN = [(0, "start"), (4, "parameters and records in"), (24, "window threshold"),
             (25, "window offsets"), (26, "window gathered"), (12, "barrier (all waves' parts in)"),
             (27, "window ranked (4 waves)"), (28, "exact weights"), (29, "top-p / min-p scan"),
             (30, "draw"), (16, "outputs written")]
FIN_OTHER = [(9, "log-normaliser and top-n staged (wave 1)"), (10, "normaliser (wave 2)")]


def phase_clocks(workload: str, rows: int | None, calls: int = 16):
    """Per-phase wall clocks (s_memrealtime, 100 MHz) of the sliced path's
    kernels on `workload`, from the LCS_PROFILE build of the library:
    medians and maxima over workgroups and calls, in us from the call's first
    slice start. Clocks of different XCDs may be offset from each other."""
    import ctypes as C
    import torch

    from locus_amd import build as B
    from locus_amd import sampler as SM
    if not os.path.exists(B.PROFILE_SO):
        raise SystemExit(f"{B.PROFILE_SO} is missing: run __graft_entry__.build()")
    SM.LIB_PATH = B.PROFILE_SO
    L = SM.lib()
    L.lcs_prof_read.restype = C.c_int
    L.lcs_prof_read.argtypes = [C.c_void_p, C.c_uint32]
    ws = [W.make(workload, rows=rows, set_index=k) for k in range(4)]
    s = SM.Sampler(device=0, max_rows=max(w.rows for w in ws), max_vocab=262144, max_hist=4096, max_top=20)
    sets = []
    for w in ws:
        d = s.upload(w)
        out = s.alloc_out(w.rows, w.n_top, w.want_logprobs, diag=False)
        sets.append(s.prepare(d, out))
    h = s.stream_handle()
    kf, nrow = 16384, 4096
    n = (kf + nrow) * 32
    S_, F_ = [], []
    for it in range(calls + 4):
        sets[it % 4](h)
        torch.cuda.synchronize()
        buf = np.zeros(n, dtype=np.uint64)
        if L.lcs_prof_read(buf.ctypes.data, n) != 0:
            raise SystemExit("lcs_prof_read failed")
        if it < 4:
            continue
        r = buf.reshape(-1, 32).astype(np.int64)
        w = ws[it % 4]
        nwg = w.rows * ((w.vocab + 8191) // 8192)
        t0 = r[:nwg, 0].min()
        S_.append((r[:nwg, :10] - t0) / 100.0)
        F_.append((r[kf:kf + w.rows] - t0) / 100.0)
    s.close()
    S, F = np.concatenate(S_), np.concatenate(F_)
    # absolute times (median over workgroups; clocks of different XCDs may be
    # offset) and each phase's own duration in its workgroup (one XCD's clock)
    lines = [f"# phase clocks, workload {workload} ({ws[0].rows} rows), {calls} calls: 'at' = us from the call's "
             "first slice start (median), then the phase's own duration in us (median / p90 / max over "
             "workgroups, or rows for row_fin)",
             "slice_stats phase                                      at   median     p90     max"]
    for k, name in enumerate(SLICE_PHASES):
        d = S[:, k] - S[:, k - 1] if k else S[:, 0] * 0.0
        lines.append(f"  {k}  {name:46s} {np.median(S[:, k]):6.2f}  {np.median(d):6.2f}  "
                     f"{np.percentile(d, 90):6.2f}  {d.max():6.2f}")
    lines.append("row_fin slot (wave 0's chain)                          at   median     p90     max")
    prev = None
    for k, name in FIN_CHAIN:
        d = F[:, k] - F[:, prev] if prev is not None else F[:, k] * 0.0
        lines.append(f"  {k:2d} {name:46s} {np.median(F[:, k]):6.2f}  {np.median(d):6.2f}  "
                     f"{np.percentile(d, 90):6.2f}  {d.max():6.2f}")
        prev = k
    for k, name in FIN_OTHER:
        d = F[:, k] - F[:, 0]
        lines.append(f"  {k:2d} {name:46s} {np.median(F[:, k]):6.2f}  (from start: {np.median(d):.2f} median, "
                     f"{d.max():.2f} max)")
    tot = F[:, 16] - F[:, 0]
    lines.append(f"row_fin per row, start to outputs: median {np.median(tot):.2f}, max {tot.max():.2f}")
    return "\n".join(lines)


EXACT_PHASES = {0: "start", 1: "distinct penalised ids (history sort)", 2: "stats pass (raw max, sums, top-n)",
                3: "maximum penalised candidate", 4: "histogram pass", 5: "prefix sums over bins",
                10: "region search", 11: "compaction: wanted bins + candidate pass",
                12: "compaction: sort of the list", 13: "compaction: regions", 20: "region search",
                21: "narrowing: key range pass", 22: "narrowing: radix step pass", 23: "narrowing: end",
                99: "walks, decision and outputs"}


def exact_clocks(workload: str, rows: int | None, calls: int = 8):
    """Per-phase wall clocks (s_memrealtime, 100 MHz) of the exact path that
    row_fin runs for rows the slice records cannot settle, from the
    LCS_PROFILE build: each phase's time since the row's previous stamp, in
    us, median / max over rows and calls, for the rows whose stamp sequence
    is the most common one."""
    import collections
    import ctypes as C
    import torch

    from locus_amd import build as B
    from locus_amd import sampler as SM
    if not os.path.exists(B.PROFILE_SO):
        raise SystemExit(f"{B.PROFILE_SO} is missing: run __graft_entry__.build()")
    SM.LIB_PATH = B.PROFILE_SO
    L = SM.lib()
    L.lcs_xprof_read.restype = C.c_int
    L.lcs_xprof_read.argtypes = [C.c_void_p, C.c_void_p]
    L.lcs_xprof_clear.restype = C.c_int
    w = W.make(workload, rows=rows)
    s = SM.Sampler(device=0, max_rows=w.rows, max_vocab=262144, max_hist=4096, max_top=20)
    d = s.upload(w)
    run = s.prepare(d, s.alloc_out(w.rows, w.n_top, w.want_logprobs, diag=False))
    h = s.stream_handle()
    seqs = []
    for it in range(calls + 2):
        if L.lcs_xprof_clear() != 0:
            raise SystemExit("lcs_xprof_clear failed")
        run(h)
        torch.cuda.synchronize()
        buf = np.zeros(4096 * 64, dtype=np.uint64)
        cnt = np.zeros(4096, dtype=np.uint32)
        if L.lcs_xprof_read(buf.ctypes.data, cnt.ctypes.data) != 0:
            raise SystemExit("lcs_xprof_read failed")
        if it < 2:
            continue
        t = buf.reshape(4096, 32, 2).astype(np.int64)
        for r in range(w.rows):
            n = int(cnt[r])
            if n:
                seqs.append((tuple(int(x) for x in t[r, :n, 1]), (t[r, :n, 0] - t[r, 0, 0]) / 100.0))
    s.close()
    if not seqs:
        return f"# exact path phase clocks, workload {workload}: no row took the exact path"
    common, nrow = collections.Counter(q for q, _ in seqs).most_common(1)[0]
    T = np.stack([ts for q, ts in seqs if q == common])
    lines = [f"# exact path phase clocks inside row_fin, workload {workload} ({w.rows} rows), {calls} calls: "
             f"{len(seqs)} row finalizes took the exact path, {nrow} with the stamp sequence below",
             "# time since the previous stamp, us: median / max over those rows",
             "  tag  phase                                           median     max"]
    for j, tag in enumerate(common):
        dt = T[:, j] - (T[:, j - 1] if j else 0.0)
        lines.append(f"  {tag:3d}  {EXACT_PHASES.get(tag, str(tag)):46s} {np.median(dt):8.2f}  {dt.max():8.2f}")
    tot = T[:, -1]
    lines.append(f"exact path per row, first to last stamp: median {np.median(tot):.2f}, max {tot.max():.2f}")
    lines.append("# every stamp sequence: rows, first-to-last median / max (us), tags")
    for q, c in collections.Counter(q for q, _ in seqs).most_common():
        tq = np.array([ts[-1] for qq, ts in seqs if qq == q])
        lines.append(f"  {c:4d}  {np.median(tq):8.2f}  {tq.max():8.2f}  {' '.join(str(x) for x in q)}")
    return "\n".join(lines)


def lmhead_rows_sweep(rows_list, vocab: int = 163840, hidden: int = 4096):
    """lcs_lmhead (argmax and log z from the epilogue, no logits written)
    against the unfused pair (torch's bf16 GEMM, i.e. hipBLASLt, to bf16
    logits, then lcs_verify on them) at several row counts: where the fused
    product's one-weight-read-per-64-rows design stops paying."""
    import ctypes as C
    import torch

    from locus_amd import sampler as SM
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(1)
    w = (torch.randn((vocab, hidden), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    L = SM.lib()
    stream = torch.cuda.current_stream()
    out = []
    for rows in rows_list:
        x = torch.randn((rows, hidden), generator=gen, device=dev).to(torch.bfloat16)
        s = SM.Sampler(device=0, max_rows=rows, max_vocab=vocab, max_hist=64, max_top=4)
        h = s.stream_handle(stream)
        am = torch.empty(rows, dtype=torch.int32, device=dev)
        lz = torch.empty(rows, dtype=torch.float32, device=dev)
        steps = max(3, 400 // rows)

        def timed(fn):
            for _ in range(2):
                fn()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(steps):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) / steps * 1e3
        b = SM._LBatch(rows, vocab, hidden, 0, SM._dptr(x), SM._dptr(w), None)
        o = SM._LOut(None, 0, SM._dptr(am), SM._dptr(lz), None, None)
        t_f = timed(lambda: L.lcs_lmhead(s.ctx, C.byref(b), C.byref(o), h))
        lb = torch.empty((rows, vocab), dtype=torch.bfloat16, device=dev)
        dr = torch.zeros(rows, dtype=torch.int32, device=dev)
        dlp = torch.empty(rows, dtype=torch.float32, device=dev)
        acc = torch.empty(rows, dtype=torch.int32, device=dev)
        vb = SM._VBatch(rows, 1, vocab, SM.LCS_BF16, vocab, SM._dptr(lb), SM._dptr(dr))
        vo = SM._VOut(SM._dptr(am), SM._dptr(dlp), SM._dptr(acc))
        t_g = timed(lambda: torch.mm(x, w.t(), out=lb))
        t_v = timed(lambda: L.lcs_verify(s.ctx, C.byref(vb), C.byref(vo), h))
        fl = 2.0 * rows * vocab * hidden
        out.append({"rows": rows, "vocab": vocab, "hidden": hidden, "lcs_lmhead_us": t_f,
                    "lcs_lmhead_tflops": fl / t_f / 1e6, "gemm_us": t_g, "gemm_tflops": fl / t_g / 1e6,
                    "verify_us": t_v, "gemm_plus_verify_us": t_g + t_v})
        s.close()
        del lb, x
        torch.cuda.empty_cache()
    return out


def draft_bench(n_seq: int = 512, ctx_len: int = 4096, ngram: int = 3, max_draft: int = 7,
                steps: int = 200, cpu_seconds: float = 3.0):
    """Batched n-gram drafts on the device (lcs_ngram_draft) for C5's 512
    sequences, each with a 4096-token context over a 64-token alphabet (a
    trailing 3-gram rarely recurs there, so most sequences are searched back
    to their first token), against the reference's per-sequence ngram_draft
    (speculative.cpp:7-28) on one host core."""
    import ctypes as C
    import torch

    from locus_amd import sampler as SM
    from oracle import pyoracle as O
    rng = np.random.default_rng(20261205)
    ctxs = rng.integers(0, 64, (n_seq, ctx_len)).astype(np.int32)
    s = SM.Sampler(device=0, max_rows=n_seq, max_vocab=1024, max_hist=64, max_top=4)
    got, _ = s.ngram_draft(list(ctxs), ngram, max_draft)
    dev = torch.device("cuda", 0)
    off = torch.from_numpy((np.arange(n_seq + 1, dtype=np.uint32) * ctx_len).view(np.int32)).to(dev)
    ids = torch.from_numpy(ctxs.reshape(-1)).to(dev)
    dr = torch.empty((n_seq, max_draft), dtype=torch.int32, device=dev)
    ln = torch.empty(n_seq, dtype=torch.int32, device=dev)
    b = SM._DBatch(n_seq, ngram, max_draft, SM._dptr(off), SM._dptr(ids))
    o = SM._DOut(SM._dptr(dr), SM._dptr(ln))
    L = SM.lib()
    stream = torch.cuda.current_stream()
    h = s.stream_handle(stream)
    for _ in range(10):
        L.lcs_ngram_draft(s.ctx, C.byref(b), C.byref(o), h)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        L.lcs_ngram_draft(s.ctx, C.byref(b), C.byref(o), h)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / steps * 1e3
    s.close()
    kind = "reference" if O.ref_available() else "port"
    t0, reps = time.perf_counter(), 0
    while time.perf_counter() - t0 < cpu_seconds:
        for c in ctxs:
            if kind == "reference":
                out = np.zeros(max_draft, dtype=np.int32)
                O.ref().ref_ngram_draft(c.ctypes.data, ctx_len, ngram, max_draft, out.ctypes.data)
            else:
                O.ngram_draft(c, ngram, max_draft)
        reps += 1
    cpu_us = (time.perf_counter() - t0) / reps * 1e6
    return {"n_seq": n_seq, "ctx_len": ctx_len, "ngram": ngram, "max_draft": max_draft,
            "mean_draft_len": float(np.mean([len(g) for g in got])), "gpu_us_per_call": us,
            "cpu_us_per_batch": cpu_us, "cpu_kind": kind, "cpu_cores": 1, "cpu": cpu_model()}


def lmhead_bench(rows: int = 64, vocab: int = 128256, hidden: int = 4096, steps: int = 50,
                 cpu_seconds: float = 3.0):
    """The fused lm-head product (lcs_lmhead) at the decode shape of C2
    (B = 64, V = 128256) with a 4096-wide hidden state: bf16 x and weight,
    f32 accumulation; timed without and with the f32 logits written, beside
    the unfused path (torch's bf16 GEMM to bf16 logits, then lcs_verify on
    them). The product reads the weight once per launch, so HBM bounds it:
    algorithmic bytes = weight + x + the epilogue's records (written and read
    once) + the per-row outputs."""
    import ctypes as C
    import torch

    from locus_amd import sampler as SM
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn((rows, hidden), generator=gen, device=dev).to(torch.bfloat16)
    w = (torch.randn((vocab, hidden), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    s = SM.Sampler(device=0, max_rows=rows, max_vocab=vocab, max_hist=64, max_top=4)
    stream = torch.cuda.current_stream()
    h = s.stream_handle(stream)
    L = SM.lib()
    am = torch.empty(rows, dtype=torch.int32, device=dev)
    lz = torch.empty(rows, dtype=torch.float32, device=dev)
    lg = torch.empty((rows, vocab), dtype=torch.float32, device=dev)

    def timed(fn):
        for _ in range(5):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps * 1e3

    b = SM._LBatch(rows, vocab, hidden, 0, SM._dptr(x), SM._dptr(w), None)
    o_fused = SM._LOut(None, 0, SM._dptr(am), SM._dptr(lz), None, None)
    o_logits = SM._LOut(SM._dptr(lg), vocab, SM._dptr(am), SM._dptr(lz), None, None)
    us_fused = timed(lambda: L.lcs_lmhead(s.ctx, C.byref(b), C.byref(o_fused), h))
    us_logits = timed(lambda: L.lcs_lmhead(s.ctx, C.byref(b), C.byref(o_logits), h))
    # unfused: library GEMM (bf16 logits), then the verify kernels over them
    lb = torch.empty((rows, vocab), dtype=torch.bfloat16, device=dev)
    dr = torch.zeros(rows, dtype=torch.int32, device=dev)
    dlp = torch.empty(rows, dtype=torch.float32, device=dev)
    acc = torch.empty(rows, dtype=torch.int32, device=dev)
    vb = SM._VBatch(rows, 1, vocab, SM.LCS_BF16, vocab, SM._dptr(lb), SM._dptr(dr))
    vo = SM._VOut(SM._dptr(am), SM._dptr(dlp), SM._dptr(acc))

    def unfused():
        torch.mm(x, w.t(), out=lb)
        L.lcs_verify(s.ctx, C.byref(vb), C.byref(vo), h)
    us_unfused = timed(unfused)
    us_gemm = timed(lambda: torch.mm(x, w.t(), out=lb))
    s.close()
    nblocks = (vocab + 255) // 256
    alg = vocab * hidden * 2 + rows * hidden * 2 + 2 * rows * nblocks * 16 + rows * 8
    alg_logits = alg + rows * vocab * 4
    # CPU: a float32 product of the same shape (numpy's BLAS, all cores) on a
    # sample of the vocabulary, scaled to the whole
    xc = x.float().cpu().numpy()
    cols = min(vocab, 8192)
    wc = w[:cols].float().cpu().numpy()
    t0, reps = time.perf_counter(), 0
    while time.perf_counter() - t0 < cpu_seconds:
        np.dot(xc, wc.T)
        reps += 1
    cpu_us = (time.perf_counter() - t0) / reps * 1e6 * vocab / cols
    return {"workload": f"lm-head {rows} x {vocab} x {hidden} bf16 (f32 accumulation)",
            "us_fused": us_fused, "us_with_logits": us_logits,
            "us_unfused_gemm_plus_verify": us_unfused, "us_library_gemm_alone": us_gemm,
            "roofline": {"bound": "hbm", "algorithmic_bytes": alg,
                         "achieved": alg / (us_fused * 1e-6) / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": alg / (us_fused * 1e-6) / 1e9 / HBM_PEAK_GBS,
                         "with_logits_frac": alg_logits / (us_logits * 1e-6) / 1e9 / HBM_PEAK_GBS},
            "tflops_fused": 2.0 * rows * vocab * hidden / (us_fused * 1e-6) / 1e12,
            "cpu_us_f32_product": cpu_us, "cpu_kind": "numpy f32 matmul", "cpu": cpu_model(),
            "cpu_threads": int(os.environ.get("OMP_NUM_THREADS", "0") or 0)}


def copy_calibration(mib: int, reps: int = 20):
    """A plain device copy of known size (for scaling FETCH_SIZE/WRITE_SIZE:
    each dispatch must read and write exactly `mib` MiB)."""
    import torch
    n = mib * (1 << 20) // 4
    a = torch.ones(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n * 4, "dispatches": reps}), flush=True)


def _db(path):
    import glob
    import sqlite3
    dbs = sorted(glob.glob(os.path.join(path, "**", "*_results.db"), recursive=True)) \
        if os.path.isdir(path) else [path]
    if not dbs:
        raise SystemExit(f"no rocprofv3 database under {path}")
    return sqlite3.connect(dbs[0]), dbs[0]


def summarize_trace(path, kernel):
    """Text summary of a `rocprofv3 --kernel-trace --stats` database: per-kernel
    calls / total / average duration, then the named kernel's average."""
    c, f = _db(path)
    rows = c.execute("select name, total_calls, total_duration, average, percentage "
                     "from top_kernels order by total_duration desc").fetchall()
    out = [f"# source: {os.path.basename(f)} (rocpd database, view top_kernels; durations in us)",
           f"{'calls':>7} {'total_us':>12} {'avg_us':>10} {'pct':>6}  kernel"]
    for name, n, tot, avg, pct in rows[:12]:
        out.append(f"{n:>7} {tot:>12.3f} {avg:>10.3f} {pct:>6.2f}  {name}")
    # one dispatch of each matching kernel per call: the call's kernel time is
    # the sum of their averages
    cond, par = _like("name", kernel)
    ks = c.execute("select name, count(*), avg(duration), min(duration), max(duration) from kernels "
                   f"where {cond} group by name", par).fetchall()
    meds = []
    for name, n, avg, mn, mx in ks:
        d = np.array([r[0] for r in c.execute("select duration from kernels where name = ?", (name,))])
        meds.append(float(np.median(d)))
        out.append(f"kernel_avg_us[{name}]: {avg / 1e3:.3f}  (n={n}, median {meds[-1] / 1e3:.3f}, "
                   f"min {mn / 1e3:.3f}, max {mx / 1e3:.3f})")
    out.append(f"call_kernel_avg_us[{kernel}]: {sum(k[2] for k in ks) / 1e3:.3f}  ({len(ks)} kernel(s) per call)")
    # (the first dispatches of a process include one-time costs; the median
    # is the steady state the timed region sees)
    out.append(f"call_kernel_median_us[{kernel}]: {sum(meds) / 1e3:.3f}")
    return "\n".join(out)


def _pmc_avg(path, kernel, counter):
    """Per-call reading of `counter`: the sum over the kernels matching
    `kernel` of each one's average per dispatch."""
    c, _ = _db(path)
    cond, par = _like("kernel_name", kernel)
    rs = c.execute("select kernel_name, count(*), avg(value) from counters_collection "
                   f"where {cond} and counter_name = ? group by kernel_name",
                   par + (counter,)).fetchall()
    if not rs:
        raise SystemExit(f"{counter} for {kernel} not found in {path}")
    return min(r[1] for r in rs), float(sum(r[2] for r in rs))


def summarize_counters(path, kernel):
    """Per-kernel average per dispatch of every counter in a `rocprofv3 --pmc`
    database, for the kernels matching `kernel`."""
    c, f = _db(path)
    cond, par = _like("kernel_name", kernel)
    rs = c.execute("select kernel_name, counter_name, count(*), avg(value) from counters_collection "
                   f"where {cond} group by kernel_name, counter_name "
                   "order by kernel_name, counter_name", par).fetchall()
    out = [f"# source: {os.path.basename(f)} (counters_collection; average per dispatch)"]
    for kname, cname, n, avg in rs:
        out.append(f"{cname:<24} {avg:>16.1f}  (n={n})  {kname}")
    return "\n".join(out)


def summarize_traffic(kernel, fetch, write, copy_fetch, copy_write, copy_bytes):
    """HBM traffic per dispatch of `kernel` from FETCH_SIZE / WRITE_SIZE passes
    (KiB per dispatch), each scaled by the same counter's reading for a plain
    device copy of `copy_bytes` bytes (reads and writes exactly that much)."""
    nf, kf = _pmc_avg(fetch, kernel, "FETCH_SIZE")
    nw, kw = _pmc_avg(write, kernel, "WRITE_SIZE")
    _, cf = _pmc_avg(copy_fetch, "copyBuffer", "FETCH_SIZE")
    _, cw = _pmc_avg(copy_write, "copyBuffer", "WRITE_SIZE")
    sf, sw = copy_bytes / (cf * 1024), copy_bytes / (cw * 1024)
    rb, wb = kf * 1024 * sf, kw * 1024 * sw
    return "\n".join([
        f"copy calibration: {copy_bytes} B copied; FETCH_SIZE {cf:.1f} KiB -> scale {sf:.4f}; "
        f"WRITE_SIZE {cw:.1f} KiB -> scale {sw:.4f}",
        f"{kernel}: FETCH_SIZE {kf:.1f} KiB/dispatch (n={nf}), WRITE_SIZE {kw:.1f} KiB/dispatch (n={nw})",
        f"read_bytes_per_launch: {rb:.0f}",
        f"write_bytes_per_launch: {wb:.0f}",
        f"traffic_bytes_per_launch: {rb + wb:.0f}",
    ])


def committed_traffic(stem, workload):
    """traffic_bytes_per_launch from the committed counter summary, if any."""
    f = os.path.join(ROOT, "profiles", f"{stem}_{workload}_traffic.txt")
    if not os.path.exists(f):
        return None
    for line in open(f):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":")[1])
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c2", choices=sorted(CONFIG_TEXT))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="only run a plain copy of MIB MiB (counter calibration)")
    ap.add_argument("--summarize-trace", metavar="DIR",
                    help="print a text summary of a rocprofv3 --kernel-trace --stats output")
    ap.add_argument("--summarize-traffic", nargs=4,
                    metavar=("FETCH_DIR", "WRITE_DIR", "COPY_FETCH_DIR", "COPY_WRITE_DIR"),
                    help="print HBM traffic per launch from four rocprofv3 --pmc outputs")
    ap.add_argument("--summarize-counters", metavar="DIR",
                    help="print per-kernel averages of every counter of a rocprofv3 --pmc output")
    ap.add_argument("--cpu-threads", type=int, default=int(os.environ.get("OMP_NUM_THREADS", "16")),
                    help="threads of the all-cores CPU baseline (0: skip it)")
    ap.add_argument("--kernel", default="slice_stats|row_fin")
    ap.add_argument("--copy-bytes", type=int, default=256 << 20)
    ap.add_argument("--mask-bench", action="store_true",
                    help="only time the host JSON allow-mask at V=128256 (CPU)")
    ap.add_argument("--draft-bench", action="store_true",
                    help="only time batched n-gram drafts on the device against the CPU reference")
    ap.add_argument("--lmhead-bench", action="store_true",
                    help="only time the fused lm-head product at the decode shape")
    ap.add_argument("--lmhead-rows", default=None, metavar="R1,R2,..",
                    help="only time lcs_lmhead against GEMM + lcs_verify at these row counts (V=163840, hidden 4096)")
    ap.add_argument("--batch-sampler", action="store_true",
                    help="only time the engine's batched step (BatchSampler::sample_step) end to end on C2")
    ap.add_argument("--phase-clocks", action="store_true",
                    help="only print the sliced path's phase clocks (the LCS_PROFILE build) on --workload")
    ap.add_argument("--exact-clocks", action="store_true",
                    help="only print the phase clocks of row_fin's exact path (the LCS_PROFILE build) on "
                         "--workload (c2w sends every row there)")
    ap.add_argument("--rows", type=int, default=None, help="rows of the workload (--phase-clocks, --exact-clocks)")
    args = ap.parse_args()
    if args.phase_clocks:
        print(phase_clocks(args.workload, args.rows))
        return
    if args.exact_clocks:
        print(exact_clocks(args.workload, args.rows))
        return
    if args.batch_sampler:
        print(json.dumps(batch_sampler_bench(args.steps, args.warmup)))
        return
    if args.lmhead_bench:
        print(json.dumps(lmhead_bench()))
        return
    if args.lmhead_rows:
        for r in lmhead_rows_sweep([int(v) for v in args.lmhead_rows.split(",")]):
            print(json.dumps(r), flush=True)
        return
    if args.mask_bench:
        print(json.dumps(mask_bench()))
        return
    if args.draft_bench:
        print(json.dumps(draft_bench()))
        return
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace, args.kernel))
        return
    if args.summarize_counters:
        print(summarize_counters(args.summarize_counters, args.kernel))
        return
    if args.summarize_traffic:
        print(summarize_traffic(args.kernel, *args.summarize_traffic, args.copy_bytes))
        return
    if args.copy_calib:
        copy_calibration(args.copy_calib)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for {args.gpus}); "
              "a batch's rows would shard across GPUs with no exchange between them", file=sys.stderr)
        sys.exit(2)
    w, ms_step, wall_ms, ms_launch, nsets = gpu_bench(args.workload, args.steps, args.warmup)
    ceiling = copy_ceiling()
    rows = w.rows
    alg = w.algorithmic_bytes()
    # the timed region's average call duration (two kernels per call on the
    # sliced and verify paths, three on the nucleus path: their sum is the call)
    achieved = alg / (ms_step * 1e-3) / 1e9
    kernel, stem = KERNEL[args.workload]
    traffic = committed_traffic(stem, args.workload)
    line = {
        "metric": METRIC,
        "value": rows / (ms_step * 1e-3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if w.dtype == "bf16" else "f32",
        "data": "synthetic",
        "config": {"workload": f"{args.workload}: {CONFIG_TEXT[args.workload]}",
                   "rows": rows, "vocab": w.vocab, "input_sets": nsets},
        "hbm_gbps": alg / (ms_step * 1e-3) / 1e9,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "kernel": kernel, "algorithmic_bytes": alg, "us_per_launch": ms_step * 1e3,
                     "us_per_launch_bracketed_median": ms_launch * 1e3,
                     "traffic_source": f"profiles/{stem}_{args.workload}_traffic.txt"
                     if traffic is not None else None,
                     "copy_ceiling": ceiling, "frac_of_copy": achieved / ceiling},
        "wall_ms_per_step": wall_ms,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.workload, args.cpu_seconds)
        if args.cpu_threads > 1 and w.rows > 1:
            line["cpu_baseline_all_cores"] = cpu_baseline(args.workload, args.cpu_seconds, args.cpu_threads)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
