#!/usr/bin/env python3
"""Benchmark of the depthwise causal conv1d hot path on one MI355X.

Workload (benchmark configuration C2, the one the headline metric is quoted on):
  C2: x (4, 5120, 2048) bf16 channel-first, weight (5120, 4), bias (5120),
      SiLU, dout N(0,1); one step = forward + backward through the public API
      (causal_conv1d_fn + torch.autograd.grad); one HIP graph holds one step per
      rotating buffer set, so that the step time is GPU time.

Reported (one JSON line):
  value        step throughput in GB/s = algorithmic bytes of the forward and
               backward kernels (167,823,360 + 251,811,840 B) / step time
  roofline     for the dominant kernel (the fused backward): algorithmic bytes
               per launch / median launch duration, measured here with HIP
               events around a graph of back-to-back launches, vs 8 TB/s.
               `traffic` (HBM bytes per launch) is read from the rocprofv3
               --pmc summary committed in profiles/ when present.
  kernels      every kernel at every benchmark configuration: median, min and
               max microseconds per launch over --runs timed graph replays
               (spread = (max - min) / min), algorithmic GB/s and fraction of
               8 TB/s at the median. C2 forward / backward / autograd
               backward; C3a / C3b channel-last (seq_idx / states) forward,
               backward and autograd backward; C5 (8, 2048, 16384) for fp32,
               fp16 and bf16 at widths 2, 3, 4; the decode updates C4a and C4b
               with the bandwidth floors of their access patterns beside them
               (a plain copy of the same bytes, the same scattered rows or
               state-line chunks without arithmetic); the varlen state gather.
  cpu_baseline the CPU oracle (C restatement of the reference's CPU kernels,
               OpenMP) on a bounded sample of C2, on this host; beside it the
               reference's pure-PyTorch baseline (F.conv1d + F.silu, autograd)
               on the same sample.

Input sets rotate so that the bytes a kernel touches between two reuses of a
buffer set exceed the 256 MB Infinity Cache, so every launch streams from HBM:
C2 4 sets (>= 504 MB between reuses), C3 4 sets (>= 403 MB), C4a 42 sets
(>= 537 MB), C4b 5 sets (>= 671 MB of whole state lines), C5 one set of 1-3 GB.

Modes: --mode bench (default), --mode kernels (eager launch loop of every
kernel and floor above, for rocprofv3 --kernel-trace / --pmc; --no-configs
keeps only C2 and C4a), --mode copy (a plain 1 GiB device copy, the
calibration kernel for FETCH_SIZE / WRITE_SIZE).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "causal-conv1d-mojo_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "fwd/bwd achieved HBM GB/s (% peak) at B4×D5120×L2048 bf16; update µs/call"
HBM_PEAK_GBPS = 8000.0
MALL_BYTES = 256 * 2 ** 20
B, D, L, W = 4, 5120, 2048, 4
# algorithmic bytes: every input read once, every output written once
FWD_BYTES = 2 * B * D * L * 2 + D * W * 2 + D * 2                      # 167,823,360
BWD_BYTES = 3 * B * D * L * 2 + D * W * 2 + D * 2 + D * W * 4 + D * 4  # 251,811,840
# autograd backward: the same kernel, dweight / dbias written once in bf16 by the reduction
BWD_TYPED_BYTES = 3 * B * D * L * 2 + D * W * 2 + D * 2 + D * W * 2 + D * 2
UPD_B, UPD_POOL = 256, 512
UPD_BYTES = UPD_B * D * (2 + 6 + 6 + 2) + D * W * 2 + D * 2 + UPD_B * 4  # 21,023,744
UPD_TOUCHED = UPD_B * D * (2 + 6 + 2)  # distinct bytes a call touches: x, its state rows, out
C4B_S = 64
C4B_BYTES = UPD_B * D * (8 + 6 + 8 + 8) + D * W * 2 + D * 2 + 2 * UPD_B * 4  # 39,374,848
C4B_LINE_BYTES = UPD_B * D * 128  # whole 128-byte state lines under the touched chunks

FLOOR_LIB = ROOT / "libcc1d_floor.so"  # built by csrc/build.py from csrc/bench/cc1d_floor.hip


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def _parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--mode", choices=["bench", "kernels", "copy"], default="bench")
    ap.add_argument("--launches", type=int, default=40, help="launches per kernel timing graph")
    ap.add_argument("--runs", type=int, default=5, help="timed graph replays per kernel (min / median / max)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the C3/C4b/C5/varlen report lines")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="target duration of each CPU-baseline leg")
    ap.add_argument("--settle", type=float, default=0.3,
                    help="seconds of untimed C2 kernels before the first timing (clock ramp)")
    ap.add_argument("--kernel-settle", type=float, default=0.05,
                    help="seconds of untimed replays of each per-kernel timing graph (clock ramp)")
    return ap.parse_args()


# ------------------------------------------------------------------ timing helpers


def _graph(torch, fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def _replay_times(torch, g, runs):
    """Milliseconds of each of `runs` replays of g (HIP events on torch's current stream,
    which is where graph replays run), after one untimed replay."""
    g.replay()
    torch.cuda.synchronize()
    out = []
    for _ in range(runs):
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        g.replay()
        t1.record()
        torch.cuda.synchronize()
        out.append(t0.elapsed_time(t1))
    return out


def _time_launch_set(torch, fns, launches, runs, settle):
    """Microseconds per launch, one value per run, of a graph of `launches` launches
    cycling through the closures `fns` (one per rotating buffer set), after `settle`
    seconds of untimed replays: the host-side set-up between two cases leaves the GPU
    idle, and for tens of ms after that it runs below its steady clocks (the C2
    backward measured 48.6 us per launch straight after its set-up and 43.5 us after
    50 ms of replays, in one process)."""
    def loop():
        for i in range(launches):
            fns[i % len(fns)]()
    g = _graph(torch, loop)
    t_end = time.perf_counter() + settle
    while time.perf_counter() < t_end:
        g.replay()
        torch.cuda.synchronize()
    us = [ms * 1e3 / launches for ms in _replay_times(torch, g, runs)]
    del g
    return us


def _entry(us_runs, nbytes, **extra):
    """Report fields of one kernel: median / min / max us per launch over the runs,
    spread, algorithmic GB/s and fraction of 8 TB/s at the median."""
    med = statistics.median(us_runs)
    mn, mx = min(us_runs), max(us_runs)
    gbps = nbytes / (med * 1e-6) / 1e9
    return {"us_per_launch": round(med, 2), "us_min": round(mn, 2), "us_max": round(mx, 2),
            "spread_pct": round((mx - mn) / mn * 100.0, 2), "runs": len(us_runs),
            "algorithmic_bytes": int(nbytes), "gbps": round(gbps, 1), "frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4),
            **extra}


def _pmc(kernel, key="hbm_bytes_per_launch"):
    """A field of the committed rocprofv3 --pmc summary (profiles/pmc_summary.json), or None."""
    p = ROOT / "profiles" / "pmc_summary.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get(kernel, {}).get(key)
    except (ValueError, OSError):
        return None


class Floors:
    """ctypes binding of the bench's floor kernels (csrc/bench/cc1d_floor.hip)."""

    def __init__(self):
        if not FLOOR_LIB.exists():
            raise RuntimeError(f"{FLOOR_LIB} is not built; run `python causal-conv1d-mojo_amd/csrc/build.py`")
        lib = ctypes.CDLL(str(FLOOR_LIB))
        i64, i32, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
        lib.cc1d_floor_copy.argtypes = [vp, vp, i64, vp]
        lib.cc1d_floor_rows.argtypes = [vp, vp, vp, vp, i64, i64, i64, i64, i32, vp]
        lib.cc1d_floor_chunks.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i32, i32, i32, vp]
        lib.cc1d_floor_tiles.argtypes = [vp, vp, vp, i64, i64, i32, vp]
        lib.cc1d_floor_walk.argtypes = [vp, vp, vp, i64, i64, vp]
        for f in (lib.cc1d_floor_copy, lib.cc1d_floor_rows, lib.cc1d_floor_chunks, lib.cc1d_floor_tiles,
                  lib.cc1d_floor_walk):
            f.restype = i32
        self.lib = lib

    @staticmethod
    def _check(rc, name):
        if rc != 0:
            raise RuntimeError(f"{name} failed ({rc})")

    def copy(self, torch, src, dst):
        self._check(self.lib.cc1d_floor_copy(src.data_ptr(), dst.data_ptr(), src.numel() * src.element_size() // 16,
                                             torch.cuda.current_stream().cuda_stream), "cc1d_floor_copy")

    def rows(self, torch, x, out, pool, idx, ratio):
        xvec = x.shape[1] * x.element_size() // 16
        self._check(self.lib.cc1d_floor_rows(x.data_ptr(), out.data_ptr(), pool.data_ptr(), idx.data_ptr(),
                                             x.shape[0], xvec, pool[0].numel() * pool.element_size() // 16,
                                             pool.shape[0], ratio, torch.cuda.current_stream().cuda_stream),
                    "cc1d_floor_rows")

    def tiles(self, torch, x, g, out, seg):
        """x, g, out: (rows, row) tensors, contiguous rows"""
        self._check(self.lib.cc1d_floor_tiles(x.data_ptr(), g.data_ptr(), out.data_ptr(), x.shape[0],
                                              x.shape[1] * x.element_size(), seg,
                                              torch.cuda.current_stream().cuda_stream), "cc1d_floor_tiles")

    def walk(self, torch, x, g, out):
        """x, g, out: (rows, row) tensors, contiguous rows; rows a multiple of 1024"""
        self._check(self.lib.cc1d_floor_walk(x.data_ptr(), g.data_ptr(), out.data_ptr(), x.shape[0],
                                             x.shape[1] * x.element_size(), torch.cuda.current_stream().cuda_stream),
                    "cc1d_floor_walk")

    def chunks(self, torch, x, out, pool, idx, cs, nchunks, gran=1):
        """gran 1: the nchunks 16-byte chunks; 4 / 8: the whole 64-byte sectors / 128-byte lines
        holding them"""
        line_chunks = pool.shape[2] * pool.element_size() // 16
        xwords = x.shape[2] * x.element_size() // 4
        self._check(self.lib.cc1d_floor_chunks(x.data_ptr(), out.data_ptr(), pool.data_ptr(), idx.data_ptr(),
                                               cs.data_ptr(), x.shape[0], x.shape[1], line_chunks,
                                               pool[0].numel() * pool.element_size() // 16, pool.shape[0],
                                               nchunks, xwords, gran, torch.cuda.current_stream().cuda_stream),
                    "cc1d_floor_chunks")


# ------------------------------------------------------------------ C2 step (value)


def _c2_sets(torch, n):
    sets = []
    for i in range(n):
        g = torch.Generator(device="cuda").manual_seed(100 + i)
        x = torch.randn(B, D, L, generator=g, device="cuda").bfloat16()
        dout = torch.randn(B, D, L, generator=g, device="cuda").bfloat16()
        sets.append((x, dout))
    g = torch.Generator(device="cuda").manual_seed(0)
    w = torch.randn(D, W, generator=g, device="cuda").bfloat16()
    b = torch.randn(D, generator=g, device="cuda").bfloat16()
    return sets, w, b


def bench_step(torch, cc, args, sets, w, b):
    nsets = len(sets)
    params = [w.detach().requires_grad_(), b.detach().requires_grad_()]

    def make_step(x, dout):
        xl = x.requires_grad_()

        def step():
            out = cc.causal_conv1d_fn(xl, params[0], params[1], activation="silu")
            torch.autograd.grad(out, (xl, params[0], params[1]), dout)

        return step

    # One graph holds one step per buffer set, so a replay runs `nsets` steps back to
    # back and the host's per-replay launch cost (about one step's worth here) is
    # paid once per `nsets` steps; single-step graphs cover a remainder.
    steps = [make_step(x, dout) for x, dout in sets]

    def all_sets():
        for st in steps:
            st()

    multi = _graph(torch, all_sets)
    singles = [_graph(torch, st) for st in steps]
    full, rest = divmod(args.steps, nsets)
    wfull, wrest = divmod(args.warmup, nsets)
    # Untimed pre-roll: after an idle period the GPU runs below its steady clocks
    # for tens of ms, so the graph is replayed for `--settle` seconds first.
    t_end = time.perf_counter() + args.settle
    rolls = 0
    while time.perf_counter() < t_end:
        for _ in range(8):
            multi.replay()
        torch.cuda.synchronize()
        rolls += 8
    log(f"settle: {rolls * nsets} untimed steps in {args.settle:.2f} s")
    for _ in range(wfull):
        multi.replay()
    for i in range(wrest):
        singles[i].replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t0.record()
    for _ in range(full):
        multi.replay()
    for i in range(rest):
        singles[i].replay()
    t1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = t0.elapsed_time(t1) / args.steps
    log(f"step: {ms * 1e3:.1f} us/step over {args.steps} steps ({nsets} buffer sets, {nsets} steps per graph "
        f"replay, wall {wall:.3f} s)")
    del multi, singles
    return ms


# ------------------------------------------------------------------ kernel cases


def _c2_cases(torch, sets, w, b):
    """C2 forward, backward (the reference-shaped op: fp32 accumulators) and the autograd
    backward (typed gradients: backward kernel + fixed-order reduction)."""
    ops = torch.ops.causal_conv1d_amd
    dw = torch.zeros(D, W, dtype=torch.float32, device="cuda")
    db = torch.zeros(D, dtype=torch.float32, device="cuda")
    dwt = torch.empty(D, W, dtype=torch.bfloat16, device="cuda")
    dbt = torch.empty(D, dtype=torch.bfloat16, device="cuda")
    bufs = [(x.detach(), dout, torch.empty_like(x), torch.empty_like(x)) for x, dout in sets]
    return {
        "fwd": ([lambda x=x, o=o: ops._fwd_inplace(x, w, b, None, None, o, True, None) for x, _, o, _ in bufs],
                FWD_BYTES, 1, {}),
        "bwd": ([lambda x=x, d=d, dx=dx: ops._bwd_full_inplace(x, w, b, d, None, None, dx, dw, db, None, True)
                 for x, d, _, dx in bufs], BWD_BYTES, 1, {"op": "_bwd_full_inplace (fp32 accumulators)"}),
        "bwd_typed": ([lambda x=x, d=d, dx=dx: ops._bwd_typed_inplace(x, w, b, d, None, None, None, dx, dwt, dbt,
                                                                       None, True)
                       for x, d, _, dx in bufs], BWD_TYPED_BYTES, 1,
                      {"op": "_bwd_typed_inplace (the autograd backward: bwd_rows_vec + bwd_reduce)"}),
    }


def _c2_seq_cases(torch, sets, w, b):
    """C2's shape with seq_idx: every batch row packs 8 sequences of random lengths (7 uniform
    split points, C3's pattern), so each row's kernels run the id-gated arithmetic."""
    ops = torch.ops.causal_conv1d_amd
    g = torch.Generator().manual_seed(5)
    seq = torch.zeros(B, L, dtype=torch.int32)
    for r in range(B):
        cuts = torch.sort(torch.randperm(L - 1, generator=g)[:7] + 1).values
        for i, c in enumerate(cuts.tolist()):
            seq[r, c:] = i + 1
    seq = seq.cuda()
    dw = torch.zeros(D, W, dtype=torch.float32, device="cuda")
    db = torch.zeros(D, dtype=torch.float32, device="cuda")
    dwt = torch.empty(D, W, dtype=torch.bfloat16, device="cuda")
    dbt = torch.empty(D, dtype=torch.bfloat16, device="cuda")
    bufs = [(x.detach(), dout, torch.empty_like(x), torch.empty_like(x)) for x, dout in sets]
    sb = B * L * 4
    note = {"workload": "C2 shape (4 x 5120 x 2048 bf16, W4, bias, SiLU) with seq_idx: 8 sequences per row"}
    return {
        "fwd_seq": ([lambda x=x, o=o: ops._fwd_inplace(x, w, b, seq, None, o, True, None) for x, _, o, _ in bufs],
                    FWD_BYTES + sb, 1, note),
        "bwd_seq": ([lambda x=x, d=d, dx=dx: ops._bwd_full_inplace(x, w, b, d, seq, None, dx, dw, db, None, True)
                     for x, d, _, dx in bufs], BWD_BYTES + sb, 1, note),
        "bwd_typed_seq": ([lambda x=x, d=d, dx=dx: ops._bwd_typed_inplace(x, w, b, d, seq, None, None, dx, dwt, dbt,
                                                                           None, True)
                           for x, d, _, dx in bufs], BWD_TYPED_BYTES + sb, 1, note),
    }


LR = L - 7  # 2041: not a multiple of the 8-element (16-byte) vector


def _c2_ragged_cases(torch, w, b, nsets=4):
    """C2's shape at seqlen 2041: contiguous rows of an odd length start at every offset inside
    their 16-byte vector, so the row kernels' ragged instantiation runs (own buffer sets, as
    many as C2's)."""
    ops = torch.ops.causal_conv1d_amd
    bufs = []
    for i in range(nsets):
        g = torch.Generator(device="cuda").manual_seed(300 + i)
        x = torch.randn(B, D, LR, generator=g, device="cuda").bfloat16()
        dout = torch.randn(B, D, LR, generator=g, device="cuda").bfloat16()
        bufs.append((x, dout, torch.empty_like(x), torch.empty_like(x)))
    dw = torch.zeros(D, W, dtype=torch.float32, device="cuda")
    db = torch.zeros(D, dtype=torch.float32, device="cuda")
    dwt = torch.empty(D, W, dtype=torch.bfloat16, device="cuda")
    dbt = torch.empty(D, dtype=torch.bfloat16, device="cuda")
    act = B * D * LR * 2  # one activation tensor
    fwd_bytes = 2 * act + D * W * 2 + D * 2
    bwd_bytes = 3 * act + D * W * 2 + D * 2 + D * W * 4 + D * 4
    typed_bytes = 3 * act + D * W * 2 + D * 2 + D * W * 2 + D * 2
    note = {"workload": f"C2 shape at seqlen {LR} (4 x 5120 x {LR} bf16, W4, bias, SiLU): ragged rows"}
    return {
        "fwd_ragged": ([lambda x=x, o=o: ops._fwd_inplace(x, w, b, None, None, o, True, None)
                        for x, _, o, _ in bufs], fwd_bytes, 1, note),
        "bwd_ragged": ([lambda x=x, d=d, dx=dx: ops._bwd_full_inplace(x, w, b, d, None, None, dx, dw, db, None,
                                                                       True)
                        for x, d, _, dx in bufs], bwd_bytes, 1, note),
        "bwd_typed_ragged": ([lambda x=x, d=d, dx=dx: ops._bwd_typed_inplace(x, w, b, d, None, None, None, dx,
                                                                              dwt, dbt, None, True)
                              for x, d, _, dx in bufs], typed_bytes, 1, note),
    }


def _c2_floor_cases(torch, sets, floors):
    """The C2 backward's streams with no arithmetic: x and dout read, dx written, on the
    same sets viewed as (B * D) rows of 4 KB: a wavefront per 4 rows x 1 KB, or per row
    (4 KB, the backward kernel's own item), 16 bytes per lane per load; and the forward's
    streams (x read, out written) as a plain copy."""
    bufs = [(x.detach().reshape(B * D, L), dout.reshape(B * D, L), torch.empty(B * D, L, dtype=x.dtype,
                                                                                 device=x.device))
            for x, dout in sets]
    cases = {f"floor_tiles{seg}_c2": ([lambda u=u, seg=seg: floors.tiles(torch, u[0], u[1], u[2], seg) for u in bufs],
                                      3 * B * D * L * 2, 1, {}) for seg in (1024, 4096)}
    # the forward's streams: x read, out written, one 16-byte vector per lane
    cases["floor_copy_c2"] = ([lambda u=u: floors.copy(torch, u[0], u[2]) for u in bufs], 2 * B * D * L * 2, 1,
                              {"note": "plain copy of x into out (the forward's bytes), no arithmetic"})
    return cases


def _update_sets(torch, n, seqlen=1, S=W - 1, seed=7):
    sets = []
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(D, W, generator=g, device="cuda").bfloat16()
    b = torch.randn(D, generator=g, device="cuda").bfloat16()
    for _ in range(n):
        x = torch.randn(UPD_B, D, seqlen, generator=g, device="cuda").bfloat16()
        pool = torch.randn(UPD_POOL, D, S, generator=g, device="cuda").bfloat16()
        idx = torch.randperm(UPD_POOL, generator=g, device="cuda")[:UPD_B].to(torch.int32)
        cs = torch.randint(0, C4B_S, (UPD_B,), generator=g, device="cuda", dtype=torch.int32)
        sets.append((x, pool, idx, cs, torch.empty_like(x)))
    return sets, w, b


def _c4a_cases(torch, cc, floors):
    """C4a decode (linear, one token) and its floors, over enough rotating sets that the
    bytes touched between two reuses of a set exceed twice the Infinity Cache."""
    nsets = -(-2 * MALL_BYTES // UPD_TOUCHED) + 1  # 42
    sets, w, b = _update_sets(torch, nsets)
    upd = cc._native.native_update
    cases = {
        "update_c4a": ([lambda u=u: upd(u[0], w, b, u[1], u[2], None, u[4], True) for u in sets], UPD_BYTES, 1,
                       {"workload": "C4a: x (256,5120,1) bf16, pool (512,5120,3), 256 random rows, W4, bias, SiLU",
                        "buffer_sets": nsets,
                        "bytes_between_reuses": (nsets - 1) * UPD_TOUCHED}),
        "update_c4a_cache_resident": ([lambda u=sets[0]: upd(u[0], w, b, u[1], u[2], None, u[4], True)], UPD_BYTES,
                                      1, {"note": "one buffer set reused every call (a decode loop over one layer)"}),
    }
    if floors is not None:
        # a plain copy of the same bytes (10.5 MB read, 10.5 MB written), rotating as the update does
        half = UPD_BYTES // 2 // 16 * 16
        cp = [(torch.empty(half, dtype=torch.uint8, device="cuda").fill_(1),
               torch.empty(half, dtype=torch.uint8, device="cuda")) for _ in range(nsets)]
        cases["floor_copy_c4a"] = ([lambda a=a, c=c: floors.copy(torch, a, c) for a, c in cp], 2 * half, 1,
                                   {"note": "plain copy of the update's bytes, one 16-byte vector per lane"})
        cases["runtime_copy_c4a"] = ([lambda a=a, c=c: c.copy_(a) for a, c in cp], 2 * half, 1,
                                     {"note": "the runtime's own device-to-device copy (torch copy_, a memcpy node "
                                              "in the graph) of the same bytes"})
        cases["floor_rows_c4a"] = ([lambda u=u: floors.rows(torch, u[0][..., 0], u[4][..., 0], u[1], u[2], W - 1)
                                    for u in sets], UPD_BYTES, 1,
                                   {"note": "the update's scattered rows without arithmetic: x row and pool row "
                                            "idx[b] read, out row and pool row written, all coalesced"})
    return cases


def _c3_cases(torch, floors=None):
    ops = torch.ops.causal_conv1d_amd
    cases = {}
    # C3: stored (1, 8192, 4096) bf16 channel-last, viewed (1, 4096, 8192); W4, SiLU, no bias
    L3, D3 = 8192, 4096
    sets = []
    g = torch.Generator(device="cuda").manual_seed(3)
    w3 = torch.randn(D3, W, generator=g, device="cuda").bfloat16()
    cuts = torch.sort(torch.randperm(L3 - 1, generator=torch.Generator().manual_seed(0))[:7] + 1).values
    seq = torch.zeros(1, L3, dtype=torch.int32)
    for i, c in enumerate(cuts.tolist()):
        seq[:, c:] = i + 1
    seq = seq.cuda()
    init = torch.randn(1, D3, W - 1, generator=g, device="cuda").bfloat16()
    for _ in range(4):
        x = torch.randn(1, L3, D3, generator=g, device="cuda").bfloat16().transpose(1, 2)
        dout = torch.randn(1, L3, D3, generator=g, device="cuda").bfloat16().transpose(1, 2)
        sets.append((x, dout, torch.empty_like(x), torch.empty_like(x)))
    dw3 = torch.zeros(D3, W, dtype=torch.float32, device="cuda")
    dw3t = torch.empty(D3, W, dtype=torch.bfloat16, device="cuda")
    fs = torch.empty(1, D3, W - 1, dtype=torch.bfloat16, device="cuda")
    di = torch.empty_like(init)
    n3 = L3 * D3 * 2
    for name, kw_f, kw_b, extra_f, extra_b, extra_t in (
            ("c3a", (seq, None, None), (seq, None), 32768 + D3 * W * 2, 2 * 32768 + D3 * W * 2 + D3 * W * 4,
             2 * 32768 + 2 * D3 * W * 2),
            ("c3b", (None, init, fs), (None, init), D3 * W * 2 + 2 * 24576, D3 * W * 2 + D3 * W * 4 + 2 * 24576,
             2 * D3 * W * 2 + 2 * 24576)):
        s_, i_, f_ = kw_f
        fns = [lambda x=x, o=o, s_=s_, i_=i_, f_=f_: ops._fwd_inplace(x, w3, None, s_, i_, o, True, f_)
               for x, _, o, _ in sets]
        cases[f"{name}_fwd"] = (fns, 2 * n3 + extra_f, 1, {})
        sb, ib = kw_b
        dib = di if ib is not None else None
        fns = [lambda x=x, d=d, dx=dx, sb=sb, ib=ib, dib=dib: ops._bwd_full_inplace(
            x, w3, None, d, sb, ib, dx, dw3, None, dib, True) for x, d, _, dx in sets]
        cases[f"{name}_bwd"] = (fns, 3 * n3 + extra_b, 1, {"op": "_bwd_full_inplace (fp32 accumulators)"})
        fns = [lambda x=x, d=d, dx=dx, sb=sb, ib=ib, dib=dib: ops._bwd_typed_inplace(
            x, w3, None, d, sb, ib, None, dx, dw3t, None, dib, True) for x, d, _, dx in sets]
        cases[f"{name}_bwd_typed"] = (fns, 3 * n3 + extra_t, 1,
                                      {"op": "_bwd_typed_inplace (the autograd backward: bwd_clw + bwd_reduce)"})
    if floors is not None:
        # the backward's access pattern with no arithmetic: x and dout read, dx written, on
        # the same sets (rows of 8 KB); seg 256: a wavefront per 16 rows x 256 bytes (a dword
        # per lane, the kernel's own slices); seg 1024: 4 rows x 1 KB (16 bytes per lane)
        for seg in (256, 1024):
            fns = [lambda x=x, d=d, dx=dx, seg=seg: floors.tiles(
                torch, x.transpose(1, 2)[0], d.transpose(1, 2)[0], dx.transpose(1, 2)[0], seg)
                for x, d, _, dx in sets]
            cases[f"floor_tiles{seg}_c3"] = (fns, 3 * n3, 1, {})
        # the backward's own walk (128-row runs of 256-byte slices, 4-row chunks) without arithmetic
        fns = [lambda x=x, d=d, dx=dx: floors.walk(torch, x.transpose(1, 2)[0], d.transpose(1, 2)[0],
                                                   dx.transpose(1, 2)[0]) for x, d, _, dx in sets]
        cases["floor_walk_c3"] = (fns, 3 * n3, 1, {"note": "bwd_clw's walk, grid and blocks, no arithmetic"})
        # the forward's streams: x read, out written, as a plain copy
        fns = [lambda x=x, o=o: floors.copy(torch, x.transpose(1, 2), o.transpose(1, 2)) for x, _, o, _ in sets]
        cases["floor_copy_c3"] = (fns, 2 * n3, 1, {"note": "plain copy of x into out (the forward's bytes)"})
    return cases, (cuts, L3, D3)


def _c5_cases(torch):
    """C5: (8, 2048, 16384), no bias, no activation, forward and backward for every dtype and
    width of the configuration."""
    ops = torch.ops.causal_conv1d_amd
    B5, D5, L5 = 8, 2048, 16384
    cases = {}
    g = torch.Generator(device="cuda").manual_seed(5)
    for dt, tag in ((torch.float32, "fp32"), (torch.float16, "fp16"), (torch.bfloat16, "bf16")):
        es = torch.finfo(dt).bits // 8
        x = torch.randn(B5, D5, L5, generator=g, device="cuda").to(dt)
        dout = torch.randn(B5, D5, L5, generator=g, device="cuda").to(dt)
        out, dx = torch.empty_like(x), torch.empty_like(x)
        n5 = B5 * D5 * L5 * es
        for w_ in (2, 3, 4):
            w5 = torch.randn(D5, w_, generator=g, device="cuda").to(dt)
            dw5 = torch.zeros(D5, w_, dtype=torch.float32, device="cuda")
            cases[f"c5_{tag}_w{w_}_fwd"] = ([lambda x=x, w5=w5, out=out: ops._fwd_inplace(
                x, w5, None, None, None, out, False, None)], 2 * n5 + D5 * w_ * es, 8, {})
            cases[f"c5_{tag}_w{w_}_bwd"] = ([lambda x=x, w5=w5, dout=dout, dx=dx, dw5=dw5: ops._bwd_full_inplace(
                x, w5, None, dout, None, None, dx, dw5, None, None, False)], 3 * n5 + D5 * w_ * (es + 4), 8, {})
    return cases


def _c4b_cases(torch, cc, floors):
    """C4b: x (256, 5120, 4), circular state_len 64 in a pool of 512, cache_seqlens in [0, 64)."""
    nsets = -(-2 * MALL_BYTES // C4B_LINE_BYTES) + 1  # 5: whole lines touched between reuses > 2x MALL
    sets, w, b = _update_sets(torch, nsets, seqlen=4, S=C4B_S, seed=11)
    fns = [lambda u=u: cc._native.native_update(u[0], w, b, u[1], u[2], u[3], u[4], True) for u in sets]
    hbm = _pmc("c4b_update")
    extra = {"buffer_sets": nsets, "note": "14 of 128 bytes of each state line are touched; DRAM bursts bound this"}
    cases = {"update_c4b": (fns, C4B_BYTES, 1, extra)}
    if floors is not None:
        for nch in (1, 2):
            cases[f"floor_chunks{nch}_c4b"] = (
                [lambda u=u, nch=nch: floors.chunks(torch, u[0], u[4], u[1], u[2], u[3], nch) for u in sets],
                C4B_BYTES, 1, {"note": f"{nch} 16-byte chunk(s) of each state line read and written back, x / out "
                                       "moved, no arithmetic"})
        for gran, name in ((4, "sector"), (8, "line")):
            cases[f"floor_{name}_c4b"] = (
                [lambda u=u, gran=gran: floors.chunks(torch, u[0], u[4], u[1], u[2], u[3], 2, gran) for u in sets],
                C4B_BYTES, 1, {"note": f"the whole aligned {16 * gran}-byte granule(s) holding two 16-byte chunks "
                                       "of each state line read and written back (no partial granule written), "
                                       "x / out moved, no arithmetic"})
    return cases, hbm


def _varlen_case(torch, cc, c3info):
    cuts, L3, D3 = c3info
    g = torch.Generator(device="cuda").manual_seed(9)
    xv = torch.randn(L3, D3, generator=g, device="cuda").bfloat16()
    cu = torch.tensor([0] + cuts.tolist() + [L3], dtype=torch.int32, device="cuda")
    nseq = cu.numel() - 1
    st = torch.empty(nseq, W - 1, D3, dtype=torch.bfloat16, device="cuda").transpose(1, 2)
    return {"varlen_states": ([lambda: cc._native.native_varlen_states(xv, cu, st)],
                              2 * nseq * (W - 1) * D3 * 2 + cu.numel() * 4, 1,
                              {"note": "gathers 8 x 3 rows of 4096 channels (197 KB each way): launch-bound"})}


def _run_cases(torch, cases, args, res):
    for name, (fns, nbytes, div, extra) in cases.items():
        us = _time_launch_set(torch, fns, max(4, args.launches // div), args.runs, args.kernel_settle)
        res[name] = _entry(us, nbytes, **extra)
        log(f"{name}: {res[name]['us_per_launch']} us/launch (min {res[name]['us_min']}, max {res[name]['us_max']}; "
            f"{res[name]['frac_of_peak']:.3f} of peak)")


def bench_configs(torch, cc, floors, args):
    """Every kernel at the other benchmark configurations (reported, not the headline)."""
    res = {}
    c3, c3info = _c3_cases(torch, floors)
    _run_cases(torch, c3, args, res)
    for name in ("c3a_bwd", "c3b_bwd", "c3a_bwd_typed", "c3b_bwd_typed"):
        if "floor_tiles256_c3" in res:
            res[name]["floor_same_pattern_us"] = res["floor_tiles256_c3"]["us_per_launch"]
            res[name]["floor_widest_pattern_us"] = res["floor_tiles1024_c3"]["us_per_launch"]
            res[name]["floor_walk_us"] = res["floor_walk_c3"]["us_per_launch"]
    for name in ("c3a_fwd", "c3b_fwd"):
        if "floor_copy_c3" in res:
            res[name]["floor_copy_us"] = res["floor_copy_c3"]["us_per_launch"]
    del c3
    torch.cuda.empty_cache()
    c5 = _c5_cases(torch)
    _run_cases(torch, c5, args, res)
    del c5
    torch.cuda.empty_cache()
    c4b, hbm = _c4b_cases(torch, cc, floors)
    _run_cases(torch, c4b, args, res)
    e = res["update_c4b"]
    e["us_per_call"] = e["us_per_launch"]
    if hbm:
        # HBM bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE (calibrated)
        e["hbm_bytes_per_launch"] = int(hbm)
        e["hbm_gbps"] = round(hbm / (e["us_per_launch"] * 1e-6) / 1e9, 1)
        e["hbm_frac_of_peak"] = round(e["hbm_gbps"] / HBM_PEAK_GBPS, 4)
    if "floor_chunks2_c4b" in res:
        e["floor_chunks1_us"] = res["floor_chunks1_c4b"]["us_per_launch"]
        e["floor_chunks2_us"] = res["floor_chunks2_c4b"]["us_per_launch"]
        e["floor_sector_us"] = res["floor_sector_c4b"]["us_per_launch"]
        e["floor_line_us"] = res["floor_line_c4b"]["us_per_launch"]
    del c4b
    torch.cuda.empty_cache()
    _run_cases(torch, _varlen_case(torch, cc, c3info), args, res)
    return res


# ------------------------------------------------------------------ CPU baseline


def _cpu_model():
    model, fam, mod, step = "unknown", None, None, None
    try:
        for ln in open("/proc/cpuinfo"):
            k, _, v = ln.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name" and model == "unknown":
                model = v
            elif k == "cpu family" and fam is None:
                fam = v
            elif k == "model" and mod is None:
                mod = v
            elif k == "stepping" and step is None:
                step = v
    except OSError:
        pass
    return f"{model} (family {fam}, model {mod}, stepping {step})"


def _cpu_sample(torch, d):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, d, L, generator=g).bfloat16()
    w = torch.randn(d, W, generator=g).bfloat16()
    b = torch.randn(d, generator=g).bfloat16()
    dout = torch.randn(B, d, L, generator=torch.Generator().manual_seed(1)).bfloat16()
    return x, w, b, dout


def _repeat(fn, seconds, max_reps=10000):
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if (el >= seconds and reps >= 3) or reps >= max_reps:
            return reps, el


def cpu_baseline(torch, seconds):
    """Two legs on the same bounded sample of C2 (512 of the 5120 channels, all 4 batches,
    full length), fwd + bwd repeated for about `seconds` each:
      * the C oracle, which restates the reference's Mojo CPU kernels (OpenMP over rows);
      * the reference's pure-PyTorch baseline, F.conv1d(groups=D) + F.silu with autograd
        (scripts/plot_bench.py:165-169), on torch's CPU threads."""
    import torch.nn.functional as F

    from oracle import oracle as O

    d = 512
    x, w, b, dout = _cpu_sample(torch, d)
    nbytes = (FWD_BYTES + BWD_BYTES) * d / D
    out, dx = torch.empty_like(x), torch.empty_like(x)

    def port():
        O.fwd(x, w, b, None, None, out, True)
        O.bwd(x, w, b, dout, None, None, dx, torch.zeros(d, W), torch.zeros(d), None, True)

    reps, el = _repeat(port, seconds)
    per = el / reps
    res = {"value": round(nbytes / per / 1e9, 2), "unit": "GB/s", "cores": O.num_threads(), "kind": "port",
           "sample": f"C2 fwd+bwd restricted to 512 of 5120 channels (x (4,512,2048) bf16), {reps} reps "
                     f"in {el:.1f} s, {per * 1e3:.1f} ms per fwd+bwd; C oracle restating the reference's "
                     f"Mojo CPU kernels (the Mojo path itself cannot be built here)",
           "cpu_model": _cpu_model()}

    xg, wg, bg = (t.clone().requires_grad_() for t in (x, w, b))

    def torch_ref():
        o = F.silu(F.conv1d(xg, wg.unsqueeze(1), bg, padding=W - 1, groups=d)[..., :L])
        torch.autograd.grad(o, (xg, wg, bg), dout)

    reps, el = _repeat(torch_ref, seconds)
    per = el / reps
    res["torch_cpu"] = {"value": round(nbytes / per / 1e9, 2), "unit": "GB/s", "threads": torch.get_num_threads(),
                        "sample": f"same sample, bf16 F.conv1d + F.silu forward and autograd backward, {reps} reps "
                                  f"in {el:.1f} s, {per * 1e3:.1f} ms per fwd+bwd"}
    log(f"cpu baseline: {res}")
    return res


# ------------------------------------------------------------------ modes


def mode_kernels(torch, cc, floors, args):
    """Eager launch loop (for rocprofv3 kernel traces / counters)."""
    sets, w, b = _c2_sets(torch, 4)
    cases = dict(_c2_cases(torch, sets, w, b))
    cases.update(_c2_floor_cases(torch, sets, floors))
    cases.update(_c4a_cases(torch, cc, floors))
    if not args.no_configs:
        cases.update(_c2_seq_cases(torch, sets, w, b))
        cases.update(_c2_ragged_cases(torch, w, b))
        c3, c3info = _c3_cases(torch, floors)
        cases.update(c3)
        cases.update(_c5_cases(torch))
        cases.update(_c4b_cases(torch, cc, floors)[0])
        cases.update(_varlen_case(torch, cc, c3info))
    for i in range(args.steps):
        for fns, _, _, _ in cases.values():
            fns[i % len(fns)]()
    torch.cuda.synchronize()
    log(f"kernels mode: {args.steps} iterations of {len(cases)} cases done: {', '.join(cases)}")


def mode_copy(torch, args):
    n = 2 ** 30 // 4
    a = torch.ones(n, dtype=torch.float32, device="cuda")
    c = torch.empty_like(a)
    for _ in range(args.steps):
        c.copy_(a)
    torch.cuda.synchronize()
    log(f"copy mode: {args.steps} copies of 1 GiB done")


def main():
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the op needs no "
              f"collectives and every GPU box here has a single MI355X.", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)
    import causal_conv1d_amd as cc
    from causal_conv1d_amd import _lib

    _lib.load()  # fail loudly if the HIP library is missing
    floors = Floors()
    if args.mode == "kernels":
        return mode_kernels(torch, cc, floors, args)
    if args.mode == "copy":
        return mode_copy(torch, args)

    nsets = 4  # 3 other sets between reuses: 504 MB for the forward, 755 MB for the backward
    sets, w, b = _c2_sets(torch, nsets)
    ms = bench_step(torch, cc, args, sets, w, b)
    kern = {}
    _run_cases(torch, _c2_cases(torch, sets, w, b), args, kern)
    _run_cases(torch, _c2_floor_cases(torch, sets, floors), args, kern)
    if not args.no_configs:
        _run_cases(torch, _c2_seq_cases(torch, sets, w, b), args, kern)
        _run_cases(torch, _c2_ragged_cases(torch, w, b, nsets), args, kern)
    for k in ("fwd", "bwd", "bwd_typed"):
        kern[k]["buffer_sets"] = nsets
    kern["fwd"]["floor_copy_us"] = kern["floor_copy_c2"]["us_per_launch"]
    for k in ("bwd", "bwd_typed"):
        kern[k]["floor_same_streams_us"] = kern["floor_tiles4096_c2"]["us_per_launch"]
        kern[k]["floor_streams_4rows_us"] = kern["floor_tiles1024_c2"]["us_per_launch"]
    del sets
    torch.cuda.empty_cache()
    _run_cases(torch, _c4a_cases(torch, cc, floors), args, kern)
    u = kern["update_c4a"]
    u["us_per_call"] = u["us_per_launch"]
    u["us_per_call_cache_resident"] = kern.pop("update_c4a_cache_resident")["us_per_launch"]
    u["floor_copy_us"] = kern["floor_copy_c4a"]["us_per_launch"]
    u["floor_rows_us"] = kern["floor_rows_c4a"]["us_per_launch"]
    u["runtime_copy_us"] = kern["runtime_copy_c4a"]["us_per_launch"]
    torch.cuda.empty_cache()
    if not args.no_configs:
        kern.update(bench_configs(torch, cc, floors, args))
    torch.cuda.empty_cache()
    cpu = None if args.no_cpu_baseline else cpu_baseline(torch, args.cpu_seconds)

    step_bytes = FWD_BYTES + BWD_BYTES
    value = step_bytes / (ms * 1e-3) / 1e9
    bwd = kern["bwd"]
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "C2: causal_conv1d_fn fwd + autograd bwd, x (4,5120,2048) bf16 channel-first, "
                        "weight (5120,4), bias, SiLU; a HIP graph of one step per rotating buffer set",
            "batch": B, "dim": D, "seqlen": L, "width": W, "accumulate": "fp32",
            "step_algorithmic_bytes": step_bytes, "buffer_sets": nsets,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "bwd_rows_vec (fused backward)",
            "achieved": bwd["gbps"],
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(bwd["gbps"] / HBM_PEAK_GBPS, 4),
            "traffic": _pmc("bwd"),
            "algorithmic_bytes_per_launch": BWD_BYTES,
            "us_per_launch": bwd["us_per_launch"],
            "us_min": bwd["us_min"],
            "us_max": bwd["us_max"],
            "floor_same_streams_us": bwd["floor_same_streams_us"],
        },
        "kernels": kern,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
