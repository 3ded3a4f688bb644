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
               per launch / average launch duration, measured here with HIP
               events around a graph of back-to-back launches, vs 8 TB/s.
               `traffic` (HBM bytes per launch) is read from the rocprofv3
               --pmc summary committed in profiles/ when present.
  kernels      the same measurement for the forward kernel and for the decode
               update (C4a: 256 x 5120 bf16, pool 512 x 5120 x 3, random rows),
               in GB/s and microseconds per call.
  cpu_baseline the CPU oracle (C restatement of the reference's CPU kernels,
               OpenMP) on a bounded sample of C2, on this host.

Input sets are rotated so that the data touched between two reuses of a
buffer exceeds the 256 MB Infinity Cache: every launch streams from HBM.

Modes: --mode bench (default), --mode kernels (eager launch loop of the C2
forward / backward / C4a update, plus the C3 / C5 / C4b / varlen-states
launches unless --no-configs, for rocprofv3 --kernel-trace / --pmc), --mode copy (a plain
1 GiB device copy, the calibration kernel for FETCH_SIZE / WRITE_SIZE).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "causal-conv1d-mojo_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "fwd/bwd achieved HBM GB/s (% peak) at B4×D5120×L2048 bf16; update µs/call"
HBM_PEAK_GBPS = 8000.0
B, D, L, W = 4, 5120, 2048, 4
# algorithmic bytes: every input read once, every output written once
FWD_BYTES = 2 * B * D * L * 2 + D * W * 2 + D * 2                      # 167,823,360
BWD_BYTES = 3 * B * D * L * 2 + D * W * 2 + D * 2 + D * W * 4 + D * 4  # 251,811,840
UPD_B, UPD_POOL = 256, 512
UPD_BYTES = UPD_B * D * (2 + 6 + 6 + 2) + D * W * 2 + D * 2 + UPD_B * 4  # 21,023,744
MALL_BYTES = 256 * 2 ** 20


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def _parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--mode", choices=["bench", "kernels", "copy"], default="bench")
    ap.add_argument("--launches", type=int, default=40, help="launches per kernel timing graph")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the C3/C4b/C5/varlen report lines")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU-baseline duration")
    ap.add_argument("--settle", type=float, default=0.3,
                    help="seconds of untimed C2 kernels before the first timing (clock ramp)")
    return ap.parse_args()


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


def _time_graph(torch, g, reps):
    """Average ms per replay over `reps` replays, HIP events on torch's current stream."""
    g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / reps


def _pmc_traffic(kernel):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, or None."""
    p = ROOT / "profiles" / "pmc_summary.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get(kernel, {}).get("hbm_bytes_per_launch")
    except (ValueError, OSError):
        return None


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


def bench_kernels(torch, sets, w, b, launches):
    """Per-launch duration of the forward and backward kernels (custom ops, no autograd)."""
    nsets = len(sets)
    outs = [torch.empty_like(x) for x, _ in sets]
    dxs = [torch.empty_like(x) for x, _ in sets]
    dw = torch.zeros(D, W, dtype=torch.float32, device="cuda")
    db = torch.zeros(D, dtype=torch.float32, device="cuda")
    xs = [x.detach() for x, _ in sets]

    def fwd_loop():
        for i in range(launches):
            torch.ops.causal_conv1d_amd._fwd_inplace(xs[i % nsets], w, b, None, None, outs[i % nsets], True, None)

    def bwd_loop():
        for i in range(launches):
            x, dout = xs[i % nsets], sets[i % nsets][1]
            torch.ops.causal_conv1d_amd._bwd_full_inplace(x, w, b, dout, None, None, dxs[i % nsets], dw, db, None,
                                                          True)

    res = {}
    for name, loop, nbytes in (("fwd", fwd_loop, FWD_BYTES), ("bwd", bwd_loop, BWD_BYTES)):
        g = _graph(torch, loop)
        ms = min(_time_graph(torch, g, 3) for _ in range(3)) / launches
        res[name] = {"us_per_launch": round(ms * 1e3, 2), "algorithmic_bytes": nbytes,
                     "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "frac_of_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
        log(f"{name}: {res[name]}")
        del g
    return res


def _update_sets(torch, n):
    sets = []
    g = torch.Generator(device="cuda").manual_seed(7)
    w = torch.randn(D, W, generator=g, device="cuda").bfloat16()
    b = torch.randn(D, generator=g, device="cuda").bfloat16()
    for _ in range(n):
        x = torch.randn(UPD_B, D, generator=g, device="cuda").bfloat16()
        pool = torch.randn(UPD_POOL, D, W - 1, generator=g, device="cuda").bfloat16()
        idx = torch.randperm(UPD_POOL, generator=g, device="cuda")[:UPD_B].to(torch.int32)
        sets.append((x, pool, idx, torch.empty_like(x)))
    return sets, w, b


def bench_update(torch, cc, launches):
    nsets = -(-MALL_BYTES // (UPD_POOL * D * (W - 1) * 2 + 2 * UPD_B * D * 2)) + 1
    sets, w, b = _update_sets(torch, nsets)
    lib_update = cc._native.native_update

    def loop():
        for i in range(launches):
            x, pool, idx, out = sets[i % nsets]
            lib_update(x.unsqueeze(-1), w, b, pool, idx, None, out.unsqueeze(-1), True)

    g = _graph(torch, loop)
    ms = min(_time_graph(torch, g, 3) for _ in range(3)) / launches
    us = ms * 1e3
    del g

    # A decode loop reuses one state pool every step: with one buffer set the 21 MB of
    # a call stay in the 256 MB Infinity Cache between calls. Reported beside the
    # HBM-streaming figure above, never as it.
    def warm_loop():
        x, pool, idx, out = sets[0]
        for _ in range(launches):
            lib_update(x.unsqueeze(-1), w, b, pool, idx, None, out.unsqueeze(-1), True)

    g = _graph(torch, warm_loop)
    us_warm = min(_time_graph(torch, g, 3) for _ in range(3)) / launches * 1e3
    del g
    res = {"workload": "C4a: x (256,5120,1) bf16, pool (512,5120,3), 256 random rows, W4, bias, SiLU",
           "us_per_call": round(us, 2), "algorithmic_bytes": UPD_BYTES,
           "gbps": round(UPD_BYTES / (us * 1e-6) / 1e9, 1),
           "frac_of_peak": round(UPD_BYTES / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4), "buffer_sets": nsets,
           "us_per_call_cache_resident": round(us_warm, 2)}
    log(f"update: {res}")
    return res


def _time_launch_set(torch, fns, launches):
    """Average ms per launch of a graph that cycles through the closures `fns`."""
    def loop():
        for i in range(launches):
            fns[i % len(fns)]()
    g = _graph(torch, loop)
    ms = min(_time_graph(torch, g, 3) for _ in range(3)) / launches
    del g
    return ms


def _entry(ms, nbytes, **extra):
    gbps = nbytes / (ms * 1e-3) / 1e9
    return {"us_per_launch": round(ms * 1e3, 2), "algorithmic_bytes": int(nbytes), "gbps": round(gbps, 1),
            "frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4), **extra}


def _config_cases(torch, cc):
    """Launch closures of the other benchmark configurations: name -> (closures cycling
    over rotating buffer sets, algorithmic bytes per launch, launches per timing graph
    divisor, extra report fields)."""
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
    for _ in range(3):
        x = torch.randn(1, L3, D3, generator=g, device="cuda").bfloat16().transpose(1, 2)
        dout = torch.randn(1, L3, D3, generator=g, device="cuda").bfloat16().transpose(1, 2)
        sets.append((x, dout, torch.empty_like(x), torch.empty_like(x)))
    dw3 = torch.zeros(D3, W, dtype=torch.float32, device="cuda")
    fs = torch.empty(1, D3, W - 1, dtype=torch.bfloat16, device="cuda")
    di = torch.empty_like(init)
    n3 = L3 * D3 * 2
    for name, kw_f, kw_b, extra_f, extra_b in (
            ("c3a", (seq, None, None), (seq, None), 32768 + D3 * W * 2, 2 * 32768 + D3 * W * 2 + D3 * W * 4),
            ("c3b", (None, init, fs), (None, init), D3 * W * 2 + 2 * 24576, D3 * W * 2 + D3 * W * 4 + 2 * 24576)):
        s_, i_, f_ = kw_f
        fns = [lambda x=x, o=o, s_=s_, i_=i_, f_=f_: ops._fwd_inplace(x, w3, None, s_, i_, o, True, f_)
               for x, _, o, _ in sets]
        cases[f"{name}_fwd"] = (fns, 2 * n3 + extra_f, 1, {})
        sb, ib = kw_b
        fns = [lambda x=x, d=d, dx=dx, sb=sb, ib=ib: ops._bwd_full_inplace(x, w3, None, d, sb, ib, dx, dw3, None,
                                                                           di if ib is not None else None, True)
               for x, d, _, dx in sets]
        cases[f"{name}_bwd"] = (fns, 3 * n3 + extra_b, 1, {})
    # C5: (8, 2048, 16384), no bias, no activation, bf16 and fp32 at W4 (W2/W3 in the tests)
    B5, D5, L5 = 8, 2048, 16384
    for dt, tag in ((torch.bfloat16, "bf16"), (torch.float32, "fp32")):
        es = 2 if dt == torch.bfloat16 else 4
        x = torch.randn(B5, D5, L5, generator=g, device="cuda").to(dt)
        dout = torch.randn(B5, D5, L5, generator=g, device="cuda").to(dt)
        out, dx = torch.empty_like(x), torch.empty_like(x)
        w5 = torch.randn(D5, W, generator=g, device="cuda").to(dt)
        dw5 = torch.zeros(D5, W, dtype=torch.float32, device="cuda")
        n5 = B5 * D5 * L5 * es
        cases[f"c5_{tag}_fwd"] = ([lambda x=x, w5=w5, out=out: ops._fwd_inplace(x, w5, None, None, None, out, False,
                                                                                 None)], 2 * n5 + D5 * W * es, 8, {})
        cases[f"c5_{tag}_bwd"] = ([lambda x=x, w5=w5, dout=dout, dx=dx, dw5=dw5: ops._bwd_full_inplace(
            x, w5, None, dout, None, None, dx, dw5, None, None, False)], 3 * n5 + D5 * W * (es + 4), 8, {})
    # C4b: x (256, 5120, 4), circular state_len 64 in a pool of 512, cache_seqlens in [0, 64)
    usets = []
    w4 = torch.randn(D, W, generator=g, device="cuda").bfloat16()
    b4 = torch.randn(D, generator=g, device="cuda").bfloat16()
    for _ in range(4):
        x = torch.randn(UPD_B, D, 4, generator=g, device="cuda").bfloat16()
        pool = torch.randn(UPD_POOL, D, 64, generator=g, device="cuda").bfloat16()
        idx = torch.randperm(UPD_POOL, generator=g, device="cuda")[:UPD_B].to(torch.int32)
        cs = torch.randint(0, 64, (UPD_B,), generator=g, device="cuda", dtype=torch.int32)
        usets.append((x, pool, idx, cs, torch.empty_like(x)))
    fns = [lambda u=u: cc._native.native_update(u[0], w4, b4, u[1], u[2], u[3], u[4], True) for u in usets]
    nb = UPD_B * D * (8 + 6 + 8 + 8) + D * W * 2 + D * 2 + 2 * UPD_B * 4
    cases["update_c4b"] = (fns, nb, 1, {"note": "14 of 128 bytes of each state row are touched; DRAM bursts "
                                                "bound this"})
    # varlen states: x (8192, 4096) bf16 packing the 8 C3 sequences, state_len W-1
    xv = torch.randn(L3, D3, generator=g, device="cuda").bfloat16()
    cu = torch.tensor([0] + cuts.tolist() + [L3], dtype=torch.int32, device="cuda")
    nseq = cu.numel() - 1
    st = torch.empty(nseq, W - 1, D3, dtype=torch.bfloat16, device="cuda").transpose(1, 2)
    cases["varlen_states"] = ([lambda: cc._native.native_varlen_states(xv, cu, st)],
                              2 * nseq * (W - 1) * D3 * 2 + cu.numel() * 4, 1,
                              {"note": "gathers 8 x 3 rows of 4096 channels (197 KB each way): launch-bound"})
    return cases


def bench_configs(torch, cc, launches):
    """Kernel throughput at the other benchmark configurations (reported, not the headline)."""
    res = {}
    for name, (fns, nbytes, div, extra) in _config_cases(torch, cc).items():
        ms = _time_launch_set(torch, fns, max(4, launches // div))
        res[name] = _entry(ms, nbytes, **extra)
        if name == "update_c4b":
            res[name]["us_per_call"] = res[name]["us_per_launch"]
        log(f"{name}: {res[name]['us_per_launch']} us/launch ({res[name]['frac_of_peak']:.3f} of peak)")
    return res


def cpu_baseline(torch, seconds):
    """The CPU oracle on a bounded sample of C2 (512 of the 5120 channels, all 4
    batches, full length), fwd + bwd repeated for about `seconds`."""
    from oracle import oracle as O

    d = 512
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, d, L, generator=g).bfloat16()
    w = torch.randn(d, W, generator=g).bfloat16()
    b = torch.randn(d, generator=g).bfloat16()
    dout = torch.randn(B, d, L, generator=g).bfloat16()
    out = torch.empty_like(x)
    dx = torch.empty_like(x)
    nbytes = (FWD_BYTES + BWD_BYTES) * d / D
    reps, t0 = 0, time.perf_counter()
    while True:
        O.fwd(x, w, b, None, None, out, True)
        dw = torch.zeros(d, W)
        db = torch.zeros(d)
        O.bwd(x, w, b, dout, None, None, dx, dw, db, None, True)
        reps += 1
        el = time.perf_counter() - t0
        if (el >= seconds and reps >= 3) or reps >= 10000:
            break
    per = el / reps
    res = {"value": round(nbytes / per / 1e9, 2), "unit": "GB/s", "cores": O.num_threads(), "kind": "port",
           "sample": f"C2 fwd+bwd restricted to 512 of 5120 channels (x (4,512,2048) bf16), {reps} reps "
                     f"in {el:.1f} s, {per * 1e3:.1f} ms per fwd+bwd; C oracle restating the reference's "
                     f"Mojo CPU kernels (the Mojo path itself cannot be built here)",
           "cpu_model": _cpu_model()}
    log(f"cpu baseline: {res}")
    return res


def _cpu_model():
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def mode_kernels(torch, cc, args):
    """Eager launch loop (for rocprofv3 kernel traces / counters)."""
    sets, w, b = _c2_sets(torch, 3)
    outs = [torch.empty_like(x) for x, _ in sets]
    dxs = [torch.empty_like(x) for x, _ in sets]
    dw = torch.zeros(D, W, dtype=torch.float32, device="cuda")
    db = torch.zeros(D, dtype=torch.float32, device="cuda")
    usets, uw, ub = _update_sets(torch, 13)
    cases = {} if args.no_configs else _config_cases(torch, cc)
    for i in range(args.steps):
        x, dout = sets[i % 3]
        torch.ops.causal_conv1d_amd._fwd_inplace(x, w, b, None, None, outs[i % 3], True, None)
        torch.ops.causal_conv1d_amd._bwd_full_inplace(x, w, b, dout, None, None, dxs[i % 3], dw, db, None, True)
        ux, pool, idx, uo = usets[i % 13]
        cc._native.native_update(ux.unsqueeze(-1), uw, ub, pool, idx, None, uo.unsqueeze(-1), True)
        for fns, _, _, _ in cases.values():
            fns[i % len(fns)]()
    torch.cuda.synchronize()
    log(f"kernels mode: {args.steps} iterations of fwd + bwd + update" + ("" if args.no_configs else
        " + the C3 / C5 / C4b launches") + " done")


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
    if args.mode == "kernels":
        return mode_kernels(torch, cc, args)
    if args.mode == "copy":
        return mode_copy(torch, args)

    nsets = max(2, -(-MALL_BYTES // (4 * B * D * L * 2)) + 1)
    sets, w, b = _c2_sets(torch, nsets)
    ms = bench_step(torch, cc, args, sets, w, b)
    kern = bench_kernels(torch, sets, w, b, args.launches)
    del sets
    torch.cuda.empty_cache()
    upd = bench_update(torch, cc, args.launches)
    torch.cuda.empty_cache()
    cfgs = {} if args.no_configs else bench_configs(torch, cc, args.launches)
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
            "step_algorithmic_bytes": step_bytes,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "bwd_rows_vec (fused backward)",
            "achieved": bwd["gbps"],
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(bwd["gbps"] / HBM_PEAK_GBPS, 4),
            "traffic": _pmc_traffic("bwd"),
            "algorithmic_bytes_per_launch": BWD_BYTES,
            "us_per_launch": bwd["us_per_launch"],
        },
        "kernels": {"fwd": kern["fwd"], "bwd": kern["bwd"], "update_c4a": upd, **cfgs},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
