"""Randomized parity sweep on MI355X: seeded random shapes, layouts and options
against the oracle.

Each case draws, from its own seed, batch, dim, seqlen, width (2..9; 2..5 for
fp32, as the API allows), dtype, layout (contiguous; channel-last view; a slice
of a larger buffer; every other time step of a buffer), bias, activation and
one of three modes: plain, seq_idx (random runs, some padded with -1), or
initial_states with return_final_states and both gradients; the weight is
sometimes a transposed view and dout sometimes channel-last. Forward and
backward go through the public API (causal_conv1d_fn + autograd), so the
dispatcher's choice among the row, channel-last and generic kernels meets
shapes that no hand-written case picks. A second sweep does the same for the
decode update (widths 2..9 for every dtype there): linear or circular buffers,
with and without a state pool; a third gathers varlen states from random
packings (empty sequences included). The case's parameters are in its id.
A "large" class adds rows of several segments, whole channel-last channel
groups and sequences of 1000-5000 steps. CC1D_RANDOM_SCALE=N multiplies every
sweep's case count (new seeds, same distributions).
"""

from __future__ import annotations

import os
import random

import pytest
import torch

import causal_conv1d_amd as cc
from _util import assert_close, assert_equal, assert_reduction_close, scales
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
LAYOUTS = ["contig", "cl", "sliced", "tstride2"]


def _fn_case(seed):
    r = random.Random(seed)
    mode = r.choice(["plain", "seq", "states"])
    dt = r.choice(list(DT))
    return dict(
        seed=seed,
        B=r.randint(1, 3),
        D=r.choice([r.randint(1, 40), r.randint(41, 300), 8 * r.randint(1, 40), 64 * r.randint(1, 4)]),
        L=r.choice([r.randint(1, 20), r.randint(21, 600), 16 * r.randint(1, 40)]),
        W=r.randint(2, 5 if dt == "fp32" else 9),  # the API's width limits (fp32: 2..5)
        dt=dt,
        layout=r.choice(LAYOUTS),
        bias=r.random() < 0.7,
        act=r.choice([None, "silu"]),
        mode=mode,
        wt=r.random() < 0.3,     # weight as the transpose of a (width, dim) tensor
        dcl=r.random() < 0.3,    # dout in the channel-last layout
    )


def _fn_id(c):
    return (f"s{c['seed']}-{c['dt']}-B{c['B']}D{c['D']}L{c['L']}W{c['W']}-{c['layout']}-{c['mode']}"
            f"-{'bias' if c['bias'] else 'nobias'}-{c['act']}{'-wT' if c['wt'] else ''}{'-doutcl' if c['dcl'] else ''}")


SCALE = int(os.environ.get("CC1D_RANDOM_SCALE", "1"))


def _fn_large_case(seed):
    """The same draws with a large shape: several row segments, whole channel-last groups."""
    r = random.Random(7_000_000 + seed)
    c = _fn_case(seed)
    c.update(
        B=r.randint(1, 2),
        D=r.choice([128 * r.randint(1, 8), 512 * r.randint(1, 2), r.randint(300, 700)]),
        L=r.choice([2048 * r.randint(1, 2), r.randint(2000, 5000), 1024 * r.randint(1, 4) + r.choice([0, 8, 264])]),
        W=r.randint(2, 5 if c["dt"] == "fp32" else 9),
        layout=r.choice(["contig", "cl", "cl", "sliced"]),
    )
    return c


FN_CASES = [_fn_case(s) for s in range(360 * SCALE)] + [_fn_large_case(s) for s in range(24 * SCALE)]


def _rand(g, *shape, dtype):
    return torch.randn(*shape, generator=g).to(dtype)


def _random_seq_idx(g, B, L):
    """Non-decreasing ids in random runs; about a third of the cases pad one run with -1."""
    s = torch.zeros(B, L, dtype=torch.int32)
    for bi in range(B):
        k = int(torch.randint(0, 6, (1,), generator=g))
        cuts = sorted(torch.randint(1, max(L, 2), (k,), generator=g).tolist()) if L > 1 else []
        for i, c in enumerate(cuts):
            s[bi, c:] = i + 1
        if cuts and float(torch.rand(1, generator=g)) < 0.35:
            run = int(torch.randint(0, len(cuts) + 1, (1,), generator=g))
            s[bi][s[bi] == run] = -1
    return s


def _device_view(x, layout):
    """(leaf on the GPU, view of it with x's values in the requested layout)."""
    B, D, L = x.shape
    if layout == "contig":
        base = x.clone().to(DEV)
        return base, lambda t: t
    if layout == "cl":
        base = x.transpose(1, 2).contiguous().to(DEV)
        return base, lambda t: t.transpose(1, 2)
    if layout == "sliced":
        base = torch.zeros(B, D + 2, L + 5, dtype=x.dtype)
        base[:, 1:D + 1, 2:L + 2] = x
        return base.to(DEV), lambda t: t[:, 1:D + 1, 2:L + 2]
    base = torch.zeros(B, D, 2 * L, dtype=x.dtype)
    base[..., ::2] = x
    return base.to(DEV), lambda t: t[..., ::2]


@pytest.mark.parametrize("c", FN_CASES, ids=_fn_id)
def test_random_forward_backward(c):
    dtype = DT[c["dt"]]
    B, D, L, W = c["B"], c["D"], c["L"], c["W"]
    g = torch.Generator().manual_seed(1000 + c["seed"])
    x = _rand(g, B, D, L, dtype=dtype)
    w = _rand(g, D, W, dtype=dtype)
    b = _rand(g, D, dtype=dtype) if c["bias"] else None
    dout = _rand(g, B, D, L, dtype=dtype)
    seq = _random_seq_idx(g, B, L) if c["mode"] == "seq" else None
    init = _rand(g, B, D, W - 1, dtype=dtype) if c["mode"] == "states" else None
    dfs = _rand(g, B, D, W - 1, dtype=dtype) if c["mode"] == "states" else None

    base, view = _device_view(x, c["layout"])
    base.requires_grad_()
    if c["wt"]:
        wg = w.t().contiguous().to(DEV).requires_grad_()
        wv = wg.t()
    else:
        wg = w.to(DEV).requires_grad_()
        wv = wg
    dg = dout.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) if c["dcl"] else dout.to(DEV)
    bg = b.to(DEV).requires_grad_() if b is not None else None
    ig = init.to(DEV).requires_grad_() if init is not None else None
    kw = dict(activation=c["act"], seq_idx=None if seq is None else seq.to(DEV), initial_states=ig)
    if c["mode"] == "states":
        out, fs = cc.causal_conv1d_fn(view(base), wv, bg, return_final_states=True, **kw)
        torch.autograd.backward([out, fs], [dg, dfs.to(DEV)])
    else:
        out = cc.causal_conv1d_fn(view(base), wv, bg, **kw)
        out.backward(dg)
    torch.cuda.synchronize()

    ref = O.causal_conv1d_fn(x, w, b, seq_idx=seq, initial_states=init,
                             return_final_states=c["mode"] == "states", activation=c["act"])
    if c["mode"] == "states":
        ref, rfs = ref
        assert_equal(fs.detach().cpu(), rfs, name="final_states")
    assert_close(out.detach().cpu(), ref, dtype, name="out")
    rdx, rdw, rdb, rdi = O.causal_conv1d_bwd(x, w, b, dout, seq_idx=seq, initial_states=init,
                                             dfinal_states=dfs, activation=c["act"])
    assert_close(view(base.grad).cpu(), rdx, dtype, name="dx")
    sw, sb = scales(x, w, b, dout, init=init, seq_idx=seq, activation=c["act"])
    assert_reduction_close(wg.grad.t().cpu() if c["wt"] else wg.grad.cpu(), rdw, dtype, scale=sw, name="dweight")
    if b is not None:
        assert_reduction_close(bg.grad.cpu(), rdb, dtype, scale=sb, name="dbias")
    if init is not None:
        assert_close(ig.grad.cpu(), rdi, dtype, name="dinitial_states")


def _upd_case(seed):
    r = random.Random(50_000 + seed)
    W = r.randint(2, 9)
    return dict(
        seed=seed,
        B=r.randint(1, 6),
        D=r.choice([r.randint(1, 40), r.randint(41, 300), 64 * r.randint(1, 8)]),
        T=r.randint(1, 5),
        W=W,
        S=W - 1 + r.choice([0, 0, 1, r.randint(2, 9)]),
        dt=r.choice(list(DT)),
        bias=r.random() < 0.7,
        act=r.choice([None, "silu"]),
        circ=r.random() < 0.5,
        pool=r.random() < 0.5,
        two_d=r.random() < 0.3,
    )


def _upd_id(c):
    return (f"s{c['seed']}-{c['dt']}-B{c['B']}D{c['D']}T{c['T']}W{c['W']}S{c['S']}"
            f"-{'circ' if c['circ'] else 'lin'}-{'pool' if c['pool'] else 'direct'}"
            f"-{'bias' if c['bias'] else 'nobias'}-{c['act']}{'-2d' if c['two_d'] else ''}")


UPD_CASES = [_upd_case(s) for s in range(150 * SCALE)]


@pytest.mark.parametrize("c", UPD_CASES, ids=_upd_id)
def test_random_update(c):
    dtype = DT[c["dt"]]
    B, D, T, W, S = c["B"], c["D"], c["T"], c["W"], c["S"]
    g = torch.Generator().manual_seed(2000 + c["seed"])
    x = _rand(g, B, D, T, dtype=dtype)
    if c["two_d"]:
        x = x[..., 0]
    w = _rand(g, D, W, dtype=dtype)
    b = _rand(g, D, dtype=dtype) if c["bias"] else None
    P = B + int(torch.randint(0, 5, (1,), generator=g)) if c["pool"] else B
    state = _rand(g, P, D, S, dtype=dtype)
    kw = dict(activation=c["act"])
    if c["pool"]:
        kw["conv_state_indices"] = torch.randperm(P, generator=g)[:B].to(torch.int32)
    if c["circ"]:
        kw["cache_seqlens"] = torch.randint(0, 2 * S + 3, (B,), generator=g, dtype=torch.int32)
    sg = state.to(DEV)
    out = cc.causal_conv1d_update(x.to(DEV), sg, w.to(DEV), None if b is None else b.to(DEV),
                                  **{k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in kw.items()})
    torch.cuda.synchronize()
    rs = state.clone()
    rout = O.causal_conv1d_update(x, rs, w, b, **kw)
    assert_close(out.cpu(), rout, dtype, name="out")
    assert_equal(sg.cpu(), rs, name="conv_state")


def _varlen_case(seed):
    r = random.Random(90_000 + seed)
    return dict(seed=seed, n=r.randint(1, 8), D=r.choice([r.randint(1, 40), r.randint(41, 300), 64 * r.randint(1, 8)]),
                S=r.randint(0, 12), dt=r.choice(list(DT)), maxlen=r.choice([3, 20, 300]), strided=r.random() < 0.3)


VARLEN_CASES = [_varlen_case(s) for s in range(60 * SCALE)]


@pytest.mark.parametrize("c", VARLEN_CASES, ids=lambda c: (f"s{c['seed']}-{c['dt']}-n{c['n']}D{c['D']}S{c['S']}"
                                                             f"-max{c['maxlen']}{'-strided' if c['strided'] else ''}"))
def test_random_varlen_states(c):
    dtype = DT[c["dt"]]
    g = torch.Generator().manual_seed(3000 + c["seed"])
    lens = torch.randint(0, c["maxlen"] + 1, (c["n"],), generator=g)  # zero-length sequences included
    cu = torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(lens, 0)]).to(torch.int32)
    total = int(cu[-1])
    x = _rand(g, total, c["D"], dtype=dtype)
    xg = x.to(DEV)
    if c["strided"]:  # rows of a wider buffer: a channel stride of 1 and a token stride > dim
        wide = torch.zeros(total, c["D"] + 5, dtype=dtype, device=DEV)
        wide[:, 3:3 + c["D"]] = xg
        xg = wide[:, 3:3 + c["D"]]
    out = cc.causal_conv1d_varlen_states(xg, cu.to(DEV), state_len=c["S"]).cpu()
    assert_equal(out, O.varlen_states(x, cu, c["S"]), name="states")
