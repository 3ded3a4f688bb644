"""Ragged rows on MI355X: rows whose length is not a multiple of the 16-byte
vector, or whose first element does not sit on a 16-byte boundary. The row
kernels take them directly (a row's first and last vectors are shared with
its neighbours), and are held to the oracle on the same inputs:

* every width at lengths around the vector, lane and segment sizes, through
  the public API and autograd (contiguous tensors with an odd length: every
  row starts at another offset inside its vector);
* initial_states / final_states and their gradients, seq_idx (padding at a
  row's start included);
* bases offset by 1 .. EPV-1 elements with out / dout / dx laid out like x,
  through the custom ops (the layout the public API would copy away), with
  the memory around every row left as it was;
* non-finite values in a neighbouring row, which must not reach this row's
  outputs or gradients (the reference never reads past a row's ends).

The host side of the choice (ragged rows keep the row kernels) is pinned on
the CPU by the workspace sizes in test_abi.py.
"""

from __future__ import annotations

import pytest
import torch

import causal_conv1d_amd as cc
from _util import DTYPE_IDS, DTYPES, assert_close, assert_reduction_close, make_inputs, scales, seq_pattern
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPV = {torch.float16: 8, torch.bfloat16: 8, torch.float32: 4}  # elements per 16-byte vector


def _skip_fp32_wide(dtype, width):
    if dtype == torch.float32 and width > 5:
        pytest.skip("fp32 widths above 5 are rejected by the API (reference _fn.py:405-414)")


def _autograd(x, w, b, dout, *, init=None, seq_idx=None, dfs=None, activation="silu", view=None):
    """Forward + backward through the public API on the GPU (x through a layout `view`):
    (out, final_states, dx, dw, db, dinit)."""
    xg = x.to(DEV).requires_grad_()
    wg = w.to(DEV).requires_grad_()
    bg = b.to(DEV).requires_grad_() if b is not None else None
    ig = init.to(DEV).requires_grad_() if init is not None else None
    kw = dict(initial_states=ig, activation=activation, seq_idx=None if seq_idx is None else seq_idx.to(DEV))
    fs = None
    xin = xg if view is None else view(xg)
    if dfs is not None:
        out, fs = cc.causal_conv1d_fn(xin, wg, bg, return_final_states=True, **kw)
        torch.autograd.backward([out, fs], [dout.to(DEV), dfs.to(DEV)])
    else:
        out = cc.causal_conv1d_fn(xin, wg, bg, **kw)
        out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    cpu = (lambda t: None if t is None else t.detach().cpu())
    return (cpu(out), cpu(fs), cpu(xg.grad), cpu(wg.grad), cpu(None if bg is None else bg.grad),
            cpu(None if ig is None else ig.grad))


def _check_all(got, x, w, b, dout, dtype, *, init=None, seq_idx=None, dfs=None, activation="silu"):
    out, fs, dx, dw, db, di = got
    rout = O.causal_conv1d_fn(x, w, b, seq_idx=seq_idx, initial_states=init,
                              return_final_states=dfs is not None, activation=activation)
    if dfs is not None:
        rout, rfs = rout
        assert_close(fs, rfs, dtype, name="final_states")
    assert_close(out, rout, dtype, name="out")
    rdx, rdw, rdb, rdi = O.causal_conv1d_bwd(x, w, b, dout, seq_idx=seq_idx, initial_states=init,
                                             dfinal_states=dfs, activation=activation)
    sw, sb = scales(x, w, b, dout, init=init, seq_idx=seq_idx, activation=activation)
    assert_close(dx, rdx, dtype, name="dx")
    assert_reduction_close(dw, rdw, dtype, scale=sw, name="dweight")
    if b is not None:
        assert_reduction_close(db, rdb, dtype, scale=sb, name="dbias")
    if init is not None:
        assert_close(di, rdi, dtype, name="dinitial_states")


# lengths: 1 element; inside one vector; one past a vector; about one lane row
# (64 vectors) either side; one past the 4-vector segment of bf16 / fp16; a
# row of three segments with a short tail
RAGGED_LENGTHS = [1, 7, 9, 513, 1023, 2049, 6141]


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4, 5, 6, 7, 8, 9])
@pytest.mark.parametrize("seqlen", RAGGED_LENGTHS)
def test_ragged_rows_forward_backward(dtype, width, seqlen):
    _skip_fp32_wide(dtype, width)
    x, w, b, _ = make_inputs(2, 5, seqlen, width, dtype=dtype)  # 5 rows per entry: 5 offsets
    dout = make_inputs(2, 5, seqlen, width, dtype=dtype, seed=1)[0]
    _check_all(_autograd(x, w, b, dout), x, w, b, dout, dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4, 5, 6, 7, 8, 9])
@pytest.mark.parametrize("seqlen", [2, 5, 9, 1023, 2049])
def test_ragged_rows_states(dtype, width, seqlen):
    """initial_states fill the positions before each row (also inside its first vector, which
    starts in the previous row); dfinal_states land on its last W-1 positions, wherever they
    fall in the vectors; dinitial_states come from the first W-1 positions' dpre."""
    _skip_fp32_wide(dtype, width)
    x, w, b, init = make_inputs(2, 7, seqlen, width, dtype=dtype, has_init=True)
    dout = make_inputs(2, 7, seqlen, width, dtype=dtype, seed=1)[0]
    dfs = make_inputs(2, 7, width - 1, width, dtype=dtype, seed=2)[0]
    got = _autograd(x, w, b, dout, init=init, dfs=dfs)
    _check_all(got, x, w, b, dout, dtype, init=init, dfs=dfs)


def _leading_padding(batch, seqlen):
    """Padding (-1) over each row's first positions, then two sequences."""
    s = torch.zeros(batch, seqlen, dtype=torch.int32)
    s[:, : min(5, seqlen)] = -1
    s[:, seqlen // 2:] = 1
    return s


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("pattern", ["with_padding", "repeat_ids", "random_runs", "leading_padding"])
@pytest.mark.parametrize("seqlen", [37, 1023, 4097 + 2 * 128])
@pytest.mark.parametrize("activation", [None, "silu"])
def test_ragged_rows_seq_idx(dtype, pattern, seqlen, activation):
    x, w, b, _ = make_inputs(2, 6, seqlen, 4, dtype=dtype)
    dout = make_inputs(2, 6, seqlen, 4, dtype=dtype, seed=1)[0]
    s = _leading_padding(2, seqlen) if pattern == "leading_padding" else seq_pattern(pattern, 2, seqlen)
    got = _autograd(x, w, b, dout, seq_idx=s, activation=activation)
    _check_all(got, x, w, b, dout, dtype, seq_idx=s, activation=activation)


SENTINEL = 7.0  # exact in every dtype


def _offset_view(B, D, L, off, dtype, fill=None, src=None):
    """A (B, D, L) view starting `off` elements into the rows of a (B, D + 1, L + off + 3) buffer."""
    base = torch.full((B, D + 1, L + off + 3), SENTINEL if fill is None else fill, dtype=dtype, device=DEV)
    v = base[:, :D, off:off + L]
    if src is not None:
        v.copy_(src)
    return base, v


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 4, 5, 9])
@pytest.mark.parametrize("seqlen", [3, 1021, 2052])
@pytest.mark.parametrize("mode", ["plain", "states", "seq_idx"])
def test_ragged_offset_bases_through_the_custom_ops(dtype, width, seqlen, mode):
    """x, out, dout and dx all start `off` elements into rows of the same pitch (so every row
    of each is equally far past a 16-byte boundary); the ops write only inside the views."""
    _skip_fp32_wide(dtype, width)
    ops = torch.ops.causal_conv1d_amd
    B, D = 2, 5
    for off in range(1, EPV[dtype]):
        x, w, b, init = make_inputs(B, D, seqlen, width, dtype=dtype, has_init=True, seed=off)
        dout = make_inputs(B, D, seqlen, width, dtype=dtype, seed=100 + off)[0]
        dfs = make_inputs(B, D, width - 1, width, dtype=dtype, seed=200 + off)[0]
        seq = seq_pattern("repeat_ids", B, seqlen) if mode == "seq_idx" else None
        if mode != "states":
            init = dfs = None
        _, xv = _offset_view(B, D, seqlen, off, dtype, fill=float("nan"), src=x.to(DEV))
        _, gv = _offset_view(B, D, seqlen, off, dtype, fill=float("nan"), src=dout.to(DEV))
        obase, ov = _offset_view(B, D, seqlen, off, dtype)
        dbase, dv = _offset_view(B, D, seqlen, off, dtype)
        wd, bd = w.to(DEV), b.to(DEV)
        idv = None if init is None else init.to(DEV)
        fs = None if init is None else torch.empty(B, D, width - 1, dtype=dtype, device=DEV)
        sd = None if seq is None else seq.to(DEV)
        ops._fwd_inplace(xv, wd, bd, sd, idv, ov, True, fs)
        dw = torch.zeros(D, width, dtype=torch.float32, device=DEV)
        db = torch.zeros(D, dtype=torch.float32, device=DEV)
        di = None if init is None else torch.empty_like(idv)
        ops._bwd_full_inplace(xv, wd, bd, gv, sd, idv, dv, dw, db, di, True,
                              None if dfs is None else dfs.to(DEV))
        torch.cuda.synchronize()
        for name, base, view in (("out", obase, ov), ("dx", dbase, dv)):
            outside = torch.ones_like(base, dtype=torch.bool)
            outside[:, :D, off:off + seqlen] = False
            assert (base[outside] == SENTINEL).all(), f"off={off}: {name} written outside the rows"
        case = dict(initial_states=init, seq_idx=seq, dfinal_states=dfs, activation="silu")
        rout, rfs = O.causal_conv1d_fn(x, w, b, seq_idx=seq, initial_states=init, return_final_states=True,
                                       activation="silu")
        assert_close(ov.cpu(), rout, dtype, name=f"out (off={off})")
        rdx, rdw, rdb, rdi = O.causal_conv1d_bwd(x, w, b, dout, **case)
        sw, sb = scales(x, w, b, dout, init=init, seq_idx=seq, activation="silu")
        assert_close(dv.cpu(), rdx, dtype, name=f"dx (off={off})")
        assert_reduction_close(dw.cpu(), rdw.float(), dtype, scale=sw, name=f"dweight (off={off})")
        assert_reduction_close(db.cpu(), rdb.float(), dtype, scale=sb, name=f"dbias (off={off})")
        if init is not None:
            assert_close(fs.cpu(), rfs, dtype, name=f"final_states (off={off})")
            assert_close(di.cpu(), rdi, dtype, name=f"dinitial_states (off={off})")


def _same_nonfinite_then_close(got, ref, dtype, name, scale=None):
    """Non-finite exactly where the reference is; the finite entries to the usual bar."""
    fin = torch.isfinite(ref.double())
    assert torch.equal(torch.isfinite(got.double()), fin), f"{name}: non-finite entries differ from the reference's"
    if scale is None:
        assert_close(got[fin], ref[fin], dtype, name=name)
    else:
        assert_reduction_close(got[fin], ref[fin], dtype, scale=scale[fin], name=name)


_LAYOUTS = {
    "rows": None,
    "channel_last": lambda t: t.transpose(1, 2).contiguous().transpose(1, 2),
    "strided": lambda t: torch.stack([t, t], -1)[..., 0],
}


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("seqlen", [1021, 1032])
@pytest.mark.parametrize("mode", ["linear", "silu", "seq_idx"])
@pytest.mark.parametrize("layout", list(_LAYOUTS))
def test_nonfinite_neighbours_do_not_leak(dtype, seqlen, mode, layout):
    """x: channel 2 ends in inf, channel 5 starts with NaN, channel 8 is NaN throughout; dout
    ends in inf in channel 3 and is NaN throughout channel 10. Rows: each shares vectors with
    its neighbours (1021: ragged rows), or is the last row of a segment that lies past the
    row's end (1032: aligned rows). Channel-last: the last run of 128 steps reaches past the
    end. Only the entries that the reference makes non-finite may be non-finite; everything
    else matches it."""
    B, D, W = 2, 12, 4
    x, w, b, _ = make_inputs(B, D, seqlen, W, dtype=dtype)
    dout = make_inputs(B, D, seqlen, W, dtype=dtype, seed=1)[0]
    x[:, 2, -1] = float("inf")
    x[:, 5, 0] = float("nan")
    x[:, 8, :] = float("nan")
    dout[:, 3, -1] = float("inf")
    dout[:, 10, :] = float("nan")
    clean, gclean = (torch.where(torch.isfinite(t), t, torch.zeros_like(t)) for t in (x, dout))
    act = "silu" if mode != "linear" else None
    seq = _leading_padding(B, seqlen) if mode == "seq_idx" else None
    out, _, dx, dw, db, _ = _autograd(x, w, b, dout, seq_idx=seq, activation=act, view=_LAYOUTS[layout])
    rout = O.causal_conv1d_fn(x, w, b, seq_idx=seq, activation=act)
    rdx, rdw, rdb, _ = O.causal_conv1d_bwd(x, w, b, dout, seq_idx=seq, activation=act)
    sw, sb = scales(clean, w, b, gclean, seq_idx=seq, activation=act)
    ok = [c for c in range(D) if c not in (2, 3, 5, 8, 10)]
    assert torch.isfinite(rdw[ok].double()).all(), "the case is what it says"
    _same_nonfinite_then_close(out, rout, dtype, "out")
    _same_nonfinite_then_close(dx, rdx, dtype, "dx")
    _same_nonfinite_then_close(dw, rdw, dtype, "dweight", scale=sw)
    _same_nonfinite_then_close(db, rdb, dtype, "dbias", scale=sb)


_ROW_HEAD_REASON = ("row kernels add a row's first W-1 dpre times the zeros before the row for "
                    "taps the reference skips without initial_states; a non-finite dpre there "
                    "makes all of that channel's weight gradient NaN instead of the taps "
                    "reaching into the row (the exact forms measured cost the kernel a "
                    "wavefront per SIMD)")


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("seqlen", [1021, 1032])
@pytest.mark.parametrize("activation", [None, "silu"])
@pytest.mark.parametrize("layout", [pytest.param("rows", marks=pytest.mark.xfail(strict=True, reason=_ROW_HEAD_REASON)),
                                    "channel_last", "strided"])
def test_nonfinite_dout_at_a_rows_start(dtype, seqlen, activation, layout):
    """dout of channel 6 starts with NaN, no initial_states: the reference's weight gradient is
    NaN only in the tap that reaches the row's first x (bwd_full_cpu/kernel.mojo:264-274 skip
    the taps before the row), the rest of that channel's and every other channel's match."""
    B, D, W = 2, 12, 4
    x, w, b, _ = make_inputs(B, D, seqlen, W, dtype=dtype)
    dout = make_inputs(B, D, seqlen, W, dtype=dtype, seed=1)[0]
    dout[:, 6, 0] = float("nan")
    gclean = torch.where(torch.isfinite(dout), dout, torch.zeros_like(dout))
    _, _, dx, dw, db, _ = _autograd(x, w, b, dout, activation=activation, view=_LAYOUTS[layout])
    rdx, rdw, rdb, _ = O.causal_conv1d_bwd(x, w, b, dout, activation=activation)
    sw, sb = scales(x, w, b, gclean, activation=activation)
    assert int((~torch.isfinite(rdw[6].double())).sum()) == 1, "the case is what it says"
    _same_nonfinite_then_close(dx, rdx, dtype, "dx")
    _same_nonfinite_then_close(dw, rdw, dtype, "dweight", scale=sw)
    _same_nonfinite_then_close(db, rdb, dtype, "dbias", scale=sb)


_ROW_GATE_REASON = ("the row kernels' seq_idx form adds dpre times zero for a tap whose ids differ, "
                    "where the reference adds no term: a non-finite dpre at a sequence's first "
                    "position makes all of that channel's weight gradient NaN (a select per gated "
                    "tap measured 1.5 us slower at C2's shape)")


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("seqlen", [1021, 1032])
@pytest.mark.parametrize("activation", [None, "silu"])
@pytest.mark.parametrize("layout", [pytest.param("rows", marks=pytest.mark.xfail(strict=True, reason=_ROW_GATE_REASON)),
                                    "channel_last", "strided"])
def test_nonfinite_dout_at_a_sequence_start(dtype, seqlen, activation, layout):
    """Two sequences per row; dout of channel 6 is NaN at the second one's first position. The
    reference gates off the taps that reach into the first sequence (no term), so its weight
    gradient is NaN only in the tap on that position's own x, and dx only there."""
    B, D, W = 2, 12, 4
    x, w, b, _ = make_inputs(B, D, seqlen, W, dtype=dtype)
    dout = make_inputs(B, D, seqlen, W, dtype=dtype, seed=1)[0]
    seq = torch.zeros(B, seqlen, dtype=torch.int32)
    seq[:, seqlen // 2:] = 1
    dout[:, 6, seqlen // 2] = float("nan")
    gclean = torch.where(torch.isfinite(dout), dout, torch.zeros_like(dout))
    _, _, dx, dw, db, _ = _autograd(x, w, b, dout, seq_idx=seq, activation=activation, view=_LAYOUTS[layout])
    rdx, rdw, rdb, _ = O.causal_conv1d_bwd(x, w, b, dout, seq_idx=seq, activation=activation)
    sw, sb = scales(x, w, b, gclean, seq_idx=seq, activation=activation)
    assert int((~torch.isfinite(rdw[6].double())).sum()) == 1, "the case is what it says"
    _same_nonfinite_then_close(dx, rdx, dtype, "dx")
    _same_nonfinite_then_close(dw, rdw, dtype, "dweight", scale=sw)
    _same_nonfinite_then_close(db, rdb, dtype, "dbias", scale=sb)


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("seqlen", [5, 1021, 1032])
@pytest.mark.parametrize("activation", [None, "silu"])
@pytest.mark.parametrize("layout", ["rows", "channel_last", "strided"])
def test_nonfinite_initial_states(dtype, seqlen, activation, layout):
    """Channel 1's initial_states hold inf in the slot next to the row, channel 4's a NaN in the
    farthest slot. A ragged row's first vector holds the previous row's elements, which read as
    these states; with SiLU the positions before the row then have an exact zero dpre only
    for finite states, and the reference's weight and bias gradients are NaN for the others.
    Every entry the reference makes non-finite is non-finite here, the rest match it (5, 1021:
    ragged rows; 1032: aligned; the channel-last and generic kernels take the states as their
    first window)."""
    B, D, W = 2, 6, 4
    x, w, b, init = make_inputs(B, D, seqlen, W, dtype=dtype, has_init=True)
    dout = make_inputs(B, D, seqlen, W, dtype=dtype, seed=1)[0]
    clean = init.clone()
    init[:, 1, -1] = float("inf")
    init[:, 4, 0] = float("nan")
    clean[:, 1, -1] = 0
    clean[:, 4, 0] = 0
    out, _, dx, dw, db, di = _autograd(x, w, b, dout, init=init, activation=activation,
                                       view=_LAYOUTS[layout])
    rout = O.causal_conv1d_fn(x, w, b, initial_states=init, activation=activation)
    rdx, rdw, rdb, rdi = O.causal_conv1d_bwd(x, w, b, dout, initial_states=init, activation=activation)
    sw, sb = scales(x, w, b, dout, init=clean, activation=activation)
    ok = [c for c in range(D) if c not in (1, 4)]
    assert torch.isfinite(rdw[ok].double()).all() and not torch.isfinite(rout[:, 1].double()).all(), \
        "the case is what it says"
    _same_nonfinite_then_close(out, rout, dtype, "out")
    _same_nonfinite_then_close(dx, rdx, dtype, "dx")
    _same_nonfinite_then_close(dw, rdw, dtype, "dweight", scale=sw)
    _same_nonfinite_then_close(db, rdb, dtype, "dbias", scale=sb)
    _same_nonfinite_then_close(di, rdi, dtype, "dinitial_states")


# the row planners' segment choices (4 vectors per lane from 129 vectors a row
# when the grid keeps 2048 rows; 2 when a row just past a multiple of 256
# vectors would leave its last 4-vector segment mostly empty), aligned and ragged
SEGMENT_SHAPES = [(2, 1024, 1031), (2, 1024, 1032), (2, 1024, 1536), (1, 2048, 2047), (1, 2048, 2056),
                  (1, 2048, 2100)]


@pytest.mark.parametrize("shape", SEGMENT_SHAPES, ids=[f"B{b}D{d}L{l}" for b, d, l in SEGMENT_SHAPES])
@pytest.mark.parametrize("mode", ["plain", "seq_idx"])
def test_segment_choices(shape, mode):
    B, D, L = shape
    dtype = torch.bfloat16
    x, w, b, _ = make_inputs(B, D, L, 4, dtype=dtype)
    dout = make_inputs(B, D, L, 4, dtype=dtype, seed=1)[0]
    seq = seq_pattern("random_runs", B, L) if mode == "seq_idx" else None
    _check_all(_autograd(x, w, b, dout, seq_idx=seq), x, w, b, dout, dtype, seq_idx=seq)
