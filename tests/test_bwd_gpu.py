"""GPU backward parity: autograd through causal_conv1d_fn on MI355X vs the
oracle's backward assembly (oracle.causal_conv1d_bwd, which restates
_fn.py:258-332 around bwd_full_cpu/kernel.mojo) on the same inputs.

Coverage follows the reference's tests/test_bwd.py and the backward half of
tests/test_noncontig_layouts.py: width sweep, shapes x activation x bias,
grad dtypes, dfinal_states tail, initial_states grads, seq_idx grads,
zero-size, strided layouts; plus unaligned and multi-segment rows.
"""

from __future__ import annotations

import pytest
import torch

import causal_conv1d_amd as cc
from _util import (
    DTYPE_IDS,
    DTYPES,
    SEQ_PATTERNS,
    assert_close,
    assert_reduction_close,
    grads_f64,
    make_inputs,
    scales,
    seq_pattern,
)
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _gpu_grads(x, w, b, dout, *, init=None, seq_idx=None, activation=None, dfs=None, view=None):
    """Leaf tensors on the GPU (optionally through a layout `view`), forward + backward."""
    xg = x.to(DEV).requires_grad_()
    wg = w.to(DEV).requires_grad_()
    bg = b.to(DEV).requires_grad_() if b is not None else None
    ig = init.to(DEV).requires_grad_() if init is not None else None
    xin = view(xg) if view is not None else xg
    kw = dict(initial_states=ig, activation=activation,
              seq_idx=None if seq_idx is None else seq_idx.to(DEV))
    if dfs is not None:
        out, fs = cc.causal_conv1d_fn(xin, wg, bg, return_final_states=True, **kw)
        torch.autograd.backward([out, fs], [dout.to(DEV), dfs.to(DEV)])
    else:
        out = cc.causal_conv1d_fn(xin, wg, bg, **kw)
        out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    return (xg.grad.cpu(), wg.grad.cpu(), None if bg is None else bg.grad.cpu(),
            None if ig is None else ig.grad.cpu())


def _check(got, ref, dtype, scale, has_init=False):
    dx, dw, db, di = got
    rdx, rdw, rdb, rdi = ref
    sw, sb = scale
    assert dx.dtype == dtype and dw.dtype == dtype
    assert_close(dx, rdx, dtype, name="dx")
    assert_reduction_close(dw, rdw, dtype, scale=sw, name="dweight")
    if rdb is not None:
        assert db.dtype == dtype
        assert_reduction_close(db, rdb, dtype, scale=sb, name="dbias")
    if has_init:
        assert_close(di, rdi, dtype, name="dinitial_states")


@pytest.mark.parametrize("shape", [(1, 8, 16), (2, 64, 128), (4, 256, 512), (2, 32, 2048), (1, 8, 8192)])
@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("activation", [None, "silu"])
@pytest.mark.parametrize("has_bias", [True, False], ids=["bias", "nobias"])
def test_backward_contiguous(shape, dtype, activation, has_bias):
    x, w, b, _ = make_inputs(*shape, 4, dtype=dtype, has_bias=has_bias)
    dout = make_inputs(*shape, 4, dtype=dtype, seed=1)[0]
    got = _gpu_grads(x, w, b, dout, activation=activation)
    _check(got, O.causal_conv1d_bwd(x, w, b, dout, activation=activation), dtype,
           scales(x, w, b, dout, activation=activation))


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4, 5, 6, 7, 8, 9])
@pytest.mark.parametrize("seqlen", [128, 1000])
def test_backward_width_sweep(dtype, width, seqlen):
    if dtype == torch.float32 and width > 5:
        pytest.skip("fp32 widths are 2..5")
    x, w, b, _ = make_inputs(2, 32, seqlen, width, dtype=dtype)
    dout = make_inputs(2, 32, seqlen, width, dtype=dtype, seed=1)[0]
    got = _gpu_grads(x, w, b, dout, activation="silu")
    _check(got, O.causal_conv1d_bwd(x, w, b, dout, activation="silu"), dtype, scales(x, w, b, dout, activation="silu"))


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("seqlen", [1, 2, 3, 5, 13, 100, 517, 2049, 4096 + 72])
def test_backward_unaligned_and_segmented(dtype, seqlen):
    x, w, b, _ = make_inputs(3, 12, seqlen, 4, dtype=dtype)
    dout = make_inputs(3, 12, seqlen, 4, dtype=dtype, seed=1)[0]
    got = _gpu_grads(x, w, b, dout, activation="silu")
    _check(got, O.causal_conv1d_bwd(x, w, b, dout, activation="silu"), dtype, scales(x, w, b, dout, activation="silu"))


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4])
@pytest.mark.parametrize("seqlen", [64, 62, 2, 8192])
def test_final_states_backward(dtype, width, seqlen):
    x, w, b, _ = make_inputs(2, 16, seqlen, width, dtype=dtype)
    dout = make_inputs(2, 16, seqlen, width, dtype=dtype, seed=1)[0]
    dfs = make_inputs(2, 16, width - 1, width, dtype=dtype, seed=2)[0]
    got = _gpu_grads(x, w, b, dout, activation="silu", dfs=dfs)
    _check(got, O.causal_conv1d_bwd(x, w, b, dout, dfinal_states=dfs, activation="silu"), dtype,
           scales(x, w, b, dout, activation="silu"))


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4, 5])
@pytest.mark.parametrize("seqlen", [64, 67, 2])
@pytest.mark.parametrize("has_bias", [True, False], ids=["bias", "nobias"])
def test_initial_states_backward(dtype, width, seqlen, has_bias):
    x, w, b, init = make_inputs(2, 16, seqlen, width, dtype=dtype, has_init=True, has_bias=has_bias)
    dout = make_inputs(2, 16, seqlen, width, dtype=dtype, seed=1)[0]
    got = _gpu_grads(x, w, b, dout, init=init, activation="silu")
    ref = O.causal_conv1d_bwd(x, w, b, dout, initial_states=init, activation="silu")
    _check(got, ref, dtype, scales(x, w, b, dout, init=init, activation="silu"), has_init=True)


@pytest.mark.parametrize("pattern", SEQ_PATTERNS)
@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("activation", [None, "silu"])
def test_seq_idx_backward(pattern, dtype, activation):
    x, w, b, _ = make_inputs(2, 16, 64, 4, dtype=dtype)
    dout = make_inputs(2, 16, 64, 4, dtype=dtype, seed=1)[0]
    s = seq_pattern(pattern, 2, 64)
    got = _gpu_grads(x, w, b, dout, seq_idx=s, activation=activation)
    _check(got, O.causal_conv1d_bwd(x, w, b, dout, seq_idx=s, activation=activation), dtype,
           scales(x, w, b, dout, seq_idx=s, activation=activation))


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("seqlen", [4096 + 128, 77])
def test_seq_idx_backward_segments(dtype, seqlen):
    x, w, b, _ = make_inputs(2, 8, seqlen, 4, dtype=dtype)
    dout = make_inputs(2, 8, seqlen, 4, dtype=dtype, seed=1)[0]
    s = seq_pattern("random_runs", 2, seqlen)
    got = _gpu_grads(x, w, b, dout, seq_idx=s, activation="silu")
    _check(got, O.causal_conv1d_bwd(x, w, b, dout, seq_idx=s, activation="silu"), dtype,
           scales(x, w, b, dout, seq_idx=s, activation="silu"))


_NONFINITE_VIEWS = {
    "rows": None,
    "channel_last": lambda t: t.transpose(1, 2).contiguous().transpose(1, 2),
    "strided": lambda t: torch.stack([t, t], -1)[..., 0],
}


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("layout", list(_NONFINITE_VIEWS))
def test_seq_idx_nonfinite_padding_follows_the_reference(dtype, layout):
    """Padding positions (negative ids) holding NaN / inf in x and dout. dpre there is zero
    whatever they hold (bwd_full_cpu/kernel.mojo:75-77), so the output, dx and dbias stay
    finite; the weight gradient adds 0 * x over a padding run's kept taps (kernel.mojo:264-274),
    which is NaN exactly where such an x is not finite, as in the reference. The finite
    entries are compared as usual."""
    B, D, L, W = 2, 16, 1024, 4
    x, w, b, _ = make_inputs(B, D, L, W, dtype=dtype)
    dout = make_inputs(B, D, L, W, dtype=dtype, seed=1)[0]
    s = seq_pattern("with_padding", B, L).clone()  # positions 16..31 padded (-1)
    s[:, 600:610] = -3                               # a second run, another negative id
    pad = s[0] < 0
    clean_x, clean_g = x.clone(), dout.clone()
    clean_x[:, :, pad] = 0
    clean_g[:, :, pad] = 0
    x[:, : D // 2, 16:32] = float("nan")             # channels 0..7: NaN through the first run
    x[:, D // 2 : 3 * D // 4, 603] = float("inf")    # channels 8..11: one inf in the second
    dout[:, :, pad] = float("nan")                   # every channel: NaN dout at padding
    xg = x.to(DEV).requires_grad_()
    wg = w.to(DEV).requires_grad_()
    bg = b.to(DEV).requires_grad_()
    view = _NONFINITE_VIEWS[layout]
    out = cc.causal_conv1d_fn(xg if view is None else view(xg), wg, bg, seq_idx=s.to(DEV), activation="silu")
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    rout = O.causal_conv1d_fn(x, w, b, seq_idx=s, activation="silu")
    rdx, rdw, rdb, _ = O.causal_conv1d_bwd(x, w, b, dout, seq_idx=s, activation="silu")
    assert_close(out.detach().cpu(), rout, dtype, name="out")
    assert_close(xg.grad.cpu(), rdx, dtype, name="dx")
    sw, sb = scales(clean_x, w, b, clean_g, seq_idx=s, activation="silu")
    assert_reduction_close(bg.grad.cpu(), rdb, dtype, scale=sb, name="dbias")
    dw = wg.grad.cpu()
    bad = ~torch.isfinite(rdw.double())
    assert bad[: 3 * D // 4].all() and not bad[3 * D // 4 :].any()  # the case is what it says
    assert torch.equal(torch.isnan(dw), bad), "dweight: non-finite entries differ from the reference's"
    assert_reduction_close(dw[~bad], rdw[~bad], dtype, scale=sw[~bad], name="dweight")


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4, 5, 6, 7, 8, 9])
@pytest.mark.parametrize("pattern", ["repeat_ids", "with_padding"])
def test_seq_idx_backward_widths_across_lanes_and_segments(dtype, width, pattern):
    """The seq_idx row backward scatters dx across lanes, vectors and segments (a carry per
    lane boundary, the next segment's first W-1 positions recomputed): every width, a row of
    3 segments (the last one partial), ids that reappear inside a window or are padded."""
    if dtype == torch.float32 and width > 5:
        pytest.skip("fp32 widths above 5 are rejected by the API (reference _fn.py:405-414)")
    L = 4096 + 2 * 128 + 8  # bf16/fp16: 3 segments of up to 2048; fp32: 5 of up to 1024
    x, w, b, _ = make_inputs(2, 6, L, width, dtype=dtype)
    dout = make_inputs(2, 6, L, width, dtype=dtype, seed=1)[0]
    s = seq_pattern(pattern, 2, L)
    got = _gpu_grads(x, w, b, dout, seq_idx=s, activation="silu")
    _check(got, O.causal_conv1d_bwd(x, w, b, dout, seq_idx=s, activation="silu"), dtype,
           scales(x, w, b, dout, seq_idx=s, activation="silu"))


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("layout", ["channel_last", "channel_slice", "sliced_seq"])
def test_backward_strided(dtype, layout):
    B, D, L, W = 2, 64, 128, 4
    if layout == "channel_last":
        base_shape, view = (B, L, D), (lambda t: t.transpose(1, 2))
    elif layout == "channel_slice":
        base_shape, view = (B, 2 * D, L), (lambda t: t[:, ::2, :])
    else:
        base_shape, view = (B, D, 2 * L), (lambda t: t[:, :, :L])
    g = torch.Generator().manual_seed(0)
    base = torch.randn(*base_shape, generator=g).to(dtype)
    w = torch.randn(D, W, generator=g).to(dtype)
    b = torch.randn(D, generator=g).to(dtype)
    dout = torch.randn(B, D, L, generator=g).to(dtype)
    dbase, dw, db, _ = _gpu_grads(base, w, b, dout, activation="silu", view=view)
    rdx, rdw, rdb, _ = O.causal_conv1d_bwd(view(base), w, b, dout, activation="silu")
    sw, sb = scales(view(base), w, b, dout, activation="silu")
    assert_close(view(dbase), rdx, dtype, name="dx")
    assert_reduction_close(dw, rdw, dtype, scale=sw, name="dweight")
    assert_reduction_close(db, rdb, dtype, scale=sb, name="dbias")


def test_backward_vs_fp64_autograd():
    """Direct check against float64 autograd of the closed form (not via the oracle)."""
    x, w, b, init = make_inputs(2, 32, 256, 4, dtype=torch.float32, has_init=True)
    dout = torch.randn(x.shape)
    got = _gpu_grads(x, w, b, dout, init=init, activation="silu")
    _check(got, grads_f64(x, w, b, dout, init=init, silu=True), torch.float32,
           scales(x, w, b, dout, init=init, activation="silu"), has_init=True)


def test_expanded_dout_from_sum():
    x, w, b, _ = make_inputs(2, 64, 128, 4, dtype=torch.float16)
    xg, wg, bg = (t.to(DEV).requires_grad_() for t in (x, w, b))
    cc.causal_conv1d_fn(xg, wg, bg, activation="silu").sum().backward()
    rdx, rdw, rdb, _ = O.causal_conv1d_bwd(x, w, b, torch.ones_like(x), activation="silu")
    assert_close(xg.grad.cpu(), rdx, torch.float16)
    assert_reduction_close(wg.grad.cpu(), rdw, torch.float16,
                           scale=scales(x, w, b, torch.ones_like(x), activation="silu")[0])


@pytest.mark.parametrize("shape", [(0, 64, 128), (2, 0, 128), (2, 64, 0), (0, 0, 0)])
@pytest.mark.parametrize("has_init", [False, True])
def test_zero_sized_backward(shape, has_init):
    B, D, L = shape
    x = torch.randn(B, D, L, dtype=torch.bfloat16, device=DEV, requires_grad=True)
    w = torch.randn(D, 4, dtype=torch.bfloat16, device=DEV, requires_grad=True)
    b = torch.randn(D, dtype=torch.bfloat16, device=DEV, requires_grad=True)
    init = torch.randn(B, D, 3, dtype=torch.bfloat16, device=DEV, requires_grad=True) if has_init else None
    out = cc.causal_conv1d_fn(x, w, b, initial_states=init, activation="silu")
    out.backward(torch.randn_like(out))
    assert x.grad.shape == x.shape and w.grad.shape == w.shape and b.grad.shape == b.shape
    assert torch.all(w.grad == 0) and torch.all(b.grad == 0)
    if has_init:
        assert torch.all(init.grad == 0)


def test_backward_repeat_single_contribution_is_bit_identical():
    """One (batch, segment) per channel: repeated backward passes agree bit for bit."""
    x, w, b, _ = make_inputs(1, 128, 2048, 4, dtype=torch.bfloat16)
    dout = make_inputs(1, 128, 2048, 4, dtype=torch.bfloat16, seed=1)[0]
    a = _gpu_grads(x, w, b, dout, activation="silu")
    for _ in range(2):
        again = _gpu_grads(x, w, b, dout, activation="silu")
        for u, v in zip(a, again):
            if u is not None:
                assert torch.equal(u, v)


@pytest.mark.parametrize("layout", ["rows", "channel_last", "strided"])
def test_backward_repeat_multi_batch_is_bit_identical(layout):
    """Several batches and segments per channel: the autograd backward adds each channel's
    partial sums in a fixed order, so repeats agree bit for bit (the reference's fp32
    atomics, bwd_full/kernel.mojo:766-800, do not promise that)."""
    x, w, b, _ = make_inputs(4, 128, 2048, 4, dtype=torch.float32)
    dout = make_inputs(4, 128, 2048, 4, dtype=torch.float32, seed=1)[0]
    view = {"rows": None, "channel_last": lambda t: t.transpose(1, 2), "strided": lambda t: t[..., 0]}[layout]
    if layout == "channel_last":
        x = x.transpose(1, 2).contiguous()
    elif layout == "strided":
        x = torch.stack([x, x], -1)
    a = _gpu_grads(x, w, b, dout, activation="silu", view=view)
    for _ in range(2):
        again = _gpu_grads(x, w, b, dout, activation="silu", view=view)
        for u, v in zip(a, again):
            if u is not None:
                assert torch.equal(u, v)


def _op_both(x, w, b, dout, *, seq_idx=None, init=None, dfs=None, silu=True):
    """The reference-shaped op (_bwd_full_inplace: fp32 accumulators, then casts) and the
    autograd backward's op (_bwd_typed_inplace) on the same GPU inputs."""
    xg, wg, doutg = x.to(DEV), w.to(DEV), dout.to(DEV)
    bg = b.to(DEV) if b is not None else None
    sg = seq_idx.to(DEV) if seq_idx is not None else None
    ig = init.to(DEV) if init is not None else None
    fg = dfs.to(DEV) if dfs is not None else None
    D, W = w.shape
    dx1 = torch.empty_like(xg)
    dwa = torch.zeros(D, W, dtype=torch.float32, device=DEV)
    dba = torch.zeros(D, dtype=torch.float32, device=DEV) if b is not None else None
    di1 = torch.empty_like(ig) if ig is not None else None
    torch.ops.causal_conv1d_amd._bwd_full_inplace(xg, wg, bg, doutg, sg, ig, dx1, dwa, dba, di1, silu, fg)
    dx2 = torch.empty_like(xg)
    dw2 = torch.empty(D, W, dtype=w.dtype, device=DEV)
    db2 = torch.empty(D, dtype=w.dtype, device=DEV) if b is not None else None
    di2 = torch.empty_like(ig) if ig is not None else None
    torch.ops.causal_conv1d_amd._bwd_typed_inplace(xg, wg, bg, doutg, sg, ig, fg, dx2, dw2, db2, di2, silu)
    torch.cuda.synchronize()
    acc = (dx1, dwa.to(w.dtype), None if dba is None else dba.to(w.dtype), di1)
    return acc, (dx2, dw2, db2, di2)


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("layout", ["rows", "channel_last", "strided"])
@pytest.mark.parametrize("case", ["plain", "nobias", "seq_idx", "states"])
def test_typed_op_matches_accumulator_op(dtype, layout, case):
    """Both backward ops run the same kernel: dx / dinitial_states are identical and the
    weight/bias gradients differ at most by the order of the fp32 additions."""
    B, D, L, W = 3, 96, 700, 4
    x, w, b, init = make_inputs(B, D, L, W, dtype=dtype, has_init=True)
    dout = make_inputs(B, D, L, W, dtype=dtype, seed=1)[0]
    if case == "nobias":
        b = None
    seq = seq_pattern("random_runs", B, L) if case == "seq_idx" else None
    if case != "states":
        init = None
    dfs = make_inputs(B, D, W - 1, W, dtype=dtype, seed=2)[0] if case == "states" else None
    # the layouts are made on the GPU (a host tensor with gaps would arrive contiguous)
    x, dout = x.to(DEV), dout.to(DEV)
    if layout == "channel_last":
        x = x.transpose(1, 2).contiguous().transpose(1, 2)
        dout = dout.transpose(1, 2).contiguous().transpose(1, 2)
    elif layout == "strided":
        x = torch.stack([x, x], -1)[..., 0]
        dout = torch.stack([dout, dout], -1)[..., 1]
    assert layout != "strided" or x.stride(-1) == 2
    acc, typed = _op_both(x, w, b, dout, seq_idx=seq, init=init, dfs=dfs)
    x, dout = x.cpu(), dout.cpu()
    sw, sb = scales(x, w, b, dout, init=init, seq_idx=seq, activation="silu")
    assert torch.equal(acc[0], typed[0])
    assert_reduction_close(typed[1], acc[1], dtype, scale=sw, name="dweight")
    if b is not None:
        assert_reduction_close(typed[2], acc[2], dtype, scale=sb, name="dbias")
    else:
        assert typed[2] is None
    if init is not None:
        assert torch.equal(acc[3], typed[3])
    ref = O.causal_conv1d_bwd(x.contiguous(), w, b, dout.contiguous(), seq_idx=seq, initial_states=init,
                              dfinal_states=dfs, activation="silu")
    assert_close(typed[0].cpu(), ref[0], dtype, name="dx")
    assert_reduction_close(typed[1].cpu(), ref[1], dtype, scale=sw, name="dweight")
