"""Channel-last inputs (x viewed from a (batch, seqlen, dim) buffer, unit
channel stride) on MI355X vs the oracle, forward and backward.

The reference runs this layout through its strided path
(tests/test_noncontig_layouts.py); here it has its own tiled kernels, so the
tile edges get their own cases: sequence lengths around the 16-step tile,
shorter than the halo, dims that leave a partial channel group, odd dims (the
generic fallback), seq_idx patterns whose boundaries fall inside tiles
(including ids that reappear within one window), padding, initial and final
states with their gradients, and widths 2..9.
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
    assert_equal,
    assert_reduction_close,
    make_inputs,
    scales,
    seq_pattern,
)
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cl(t):
    """(B, D, L) values in a channel-last buffer on the GPU: strides (L*D, 1, D)."""
    return t.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)


def _widths(dtype):
    return [2, 3, 4, 5] if dtype == torch.float32 else [2, 3, 4, 5, 9]


def _fwd_cases():
    for dtype, did in zip(DTYPES, DTYPE_IDS):
        for width in _widths(dtype):
            yield pytest.param(dtype, width, id=f"{did}-w{width}")


@pytest.mark.parametrize("dtype,width", list(_fwd_cases()))
@pytest.mark.parametrize("seqlen", [1, 3, 16, 17, 100, 515])
@pytest.mark.parametrize("dim", [64, 130, 33])
def test_cl_forward(dtype, width, seqlen, dim):
    x, w, b, _ = make_inputs(2, dim, seqlen, width, dtype=dtype)
    xg = _cl(x)
    assert xg.stride(1) == 1
    gpu = cc.causal_conv1d_fn(xg, w.to(DEV), b.to(DEV), activation="silu").cpu()
    assert_close(gpu, O.causal_conv1d_fn(x, w, b, activation="silu"), dtype)


@pytest.mark.parametrize("pattern", SEQ_PATTERNS)
@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 4, 5])
@pytest.mark.parametrize("seqlen", [40, 515])
def test_cl_forward_seq_idx(pattern, dtype, width, seqlen):
    x, w, b, _ = make_inputs(2, 130, seqlen, width, dtype=dtype)
    s = seq_pattern(pattern, 2, seqlen)
    gpu = cc.causal_conv1d_fn(_cl(x), w.to(DEV), b.to(DEV), seq_idx=s.to(DEV), activation="silu").cpu()
    assert_close(gpu, O.causal_conv1d_fn(x, w, b, seq_idx=s, activation="silu"), dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 4, 5])
@pytest.mark.parametrize("seqlen", [1, 2, 3, 20, 100])
def test_cl_forward_states(dtype, width, seqlen):
    x, w, b, init = make_inputs(2, 64, seqlen, width, dtype=dtype, has_init=True)
    out, fs = cc.causal_conv1d_fn(_cl(x), w.to(DEV), b.to(DEV), initial_states=init.to(DEV),
                                  return_final_states=True, activation="silu")
    rout, rfs = O.causal_conv1d_fn(x, w, b, initial_states=init, return_final_states=True, activation="silu")
    assert_close(out.cpu(), rout, dtype)
    assert_equal(fs.cpu(), rfs, name="final_states")


def _grads(x, w, b, dout, *, init=None, seq_idx=None, dfs=None, activation="silu"):
    """Autograd through a channel-last view; gradients come back as (B, D, L) values."""
    base = x.transpose(1, 2).contiguous().to(DEV).requires_grad_()
    wg = w.to(DEV).requires_grad_()
    bg = b.to(DEV).requires_grad_()
    ig = init.to(DEV).requires_grad_() if init is not None else None
    kw = dict(initial_states=ig, activation=activation, seq_idx=None if seq_idx is None else seq_idx.to(DEV))
    if dfs is not None:
        out, fs = cc.causal_conv1d_fn(base.transpose(1, 2), wg, bg, return_final_states=True, **kw)
        torch.autograd.backward([out, fs], [dout.to(DEV), dfs.to(DEV)])
    else:
        cc.causal_conv1d_fn(base.transpose(1, 2), wg, bg, **kw).backward(dout.to(DEV))
    torch.cuda.synchronize()
    return (base.grad.transpose(1, 2).cpu(), wg.grad.cpu(), bg.grad.cpu(),
            None if ig is None else ig.grad.cpu())


def _check(got, ref, dtype, scale, has_init=False):
    dx, dw, db, di = got
    rdx, rdw, rdb, rdi = ref
    sw, sb = scale
    assert_close(dx, rdx, dtype, name="dx")
    assert_reduction_close(dw, rdw, dtype, scale=sw, name="dweight")
    assert_reduction_close(db, rdb, dtype, scale=sb, name="dbias")
    if has_init:
        assert_close(di, rdi, dtype, name="dinitial_states")


@pytest.mark.parametrize("dtype,width", list(_fwd_cases()))
@pytest.mark.parametrize("seqlen", [1, 3, 16, 17, 100, 515])
@pytest.mark.parametrize("dim", [64, 130, 33])
def test_cl_backward(dtype, width, seqlen, dim):
    x, w, b, _ = make_inputs(2, dim, seqlen, width, dtype=dtype)
    dout = make_inputs(2, dim, seqlen, width, dtype=dtype, seed=1)[0]
    _check(_grads(x, w, b, dout), O.causal_conv1d_bwd(x, w, b, dout, activation="silu"), dtype,
           scales(x, w, b, dout, activation="silu"))


@pytest.mark.parametrize("pattern", SEQ_PATTERNS)
@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 4, 5])
@pytest.mark.parametrize("seqlen", [40, 515])
def test_cl_backward_seq_idx(pattern, dtype, width, seqlen):
    x, w, b, _ = make_inputs(2, 130, seqlen, width, dtype=dtype)
    dout = make_inputs(2, 130, seqlen, width, dtype=dtype, seed=1)[0]
    s = seq_pattern(pattern, 2, seqlen)
    _check(_grads(x, w, b, dout, seq_idx=s), O.causal_conv1d_bwd(x, w, b, dout, seq_idx=s, activation="silu"), dtype,
           scales(x, w, b, dout, seq_idx=s, activation="silu"))


@pytest.mark.parametrize("dtype,width", list(_fwd_cases()))
@pytest.mark.parametrize("pattern", ["with_padding", "repeat_ids", "random_runs"])
@pytest.mark.parametrize("activation", [None, "silu"])
def test_cl_backward_seq_idx_widths(dtype, width, pattern, activation):
    """Tiles holding a boundary at every width, with and without SiLU; 3 batches and 4 tile
    groups per row, so boundary tiles sit among ordinary ones in one block."""
    x, w, b, _ = make_inputs(3, 192, 300, width, dtype=dtype)
    dout = make_inputs(3, 192, 300, width, dtype=dtype, seed=1)[0]
    s = seq_pattern(pattern, 3, 300)
    got = _grads(x, w, b, dout, seq_idx=s, activation=activation)
    _check(got, O.causal_conv1d_bwd(x, w, b, dout, seq_idx=s, activation=activation), dtype,
           scales(x, w, b, dout, seq_idx=s, activation=activation))


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 4, 5])
@pytest.mark.parametrize("seqlen", [1, 2, 3, 20, 100])
def test_cl_backward_states(dtype, width, seqlen):
    x, w, b, init = make_inputs(2, 64, seqlen, width, dtype=dtype, has_init=True)
    dout = make_inputs(2, 64, seqlen, width, dtype=dtype, seed=1)[0]
    dfs = make_inputs(2, 64, width - 1, width, dtype=dtype, seed=2)[0]
    got = _grads(x, w, b, dout, init=init, dfs=dfs)
    ref = O.causal_conv1d_bwd(x, w, b, dout, initial_states=init, dfinal_states=dfs, activation="silu")
    _check(got, ref, dtype, scales(x, w, b, dout, init=init, activation="silu"), has_init=True)


def test_cl_backward_many_tile_groups():
    """Several blocks per row (1024 time steps each) and several batches: the LDS block
    reduction feeds each channel's accumulators from many blocks, and every run hands its
    last dx rows across a chunk, run and block edge (the sequence ends inside a run)."""
    x, w, b, _ = make_inputs(3, 256, 2600, 4, dtype=torch.bfloat16)
    dout = make_inputs(3, 256, 2600, 4, dtype=torch.bfloat16, seed=1)[0]
    _check(_grads(x, w, b, dout), O.causal_conv1d_bwd(x, w, b, dout, activation="silu"), torch.bfloat16,
           scales(x, w, b, dout, activation="silu"))


# the channel-last backward walks runs of the longest of 128, 64 and 16 steps
# that gives 2048 wavefronts (a wavefront per 64 lanes' channels and run):
# one shape per run length, the sequence ending inside a run
_RUN_SHAPES = {"run128": (2, 1024, 16392), "run64": (2, 1024, 8200), "run16": (1, 768, 2050)}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("run", list(_RUN_SHAPES))
@pytest.mark.parametrize("mode", ["plain", "seq_idx", "states"])
def test_cl_backward_run_lengths(dtype, run, mode):
    B, D, L = _RUN_SHAPES[run]
    if dtype == torch.float32:
        D //= 2  # one channel per lane instead of two: the same wavefronts
    x, w, b, init = make_inputs(B, D, L, 4, dtype=dtype, has_init=True)
    dout = make_inputs(B, D, L, 4, dtype=dtype, seed=1)[0]
    if mode != "states":
        init = None
    dfs = make_inputs(B, D, 3, 4, dtype=dtype, seed=2)[0] if mode == "states" else None
    s = seq_pattern("random_runs", B, L) if mode == "seq_idx" else None
    got = _grads(x, w, b, dout, init=init, seq_idx=s, dfs=dfs)
    ref = O.causal_conv1d_bwd(x, w, b, dout, seq_idx=s, initial_states=init, dfinal_states=dfs, activation="silu")
    _check(got, ref, dtype, scales(x, w, b, dout, init=init, seq_idx=s, activation="silu"), has_init=init is not None)


# sequence starts on and next to the edges of 4- and 8-step chunks, 128-step runs and
# 1024-step blocks, a padding stretch (-1) across a run edge, and an id that comes back
_EDGE_CUTS = [1, 3, 4, 127, 128, 131, 700, 1021, 1024, 1025, 1600, 2047, 2048, 2300]


def _edge_seq_idx(batch, seqlen):
    ids = torch.zeros(batch, seqlen, dtype=torch.int32)
    for i, c in enumerate(_EDGE_CUTS):
        ids[:, c:] = i + 1
    ids[:, 1900:2010] = -1
    ids[:, 2400:2450] = 5
    ids[1] = ids[1].roll(37)
    return ids


@pytest.mark.parametrize("dtype,width", [(torch.bfloat16, 4), (torch.float32, 3), (torch.float16, 7),
                                         (torch.bfloat16, 9)])
def test_cl_backward_seq_idx_run_edges(dtype, width):
    """seq_idx boundaries at chunk, run and block edges over several blocks per row."""
    x, w, b, _ = make_inputs(2, 256, 2600, width, dtype=dtype)
    dout = make_inputs(2, 256, 2600, width, dtype=dtype, seed=1)[0]
    s = _edge_seq_idx(2, 2600)
    _check(_grads(x, w, b, dout, seq_idx=s), O.causal_conv1d_bwd(x, w, b, dout, seq_idx=s, activation="silu"), dtype,
           scales(x, w, b, dout, seq_idx=s, activation="silu"))
