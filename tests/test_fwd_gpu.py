"""GPU forward parity: causal_conv1d_fn on MI355X vs the CPU oracle on the
same seeded inputs (tolerances in tests/_util.py).

Coverage follows the reference's tests/test_fwd.py and
tests/test_noncontig_layouts.py: contiguous shapes x dtype x activation x
bias, width sweep 2..9, strided / channel-last / sliced inputs, unaligned
lengths (generic kernel), initial_states, final_states (exact), chunked
round trip, seq_idx patterns, zero-size tensors, torch.compile, plus
multi-segment rows and odd shapes the vector kernels must cut correctly.
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
    conv_f64,
    final_states_expected,
    make_inputs,
    seq_pattern,
)
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _both(x, w, b=None, **kw):
    """Run the GPU op and the oracle on identical inputs; return (gpu, oracle) results on CPU."""
    act = kw.pop("activation", None)
    gpu = cc.causal_conv1d_fn(x.to(DEV), w.to(DEV), None if b is None else b.to(DEV), activation=act,
                              **{k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in kw.items()})
    ref = O.causal_conv1d_fn(x, w, b, activation=act, **kw)
    torch.cuda.synchronize()
    if isinstance(gpu, tuple):
        return tuple(t.cpu() for t in gpu), ref
    return gpu.cpu(), ref


@pytest.mark.parametrize("shape", [(1, 8, 16), (2, 64, 128), (4, 256, 512), (2, 32, 2048), (1, 16, 8192)])
@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("activation", [None, "silu", "swish"])
@pytest.mark.parametrize("has_bias", [True, False], ids=["bias", "nobias"])
def test_contiguous(shape, dtype, activation, has_bias):
    x, w, b, _ = make_inputs(*shape, 4, dtype=dtype, has_bias=has_bias)
    gpu, ref = _both(x, w, b, activation=activation)
    assert gpu.dtype == dtype and gpu.shape == x.shape
    assert_close(gpu, ref, dtype, name="out")


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4, 5, 6, 7, 8, 9])
@pytest.mark.parametrize("seqlen", [128, 1000])
def test_width_sweep(dtype, width, seqlen):
    if dtype == torch.float32 and width > 5:
        pytest.skip("fp32 widths are 2..5 (reference _fn.py:405-414)")
    x, w, b, _ = make_inputs(2, 32, seqlen, width, dtype=dtype)
    gpu, ref = _both(x, w, b, activation="silu")
    assert_close(gpu, ref, dtype)
    assert_close(gpu, conv_f64(x, w, b, silu=True), dtype, name="vs fp64 closed form")


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("seqlen", [1, 2, 3, 5, 7, 13, 100, 517, 2049])
def test_unaligned_lengths(dtype, seqlen):
    x, w, b, _ = make_inputs(3, 24, seqlen, 4, dtype=dtype)
    gpu, ref = _both(x, w, b, activation="silu")
    assert_close(gpu, ref, dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("layout", ["channel_last", "sliced_seq", "channel_slice", "batch_slice"])
def test_strided_x(dtype, layout):
    B, D, L, W = 2, 64, 128, 4
    g = torch.Generator().manual_seed(0)
    if layout == "channel_last":
        base = torch.randn(B, L, D, generator=g).to(dtype)
        view = lambda t: t.transpose(1, 2)  # noqa: E731
    elif layout == "sliced_seq":
        base = torch.randn(B, D, 2 * L, generator=g).to(dtype)
        view = lambda t: t[:, :, :L]  # noqa: E731
    elif layout == "channel_slice":
        base = torch.randn(B, 2 * D, L, generator=g).to(dtype)
        view = lambda t: t[:, ::2, :]  # noqa: E731
    else:
        base = torch.randn(2 * B, D, L, generator=g).to(dtype)
        view = lambda t: t[1::2]  # noqa: E731
    w = torch.randn(D, W, generator=g).to(dtype)
    b = torch.randn(D, generator=g).to(dtype)
    gpu = cc.causal_conv1d_fn(view(base.to(DEV)), w.to(DEV), b.to(DEV), activation="silu").cpu()
    ref = O.causal_conv1d_fn(view(base), w, b, activation="silu")
    assert_close(gpu, ref, dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
def test_noncontiguous_weight_and_bias(dtype):
    x, _, _, _ = make_inputs(2, 64, 128, 4, dtype=dtype)
    w = torch.randn(4, 64).to(dtype).t()
    b = torch.randn(128).to(dtype)[::2]
    gpu = cc.causal_conv1d_fn(x.to(DEV), torch.randn(4, 64).to(dtype).to(DEV).t().copy_(w.to(DEV)),
                              torch.randn(128).to(dtype).to(DEV)[::2].copy_(b.to(DEV)), activation="silu").cpu()
    assert_close(gpu, O.causal_conv1d_fn(x, w, b, activation="silu"), dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4, 5])
@pytest.mark.parametrize("seqlen", [64, 61, 3])
def test_initial_states(dtype, width, seqlen):
    x, w, b, init = make_inputs(2, 16, seqlen, width, dtype=dtype, has_init=True)
    gpu, ref = _both(x, w, b, initial_states=init, activation="silu")
    assert_close(gpu, ref, dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("seqlen", [1, 2, 3, 4, 16, 128, 130, 4096])
@pytest.mark.parametrize("with_init", [False, True])
def test_final_states_exact(dtype, seqlen, with_init):
    x, w, b, init = make_inputs(2, 16, seqlen, 4, dtype=dtype, has_init=with_init)
    (out, fs), (rout, rfs) = _both(x, w, b, initial_states=init, return_final_states=True, activation="silu")
    assert_close(out, rout, dtype)
    assert fs.shape == (2, 16, 3) and fs.dtype == dtype
    assert_equal(fs, rfs, name="final_states")
    assert_equal(fs, final_states_expected(x, 4), name="final_states closed form")


def test_final_states_out_user_buffer_and_zero_length():
    x, w, _, _ = make_inputs(2, 16, 32, 4, dtype=torch.bfloat16)
    fs_out = torch.full((2, 16, 3), 7.0, dtype=torch.bfloat16, device=DEV)
    ptr = fs_out.data_ptr()
    _, fs = cc.causal_conv1d_fn(x.to(DEV), w.to(DEV), return_final_states=True, final_states_out=fs_out)
    assert fs.data_ptr() == ptr
    assert_equal(fs.cpu(), x[..., -3:].contiguous())
    # seqlen 0: the final states are all padding
    x0 = torch.empty(2, 16, 0, dtype=torch.bfloat16, device=DEV)
    fs_out.fill_(7.0)
    out, fs = cc.causal_conv1d_fn(x0, w.to(DEV), return_final_states=True, final_states_out=fs_out)
    assert out.shape == (2, 16, 0)
    assert torch.all(fs.cpu() == 0)


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
def test_chunked_roundtrip(dtype):
    x, w, b, _ = make_inputs(1, 16, 96, 4, dtype=dtype)
    xg, wg, bg = x.to(DEV), w.to(DEV), b.to(DEV)
    full = cc.causal_conv1d_fn(xg, wg, bg, activation="silu")
    init, outs = None, []
    for c in (xg[..., :32], xg[..., 32:64], xg[..., 64:]):
        o, init = cc.causal_conv1d_fn(c, wg, bg, initial_states=init, return_final_states=True, activation="silu")
        outs.append(o)
    assert_close(torch.cat(outs, -1).cpu(), full.cpu(), dtype)


@pytest.mark.parametrize("pattern", SEQ_PATTERNS)
@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("activation", [None, "silu"])
def test_seq_idx(pattern, dtype, activation):
    x, w, b, _ = make_inputs(2, 16, 64, 4, dtype=dtype)
    s = seq_pattern(pattern, 2, 64)
    gpu, ref = _both(x, w, b, seq_idx=s, activation=activation)
    assert_close(gpu, ref, dtype, name=pattern)


@pytest.mark.parametrize("mode", ["no_grad", "inference_mode"])
@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
def test_seq_idx_inference_with_grad_inputs(dtype, mode):
    """Inference on inputs that require grad (reference tests/test_fwd.py:370-383): no
    autograd node is built, the output matches the oracle and requires no grad."""
    x, w, _, _ = make_inputs(1, 16, 32, 4, dtype=dtype)
    s = seq_pattern("random_runs", 1, 32)
    xg, wg = x.to(DEV).requires_grad_(), w.to(DEV).requires_grad_()
    ctx = torch.no_grad() if mode == "no_grad" else torch.inference_mode()
    with ctx:
        out = cc.causal_conv1d_fn(xg, wg, seq_idx=s.to(DEV), activation=None)
    assert not out.requires_grad
    assert_close(out.cpu(), O.causal_conv1d_fn(x, w, None, seq_idx=s, activation=None), dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4, 5])
@pytest.mark.parametrize("seqlen", [64, 4096 + 64, 77])
def test_seq_idx_widths_and_segments(dtype, width, seqlen):
    x, w, b, _ = make_inputs(2, 8, seqlen, width, dtype=dtype)
    s = seq_pattern("random_runs", 2, seqlen)
    gpu, ref = _both(x, w, b, seq_idx=s, activation="silu")
    assert_close(gpu, ref, dtype)


@pytest.mark.parametrize("shape", [(0, 64, 128), (2, 0, 128), (2, 64, 0), (0, 0, 0)])
def test_zero_sized(shape):
    x = torch.randn(*shape, dtype=torch.bfloat16, device=DEV)
    w = torch.randn(shape[1], 4, dtype=torch.bfloat16, device=DEV)
    out = cc.causal_conv1d_fn(x, w, activation="silu")
    assert out.shape == x.shape and out.numel() == 0


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
def test_multi_segment_rows(dtype):
    """Rows longer than one wavefront segment (halo handed across segments) and
    channel counts that leave partial blocks."""
    x, w, b, _ = make_inputs(3, 5, 16384 + 8 * 64, 4, dtype=dtype)
    gpu, ref = _both(x, w, b, activation="silu")
    assert_close(gpu, ref, dtype)


def test_repeat_calls_are_deterministic():
    x, w, b, _ = make_inputs(2, 64, 2048, 4, dtype=torch.bfloat16)
    xg, wg, bg = x.to(DEV), w.to(DEV), b.to(DEV)
    first = cc.causal_conv1d_fn(xg, wg, bg, activation="silu")
    for _ in range(3):
        assert torch.equal(cc.causal_conv1d_fn(xg, wg, bg, activation="silu"), first)


_COMPILE_BACKEND = "aot_eager"


def test_torch_compile_fullgraph():
    x, w, b, _ = make_inputs(2, 64, 128, 4, dtype=torch.float16, device=DEV)

    @torch.compile(fullgraph=True, backend=_COMPILE_BACKEND)
    def f(x, w, b):
        return cc.causal_conv1d_fn(x, w, b, activation="silu")

    assert torch.equal(f(x, w, b), cc.causal_conv1d_fn(x, w, b, activation="silu"))


def test_torch_compile_autograd():
    x, w, b, _ = make_inputs(2, 64, 128, 4, dtype=torch.float16, device=DEV)
    x.requires_grad_(), w.requires_grad_(), b.requires_grad_()

    @torch.compile(backend=_COMPILE_BACKEND)
    def f(x, w, b):
        return cc.causal_conv1d_fn(x, w, b, activation="silu").sum()

    f(x, w, b).backward()
    assert x.grad.shape == x.shape and w.grad.shape == w.shape and b.grad.shape == b.shape


def test_launch_status_ignores_an_earlier_unrelated_error():
    """A kernel launch reports its own status: an error that an unrelated HIP call left pending on
    the thread (here an invalid device number) is not returned as the library's failure."""
    import ctypes
    import os

    from causal_conv1d_amd._native import native_fwd

    hip = ctypes.CDLL("libamdhip64.so.7", mode=os.RTLD_NOLOAD)  # the runtime torch and the library share
    hip.hipSetDevice.argtypes = [ctypes.c_int]
    x, w, b, _ = make_inputs(2, 64, 512, 4, dtype=torch.bfloat16, device=DEV)
    out = torch.empty_like(x)
    torch.cuda.synchronize()
    try:
        assert hip.hipSetDevice(-1) != 0  # refused: leaves an error on the thread, touches no GPU state
        native_fwd(x, w, b, None, None, out, True)  # raises if cc1d_fwd returns a status other than OK
    finally:
        hip.hipGetLastError()  # take the planted error off the thread before torch checks it
    torch.cuda.synchronize()
    assert_close(out.cpu(), O.causal_conv1d_fn(x.cpu(), w.cpu(), b.cpu(), activation="silu"), torch.bfloat16)
