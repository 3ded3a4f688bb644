"""cc1d_bwd_typed_noalloc: the typed backward with the library's static device
scratch as its workspace, for callers that cannot allocate.

Through the C ABI it must give what cc1d_bwd_typed gives (same kernels, same
fixed-order reduction: bit-identical dx, dweight, dbias, dinitial_states), on
two calls in a row, the second with a smaller problem (the scratch keeps the
first call's partial sums, which the second must not see). A problem needing
more than CC1D_NOALLOC_WORKSPACE_FLOATS of workspace is refused before any
HIP call.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from _util import make_inputs, seq_pattern
from causal_conv1d_amd import _lib
from causal_conv1d_amd._native import native_bwd_typed, native_bwd_typed_noalloc

DEV = "cuda"
ERR_SCRATCH_LIMIT = 9


def _problem(case, B, D, L, dtype, seed):
    """GPU inputs of one backward call: (x, w, b, dout, seq_idx, init, dfinal_states)."""
    W = 4
    x, w, b, init = make_inputs(B, D, L, W, dtype=dtype, has_init=True, seed=seed)
    dout = make_inputs(B, D, L, W, dtype=dtype, seed=seed + 1)[0]
    seq = dfs = None
    if case == "seq_idx":
        seq = seq_pattern("random_runs", B, L)
        init = None
    elif case == "states":
        dfs = make_inputs(B, D, W - 1, W, dtype=dtype, seed=seed + 2)[0]
    else:
        init = None
    x, dout = x.to(DEV), dout.to(DEV)
    if case == "channel_last":
        x = x.transpose(1, 2).contiguous().transpose(1, 2)
        dout = dout.transpose(1, 2).contiguous().transpose(1, 2)
    to = (lambda t: None if t is None else t.to(DEV))
    return x, w.to(DEV), b.to(DEV), dout, to(seq), to(init), to(dfs)


def _run(fn, prob):
    x, w, b, dout, seq, init, dfs = prob
    dx = torch.empty_like(x)
    dw = torch.full_like(w, float("nan"))
    db = torch.full_like(b, float("nan"))
    di = torch.full_like(init, float("nan")) if init is not None else None
    fn(x, w, b, dout, seq, init, dx, dw, db, di, True, dfs)
    return dx, dw, db, di


# (case, first problem (B, D, L), second, smaller problem, dtype); the first rows_c5 problem
# is benchmark configuration C5 in fp32, whose workspace (1,310,720 floats at width 4) is the
# largest of the benchmark configurations; the channel-last one is C3 (163,840 floats)
CASES = [
    ("rows", (4, 512, 2048), (2, 96, 700), torch.bfloat16),
    ("rows_c5", (8, 2048, 16384), (2, 96, 700), torch.float32),
    ("channel_last", (1, 4096, 8192), (3, 130, 515), torch.bfloat16),
    ("seq_idx", (2, 256, 4096), (2, 64, 333), torch.float16),
    ("states", (3, 192, 1000), (1, 40, 2), torch.float32),
    ("ragged", (4, 512, 2041), (2, 96, 701), torch.bfloat16),  # odd lengths: ragged row kernels
]


@pytest.mark.gpu
@pytest.mark.parametrize("case,first,second,dtype", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_typed_backward_on_two_calls(case, first, second, dtype):
    probs = [_problem(case, *first, dtype, seed=0), _problem(case, *second, dtype, seed=10)]
    got = [_run(native_bwd_typed_noalloc, p) for p in probs]  # two calls in a row, the second smaller
    want = [_run(native_bwd_typed, p) for p in probs]
    torch.cuda.synchronize()
    for i, (g, e) in enumerate(zip(got, want)):
        for name, a, r in zip(("dx", "dweight", "dbias", "dinitial_states"), g, e):
            if r is None:
                assert a is None
                continue
            assert torch.isfinite(a.float()).all(), f"call {i}: {name} not written"
            assert torch.equal(a, r), f"call {i}: {name} differs from cc1d_bwd_typed"


def test_noalloc_refuses_problems_beyond_the_scratch():
    """Refused from the host before any HIP call (the pointers are never dereferenced)."""
    lib = _lib.load()
    B, D, L = 1, 65536, 1 << 16
    fake = ctypes.c_void_p(1 << 20)
    p = _lib.BwdParams()
    p.x = p.weight = p.dout = p.dx = fake
    p.batch, p.dim, p.seqlen, p.width = B, D, L, 4
    p.x_stride[:] = p.dout_stride[:] = p.dx_stride[:] = (D * L, L, 1)
    p.weight_stride[:] = (4, 1)
    p.dtype, p.apply_silu = 1, 1
    assert lib.cc1d_bwd_workspace_floats(ctypes.byref(p)) > _lib.NOALLOC_WORKSPACE_FLOATS
    g = _lib.BwdGrads()
    g.dweight = fake
    g.dweight_stride[:] = (4, 1)
    assert lib.cc1d_bwd_typed_noalloc(ctypes.byref(p), ctypes.byref(g), None) == ERR_SCRATCH_LIMIT
    assert b"static scratch" in lib.cc1d_strerror(ERR_SCRATCH_LIMIT)


def test_noalloc_validates_like_typed():
    lib = _lib.load()
    assert lib.cc1d_bwd_typed_noalloc(None, None, None) == 1
    p = _lib.BwdParams()
    p.batch, p.dim, p.seqlen, p.width, p.dtype = 1, 8, 16, 10, 1
    g = _lib.BwdGrads()
    assert lib.cc1d_bwd_typed_noalloc(ctypes.byref(p), ctypes.byref(g), None) == 3  # width
    p.width = 4
    assert lib.cc1d_bwd_typed_noalloc(ctypes.byref(p), ctypes.byref(g), None) == 1  # NULL dweight

