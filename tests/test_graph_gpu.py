"""HIP graph capture of the ops (reference tests/test_cuda_graph.py:138-190).

The entry points allocate nothing, synchronise nothing and issue no
memsets, so forward, backward (with its accumulator zero-fill done by a
kernel) and update can be captured. Each graph is replayed several times
with eager work and synchronisations in between, and every replay is
compared with an eager run on the same inputs.
"""

from __future__ import annotations

import pytest
import torch

import causal_conv1d_amd as cc
from _util import assert_reduction_close, make_inputs, scales

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm up outside the graph
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def test_forward_capture_replay_matches_eager():
    x, w, b, _ = make_inputs(2, 64, 2048, 4, dtype=torch.bfloat16, device=DEV)
    out_buf = torch.empty_like(x)
    g = _capture(lambda: out_buf.copy_(cc.causal_conv1d_fn(x, w, b, activation="silu")))
    for i in range(4):
        x.copy_(torch.randn_like(x))  # in-place input mutation between replays
        g.replay()
        torch.cuda.synchronize()
        eager = cc.causal_conv1d_fn(x, w, b, activation="silu")
        _ = (eager.float() * 2).sum().item()  # unrelated eager work + sync between replays
        assert torch.equal(out_buf, eager), f"replay {i}"


def test_backward_ops_capture_replay_matches_eager():
    B, D, L, W = 4, 256, 2048, 4
    x, w, b, _ = make_inputs(B, D, L, W, dtype=torch.bfloat16, device=DEV)
    dout = torch.randn_like(x)
    dx = torch.empty_like(x)
    dw = torch.empty(D, W, dtype=torch.float32, device=DEV)
    db = torch.empty(D, dtype=torch.float32, device=DEV)
    out = torch.empty_like(x)

    def step():
        torch.ops.causal_conv1d_amd._fwd_inplace(x, w, b, None, None, out, True, None)
        dw.zero_()
        db.zero_()
        torch.ops.causal_conv1d_amd._bwd_full_inplace(x, w, b, dout, None, None, dx, dw, db, None, True)

    g = _capture(step)
    for i in range(4):
        dout.copy_(torch.randn_like(dout))
        sw, sb = scales(x, w, b, dout, activation="silu")
        g.replay()
        torch.cuda.synchronize()
        snap = [t.clone() for t in (out, dx, dw, db)]
        step()
        torch.cuda.synchronize()
        for name, a, e in zip(("out", "dx"), snap[:2], (out, dx)):
            assert torch.equal(a, e), f"replay {i}: {name}"
        # dweight / dbias gather B fp32 atomic adds per entry in any order: equal up
        # to fp32 rounding (a missing zero-fill on replay would double them)
        for name, a, e, sc in zip(("dweight", "dbias"), snap[2:], (dw, db), (sw, sb)):
            assert_reduction_close(a, e, torch.float32, scale=sc, name=f"replay {i}: {name}")


def test_update_capture_replay_matches_eager():
    B, D, W = 64, 512, 4
    x, w, b, _ = make_inputs(B, D, 1, W, dtype=torch.bfloat16, device=DEV)
    x = x[..., 0].contiguous()
    pool = torch.randn(2 * B, D, W - 1, dtype=torch.bfloat16, device=DEV)
    idx = torch.randperm(2 * B, device=DEV)[:B].to(torch.int32)
    out_buf = torch.empty_like(x)
    state = pool.clone()
    g = _capture(lambda: out_buf.copy_(cc.causal_conv1d_update(x, state, w, b, activation="silu",
                                                               conv_state_indices=idx)))
    for i in range(4):
        state.copy_(pool)
        x.copy_(torch.randn_like(x))
        g.replay()
        torch.cuda.synchronize()
        got_out, got_state = out_buf.clone(), state.clone()
        state.copy_(pool)
        eager = cc.causal_conv1d_update(x, state, w, b, activation="silu", conv_state_indices=idx)
        torch.cuda.synchronize()
        assert torch.equal(got_out, eager), f"replay {i}: out"
        assert torch.equal(got_state, state), f"replay {i}: state"


def test_autograd_backward_capture_replay_is_bit_identical():
    """The autograd step (forward + typed backward, no fill kernels) in a graph: every replay
    equals the eager step bit for bit, weight/bias gradients included."""
    B, D, L, W = 4, 256, 2048, 4
    x, w, b, _ = make_inputs(B, D, L, W, dtype=torch.bfloat16, device=DEV)
    x.requires_grad_()
    w.requires_grad_()
    b.requires_grad_()
    dout = torch.randn(B, D, L, dtype=torch.bfloat16, device=DEV)
    grads = [None, None, None]

    def step():
        out = cc.causal_conv1d_fn(x, w, b, activation="silu")
        g = torch.autograd.grad(out, (x, w, b), dout)
        for i in range(3):
            if grads[i] is None:
                grads[i] = torch.empty_like(g[i])
            grads[i].copy_(g[i])

    g = _capture(step)
    for i in range(4):
        dout.copy_(torch.randn_like(dout))
        sw, sb = scales(x, w, b, dout, activation="silu")
        g.replay()
        torch.cuda.synchronize()
        snap = [t.clone() for t in grads]
        step()
        torch.cuda.synchronize()
        for name, a, e in zip(("dx", "dweight", "dbias"), snap, grads):
            assert torch.equal(a, e), f"replay {i}: {name}"
