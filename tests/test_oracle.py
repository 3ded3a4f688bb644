"""Pins the CPU oracle (oracle/cc1d_oracle.c) before it is trusted as the checker.

Each oracle function is checked against
  * the committed golden fixtures (tests/golden/, float64 library results),
  * float64 closed forms on fresh seeded inputs (grouped F.conv1d, autograd),
  * invariants (decode loop == full forward, chunked == full),
  * torch's own fp16/bf16 rounding for the scalar conversions,
and a few checks plant a mistake in the oracle's output to show that the
comparison used would catch it. No GPU needed.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from _util import (
    DTYPE_IDS,
    DTYPES,
    SEQ_PATTERNS,
    assert_close,
    assert_equal,
    assert_reduction_close,
    conv_f64,
    conv_seq_f64,
    final_states_expected,
    grads_f64,
    make_inputs,
    reduction_bound,
    reduction_scale,
    scales,
    seq_pattern,
)
from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: torch.from_numpy(z[k]) for k in z.files}


# ---------------------------------------------------------------- conversions


def test_bf16_f16_widening_matches_torch_for_every_bit_pattern():
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16)
    for dt, fn in ((torch.bfloat16, O.bf16_bits_to_f32), (torch.float16, O.f16_bits_to_f32)):
        want = bits.view(dt).float()
        got = torch.tensor([fn(int(v) & 0xFFFF) for v in bits.tolist()], dtype=torch.float32)
        nan = torch.isnan(want)
        assert torch.equal(torch.isnan(got), nan)
        assert torch.equal(got[~nan], want[~nan])


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_rounding_matches_torch_rne(dt):
    g = torch.Generator().manual_seed(5)
    vals = torch.cat([
        torch.randn(20000, generator=g) * 10.0 ** torch.randint(-8, 6, (20000,), generator=g).float(),
        torch.tensor([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, 65536.0, 1e-8, 5.96e-8, 2.98e-8,
                      6.1e-5, 3.0e38, -3.0e38, float("inf"), float("-inf")]),
    ])
    # exact ties between two representable values (round half to even)
    one = torch.ones(64)
    step = 2.0 ** -8 if dt == torch.bfloat16 else 2.0 ** -11
    ties = one + step * torch.arange(64)
    vals = torch.cat([vals, ties, -ties])
    want = vals.to(dt).view(torch.int16).to(torch.int32) & 0xFFFF
    fn = O.f32_to_bf16_bits if dt == torch.bfloat16 else O.f32_to_f16_bits
    got = torch.tensor([fn(float(v)) for v in vals.tolist()], dtype=torch.int32)
    bad = (got != want).nonzero().flatten()
    assert bad.numel() == 0, f"{bad.numel()} mismatches, first value {vals[bad[0]].item()!r}"


# ---------------------------------------------------------------- forward


def test_golden_c1_forward():
    z = _load("c1_fwd_fp32.npz")
    out = O.causal_conv1d_fn(z["x"], z["weight"], z["bias"], activation="silu")
    assert_close(out, z["out"], torch.float32, name="c1 out")


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4, 5, 9])
@pytest.mark.parametrize("silu", [False, True])
def test_forward_matches_conv1d_f64(dtype, width, silu):
    x, w, b, _ = make_inputs(2, 16, 67, width, dtype=dtype)
    out = O.causal_conv1d_fn(x, w, b, activation="silu" if silu else None)
    assert out.dtype == dtype
    assert_close(out, conv_f64(x, w, b, silu=silu), dtype, name="out")


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
def test_forward_strided_inputs(dtype):
    # channel-last x, transposed weight, sliced bias: strides only change addressing
    x = torch.randn(2, 40, 24).to(dtype).transpose(1, 2)  # (2, 24, 40), stride (960, 1, 24)
    w = torch.randn(4, 24).to(dtype).t()
    b = torch.randn(48).to(dtype)[::2]
    out = O.causal_conv1d_fn(x, w, b, activation="silu")
    assert_close(out, conv_f64(x, w, b, silu=True), dtype)


def test_forward_planted_tap_reversal_is_caught():
    x, w, b, _ = make_inputs(1, 8, 32, 4, dtype=torch.float32)
    out = O.causal_conv1d_fn(x, w.flip(1).contiguous(), b)  # plant: taps in reverse order
    with pytest.raises(AssertionError):
        assert_close(out, conv_f64(x, w, b), torch.float32)


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 4, 5])
def test_initial_states_matches_concat_form(dtype, width):
    x, w, b, init = make_inputs(2, 8, 40, width, dtype=dtype, has_init=True)
    out = O.causal_conv1d_fn(x, w, b, initial_states=init, activation="silu")
    assert_close(out, conv_f64(x, w, b, init, silu=True), dtype)


@pytest.mark.parametrize("seqlen", [1, 2, 3, 4, 16])
def test_final_states_exact(seqlen):
    x, w, b, init = make_inputs(2, 8, seqlen, 4, dtype=torch.bfloat16, has_init=True)
    # final states ignore initial_states and zero-pad on the left (_fn.py:31-50)
    _, fs = O.causal_conv1d_fn(x, w, b, initial_states=init, return_final_states=True)
    assert_equal(fs, final_states_expected(x, 4).to(torch.bfloat16))


def test_chunked_forward_equals_full():
    x, w, b, _ = make_inputs(1, 8, 96, 4, dtype=torch.float32)
    full = O.causal_conv1d_fn(x, w, b, activation="silu")
    init, outs = None, []
    for c in (x[..., :32], x[..., 32:64], x[..., 64:]):
        o, init = O.causal_conv1d_fn(c, w, b, initial_states=init, return_final_states=True, activation="silu")
        outs.append(o)
    assert_close(torch.cat(outs, -1), full, torch.float32)


@pytest.mark.parametrize("pattern", SEQ_PATTERNS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_seq_idx_matches_id_class_conv(pattern, dtype):
    x, w, b, _ = make_inputs(2, 8, 64, 4, dtype=dtype)
    s = seq_pattern(pattern, 2, 64)
    out = O.causal_conv1d_fn(x, w, b, seq_idx=s, activation="silu")
    assert_close(out, conv_seq_f64(x, w, b, s, silu=True), dtype, name=pattern)


def test_seq_idx_equality_gate_differs_from_run_split():
    """The reference gates taps on id equality; splitting at id changes would
    drop the tap that reaches back to an earlier run with the same id."""
    z = _load("seq_repeat_fp32.npz")
    x, w, b, s = z["x"], z["weight"], z["bias"], z["seq_idx"]
    out = O.causal_conv1d_fn(x, w, b, seq_idx=s, activation="silu")
    assert_close(out, z["out"], torch.float32, name="golden seq out")
    # plant: a run-split seq_idx (relabel every run) must not match the golden output
    relabel = torch.cumsum((s[:, 1:] != s[:, :-1]).int(), 1)
    runs = torch.cat([torch.zeros_like(s[:, :1]), relabel], 1).to(torch.int32)
    runs = torch.where(s < 0, torch.full_like(runs, -1), runs).contiguous()
    planted = O.causal_conv1d_fn(x, w, b, seq_idx=runs, activation="silu")
    with pytest.raises(AssertionError):
        assert_close(planted, z["out"], torch.float32)


# ---------------------------------------------------------------- backward


def test_golden_backward_with_initial_and_final_states():
    z = _load("bwd_init_fp32.npz")
    dx, dw, db, dinit = O.causal_conv1d_bwd(
        z["x"], z["weight"], z["bias"], z["dout"], initial_states=z["initial_states"],
        dfinal_states=z["dfinal_states"], activation="silu",
    )
    sw, sb = scales(z["x"], z["weight"], z["bias"], z["dout"], init=z["initial_states"], activation="silu")
    assert_close(dx, z["dx"], torch.float32, name="dx")
    assert_reduction_close(dw, z["dweight"], torch.float32, scale=sw, name="dweight")
    assert_reduction_close(db, z["dbias"], torch.float32, scale=sb, name="dbias")
    assert_close(dinit, z["dinitial_states"], torch.float32, name="dinit")


def test_golden_backward_seq_idx():
    z = _load("seq_repeat_fp32.npz")
    dx, dw, db, _ = O.causal_conv1d_bwd(z["x"], z["weight"], z["bias"], z["dout"], seq_idx=z["seq_idx"],
                                        activation="silu")
    sw, sb = scales(z["x"], z["weight"], z["bias"], z["dout"], seq_idx=z["seq_idx"], activation="silu")
    assert_close(dx, z["dx"], torch.float32, name="dx")
    assert_reduction_close(dw, z["dweight"], torch.float32, scale=sw, name="dweight")
    assert_reduction_close(db, z["dbias"], torch.float32, scale=sb, name="dbias")


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4, 5])
@pytest.mark.parametrize("silu", [False, True])
@pytest.mark.parametrize("has_init", [False, True])
def test_backward_matches_autograd_f64(dtype, width, silu, has_init):
    x, w, b, init = make_inputs(2, 8, 37, width, dtype=dtype, has_init=has_init)
    dout = torch.randn(x.shape).to(dtype)
    dx, dw, db, dinit = O.causal_conv1d_bwd(x, w, b, dout, initial_states=init,
                                            activation="silu" if silu else None)
    rdx, rdw, rdb, rdinit = grads_f64(x, w, b, dout, init=init, silu=silu)
    sw, sb = reduction_scale(x, w, b, dout, init=init, silu=silu)
    assert_close(dx, rdx, dtype, name="dx")
    assert_reduction_close(dw, rdw, dtype, scale=sw, name="dweight")
    assert_reduction_close(db, rdb, dtype, scale=sb, name="dbias")
    if has_init:
        assert_close(dinit, rdinit, dtype, name="dinit")


@pytest.mark.parametrize("pattern", SEQ_PATTERNS)
def test_backward_seq_idx_matches_autograd_f64(pattern):
    x, w, b, _ = make_inputs(2, 8, 64, 4, dtype=torch.float32)
    dout = torch.randn(x.shape)
    s = seq_pattern(pattern, 2, 64)
    dx, dw, db, _ = O.causal_conv1d_bwd(x, w, b, dout, seq_idx=s, activation="silu")
    rdx, rdw, rdb, _ = grads_f64(x, w, b, dout, seq_idx=s, silu=True)
    sw, sb = reduction_scale(x, w, b, dout, seq_idx=s, silu=True)
    assert_close(dx, rdx, torch.float32, name="dx")
    assert_reduction_close(dw, rdw, torch.float32, scale=sw, name="dweight")
    assert_reduction_close(db, rdb, torch.float32, scale=sb, name="dbias")


def test_backward_planted_missing_silu_grad_is_caught():
    x, w, b, _ = make_inputs(1, 8, 32, 4, dtype=torch.float32)
    dout = torch.randn(x.shape)
    dx, _, _, _ = O.causal_conv1d_bwd(x, w, b, dout, activation=None)  # plant: silu' dropped
    rdx, _, _, _ = grads_f64(x, w, b, dout, silu=True)
    with pytest.raises(AssertionError):
        assert_close(dx, rdx, torch.float32)


def _scale_brute_force(x, w, b, dout, init=None, seq_idx=None, silu=False):
    """Magnitude sums by explicit loops in float64 (tiny shapes only): per term
    |dout| * (s (1 + |p| (1 - s)) + |b| + sum_k |w_k xx_k|) * |xx| with SiLU."""
    B, D, L = x.shape
    W = w.shape[1]
    xd, wd, gd = x.double(), w.double(), dout.double()
    sw = torch.zeros(D, W, dtype=torch.float64)
    sb = torch.zeros(D, dtype=torch.float64)

    def xx(bi, c, s):
        if s >= 0:
            return xd[bi, c, s].item()
        return init.double()[bi, c, s + W - 1].item() if init is not None else 0.0

    def keep(bi, s, t):
        return seq_idx is None or (s >= 0 and int(seq_idx[bi, s]) == int(seq_idx[bi, t]))

    for bi in range(B):
        for c in range(D):
            for t in range(L):
                if seq_idx is not None and int(seq_idx[bi, t]) < 0:
                    continue
                kept = [k for k in range(W) if keep(bi, t + k - (W - 1), t)]
                bias = b.double()[c].item() if b is not None else 0.0
                pre = bias + sum(wd[c, k].item() * xx(bi, c, t + k - (W - 1)) for k in kept)
                d = abs(gd[bi, c, t].item())
                if silu:
                    sg = 1.0 / (1.0 + np.exp(-pre))
                    pmag = abs(bias) + sum(abs(wd[c, k].item() * xx(bi, c, t + k - (W - 1))) for k in kept)
                    d *= sg * (1 + abs(pre) * (1 - sg)) + pmag
                sb[c] += d
                for k in kept:
                    sw[c, k] += d * abs(xx(bi, c, t + k - (W - 1)))
    return sw, sb


@pytest.mark.parametrize("case", ["plain", "init", "seq"])
def test_reduction_scale_matches_brute_force(case):
    """The per-element bound's magnitude sums, pinned by explicit loops."""
    x, w, b, init = make_inputs(2, 3, 11, 4, dtype=torch.float32, has_init=case == "init")
    dout = make_inputs(2, 3, 11, 4, dtype=torch.float32, seed=1)[0]
    s = torch.tensor([[0, 0, 1, 1, 1, -1, 2, 2, 1, 1, 1]] * 2, dtype=torch.int32) if case == "seq" else None
    sw, sb = reduction_scale(x, w, b, dout, init=init, seq_idx=s, silu=True)
    bw, bb = _scale_brute_force(x, w, b, dout, init=init, seq_idx=s, silu=True)
    assert torch.allclose(sw, bw, rtol=1e-12, atol=0) and torch.allclose(sb, bb, rtol=1e-12, atol=0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("plant", ["dropped_tap", "misgated_tap"])
def test_reduction_bound_catches_error_on_low_magnitude_channel(dtype, plant):
    """A mistake on one low-magnitude channel fails the per-(channel, tap) bound, while the
    tensor-wide bound tol * (1 + max|ref|) of the reference's helper would accept it."""
    B, D, L, W = 2, 16, 256, 4
    x, w, b, _ = make_inputs(B, D, L, W, dtype=dtype)
    dout = make_inputs(B, D, L, W, dtype=dtype, seed=1)[0]
    # channel 5: gradients 1e3 (bf16) / 1e6 (fp32) times smaller than the rest
    dout[:, 5] = (dout[:, 5].float() * (1e-3 if dtype == torch.bfloat16 else 1e-6)).to(dtype)
    s = seq_pattern("random_runs", B, L) if plant == "misgated_tap" else None
    _, dw, db, _ = O.causal_conv1d_bwd(x, w, b, dout, seq_idx=s, activation="silu")
    sw, sb = reduction_scale(x, w, b, dout, seq_idx=s, silu=True)
    _, rdw, _, _ = grads_f64(x, w, b, dout, seq_idx=s, silu=True)
    assert_reduction_close(dw, rdw, dtype, scale=sw)  # the unplanted oracle passes
    planted = dw.double().clone()
    if plant == "dropped_tap":
        # tap 0 of channel 5 loses its contribution from batch 1
        drop = grads_f64(x[1:], w, b, dout[1:], silu=True)[1][5, 0]
        planted[5, 0] -= drop
    else:
        # tap 0 of channel 5 ignores the seq_idx gate at the 7 boundaries of batch 0
        _, ungated, _, _ = grads_f64(x[:1], w, b, dout[:1], silu=True)
        _, gated, _, _ = grads_f64(x[:1], w, b, dout[:1], seq_idx=s[:1], silu=True)
        planted[5, 0] += ungated[5, 0] - gated[5, 0]
    assert (planted - rdw).abs().max() <= TOL_WIDE[dtype] * (1 + rdw.abs().max())  # the old bound misses it
    assert ((planted - rdw).abs() > reduction_bound(rdw, sw, dtype)).any()
    with pytest.raises(AssertionError):
        assert_reduction_close(planted, rdw, dtype, scale=sw)


TOL_WIDE = {torch.float32: 1e-5, torch.bfloat16: 1e-2}


# ---------------------------------------------------------------- update


def _bursts(z):
    b = [int(v) for v in z["bursts"].tolist()]
    starts = np.cumsum([0] + b[:-1]).tolist()
    return list(zip(starts, b))


def test_golden_update_linear_bursts():
    z = _load("update_fp32.npz")
    state = z["state_linear"].clone()
    outs = []
    for s0, n in _bursts(z):
        outs.append(O.causal_conv1d_update(z["x"][..., s0:s0 + n].contiguous(), state, z["weight"], z["bias"],
                                           activation="silu"))
    assert_close(torch.cat(outs, -1), z["out_linear"], torch.float32, name="out")
    assert_equal(state, z["final_linear"], name="state")


def test_golden_update_circular_bursts():
    z = _load("update_fp32.npz")
    state = z["state_circular"].clone()
    cs = z["cache_seqlens"].clone()
    outs = []
    for s0, n in _bursts(z):
        outs.append(O.causal_conv1d_update(z["x"][..., s0:s0 + n].contiguous(), state, z["weight"], z["bias"],
                                           activation="silu", cache_seqlens=cs))
        cs = cs + n
    assert_close(torch.cat(outs, -1), z["out_circular"], torch.float32, name="out")
    assert_equal(state, z["final_circular"], name="state")


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4, 9])
def test_decode_loop_matches_full_forward(dtype, width):
    x, w, b, _ = make_inputs(2, 8, 20, width, dtype=dtype)
    full = O.causal_conv1d_fn(x, w, b, activation="silu")
    state = torch.zeros(2, 8, width - 1, dtype=dtype)
    dec = torch.cat([O.causal_conv1d_update(x[..., t], state, w, b, activation="silu").unsqueeze(-1)
                     for t in range(20)], -1)
    # same fp32 ops in the same order on both paths: bit-identical
    assert_equal(dec, full)


def test_update_pool_indices_and_padding():
    x, w, b, _ = make_inputs(3, 8, 2, 4, dtype=torch.float32)
    pool = torch.randn(5, 8, 3)
    idx = torch.tensor([3, -1, 0], dtype=torch.int32)
    p = pool.clone()
    out = O.causal_conv1d_update(x, p, w, b, activation="silu", conv_state_indices=idx)
    assert torch.all(out[1] == 0)
    for bi, r in ((0, 3), (2, 0)):
        st = pool[r:r + 1].clone()
        ref = O.causal_conv1d_update(x[bi:bi + 1], st, w, b, activation="silu")
        assert_equal(out[bi:bi + 1], ref)
        assert_equal(p[r:r + 1], st)
    for r in (1, 2, 4):
        assert_equal(p[r], pool[r])


# ---------------------------------------------------------------- varlen


def test_varlen_states_known_answers():
    """Known answers of the reference's tests/test_varlen.py:25-64."""
    x = torch.arange(11 * 2, dtype=torch.float32).reshape(11, 2)
    out = O.varlen_states(x, torch.tensor([0, 5, 7, 11], dtype=torch.int32), 3)
    assert out.shape == (3, 2, 3)
    assert torch.equal(out[0], x[2:5].T)
    assert torch.equal(out[1, :, 0], torch.zeros(2)) and torch.equal(out[1, :, 1:], x[5:7].T)
    assert torch.equal(out[2], x[8:11].T)
    x = torch.arange(5 * 4, dtype=torch.float32).reshape(5, 4)
    out = O.varlen_states(x, torch.tensor([0, 3, 3, 5], dtype=torch.int32), 2)
    assert torch.equal(out[1], torch.zeros(4, 2))
    x = torch.arange(4 * 3, dtype=torch.float16).reshape(4, 3)
    out = O.varlen_states(x, torch.tensor([0, 2, 4], dtype=torch.int32), 8)
    assert torch.equal(out[0, :, :6], torch.zeros(3, 6, dtype=torch.float16))
    assert torch.equal(out[0, :, 6:], x[0:2].T) and torch.equal(out[1, :, 6:], x[2:4].T)
