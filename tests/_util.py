"""Test helpers: seeded inputs, tolerances, and fp64 closed forms.

The closed forms below are formulations of the op through library routines
(grouped ``F.conv1d`` in float64, torch autograd), independent of the oracle's
loop structure. They pin the oracle; the oracle in turn is the checker for
the HIP kernels on the same seeded inputs.

Tolerances (written here once, used by every parity test):

* elementwise outputs (out, dx, dinitial_states, update out / state):
  ``allclose(rtol=1e-5, atol=1e-5)`` for fp32 and ``allclose(rtol=1e-2,
  atol=1e-2)`` for fp16/bf16 -- the parity bar of the north star.
* reductions over batch and time (dweight, dbias), per element:
  ``|a - e| <= tol * |e| + 64 * u * S`` with u = 2**-24 (the fp32 unit
  roundoff) and ``S`` the sum of the magnitudes of the element's terms,
  ``S[c,k] = sum_{b,t} m[b,c,t] * |xx(b,c,t+k-(W-1))|`` (gated as the op
  gates) and ``S[c] = sum_{b,t} m[b,c,t]``, with m the magnitude of dpre
  before cancellation (``dpre_f64(magnitude=True)``), computed in float64
  (``reduction_scale``). The first term is the dtype's parity bar on the
  result itself; the second bounds the difference between two fp32
  summation orders of the same terms (a sequential fp32 sum of random-sign
  terms drifts by about u * S / 4, and every test draws N(0,1) data) plus
  the last-ulp differences of the terms. Each channel and tap is held to
  its own magnitude, so a dropped or mis-gated tap on a low-magnitude
  channel fails even when other channels are large.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

TOL = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}
DTYPES = [torch.float16, torch.bfloat16, torch.float32]
DTYPE_IDS = ["fp16", "bf16", "fp32"]


def randn(*shape, dtype=torch.float32, device="cpu", generator=None):
    return torch.randn(*shape, generator=generator, dtype=torch.float32).to(device=device, dtype=dtype)


def make_inputs(batch, dim, seqlen, width, *, dtype, device="cpu", has_bias=True, seed=0, has_init=False):
    """N(0,1) draws in fp32 from one CPU generator (x, weight, bias, initial_states order), cast to dtype."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = randn(batch, dim, seqlen, dtype=dtype, device=device, generator=g)
    w = randn(dim, width, dtype=dtype, device=device, generator=g)
    b = randn(dim, dtype=dtype, device=device, generator=g) if has_bias else None
    init = randn(batch, dim, width - 1, dtype=dtype, device=device, generator=g) if has_init else None
    return x, w, b, init


def _cmp_device(a, b):
    """Compare where the data already is (GPU when either side is there)."""
    for t in (a, b):
        if t.device.type != "cpu":
            return t.device
    return torch.device("cpu")


def assert_close(actual, expected, dtype=None, *, name="", rtol=None, atol=None):
    dtype = dtype or actual.dtype
    tol = TOL[dtype]
    rtol = tol if rtol is None else rtol
    atol = tol if atol is None else atol
    dev = _cmp_device(actual, expected)
    a = actual.detach().to(dev, torch.float64)
    e = expected.detach().to(dev, torch.float64)
    assert a.shape == e.shape, f"{name}: shape {tuple(a.shape)} vs {tuple(e.shape)}"
    assert torch.isfinite(a).all(), f"{name}: non-finite values"
    if not torch.allclose(a, e, rtol=rtol, atol=atol):
        diff = (a - e).abs()
        idx = int(diff.argmax())
        raise AssertionError(
            f"{name}: max |diff| {diff.max().item():.3e} at flat index {idx} "
            f"(actual {a.flatten()[idx].item():.6g}, expected {e.flatten()[idx].item():.6g}, rtol={rtol}, atol={atol})"
        )


FP32_UNIT_ROUNDOFF = 2.0 ** -24
SUM_ORDER_ULPS = 64


def reduction_bound(expected, scale, dtype):
    """Per-element bound for dweight / dbias (see the module docstring)."""
    dev = expected.device
    e = expected.detach().to(dev, torch.float64)
    s = scale.detach().to(dev, torch.float64)
    return TOL[dtype] * e.abs() + SUM_ORDER_ULPS * FP32_UNIT_ROUNDOFF * s


def assert_reduction_close(actual, expected, dtype, *, scale, name=""):
    """dweight / dbias parity: every (channel, tap) within tol * |e| + 64 u S of the
    expected value, S being that element's magnitude sum (``reduction_scale``)."""
    dev = _cmp_device(actual, expected)
    a = actual.detach().to(dev, torch.float64)
    e = expected.detach().to(dev, torch.float64)
    assert a.shape == e.shape, f"{name}: shape {tuple(a.shape)} vs {tuple(e.shape)}"
    assert scale.shape == e.shape, f"{name}: scale shape {tuple(scale.shape)} vs {tuple(e.shape)}"
    assert torch.isfinite(a).all(), f"{name}: non-finite values"
    if a.numel() == 0:
        return
    bound = reduction_bound(e, scale.to(dev), dtype)
    excess = (a - e).abs() - bound
    if (excess > 0).any():
        idx = int(excess.argmax())
        raise AssertionError(
            f"{name}: |diff| {abs(a.flatten()[idx] - e.flatten()[idx]).item():.3e} > bound "
            f"{bound.flatten()[idx].item():.3e} at flat index {idx} (actual {a.flatten()[idx].item():.6g}, "
            f"expected {e.flatten()[idx].item():.6g}, magnitude sum {scale.flatten()[idx].item():.4g}); "
            f"{int((excess > 0).sum())} elements out of bound"
        )


def assert_equal(actual, expected, *, name=""):
    a = actual.detach().cpu()
    e = expected.detach().cpu()
    assert a.shape == e.shape and a.dtype == e.dtype, f"{name}: {a.shape}/{a.dtype} vs {e.shape}/{e.dtype}"
    if not torch.equal(a, e):
        diff = (a.double() - e.double()).abs()
        raise AssertionError(f"{name}: not bit-identical (max |diff| {diff.max().item():.3e}, {int((diff > 0).sum())} elements)")


# ---------------------------------------------------------------------------
# fp64 closed forms
# ---------------------------------------------------------------------------


def conv_f64(x, w, b=None, init=None, silu=False):
    """Grouped causal conv in float64 via F.conv1d (initial_states prepended when given)."""
    x = x.double()
    w = w.double()
    D, W = w.shape
    L = x.shape[-1]
    xp = torch.cat([init.double(), x], -1) if init is not None else F.pad(x, (W - 1, 0))
    out = F.conv1d(xp, w.unsqueeze(1), None if b is None else b.double(), groups=D)[..., :L]
    return F.silu(out) if silu else out


def conv_seq_f64(x, w, b, seq_idx, silu=False):
    """Packed-sequence forward in float64: for every id value v, a grouped
    conv over x with the positions of other ids zeroed, read back at the
    positions whose id is v; positions with id < 0 are 0. This is the
    id-equality gate of the reference, expressed with F.conv1d."""
    x = x.double()
    out = torch.zeros_like(x)
    for bi in range(x.shape[0]):
        ids = seq_idx[bi].cpu()
        for v in torch.unique(ids).tolist():
            if v < 0:
                continue
            mask = (ids == v).to(x.device, torch.float64)
            o = conv_f64(x[bi : bi + 1] * mask, w, b, silu=silu)
            out[bi] = torch.where(mask.bool(), o[0], out[bi])
    return out


def grads_f64(x, w, b, dout, init=None, seq_idx=None, silu=False):
    """(dx, dweight, dbias, dinit) by float64 autograd through the closed forms."""
    xg = x.detach().double().requires_grad_()
    wg = w.detach().double().requires_grad_()
    bg = b.detach().double().requires_grad_() if b is not None else None
    ig = init.detach().double().requires_grad_() if init is not None else None
    if seq_idx is not None:
        out = conv_seq_f64(xg, wg, bg, seq_idx, silu)
    else:
        out = conv_f64(xg, wg, bg, ig, silu)
    out.backward(dout.double())
    return (xg.grad, wg.grad, None if bg is None else bg.grad, None if ig is None else ig.grad)


def taps_f64(x, w, b, seq_idx=None, init=None):
    """Forward pieces in float64 from shifted products, on x's device:
    (pre, x padded on the left with initial_states or zeros, tap masks).
    masks[k][b, 0, t] says whether tap k of position t is kept: its source
    position t+k-(W-1) is >= 0 and has the same seq_idx as t (no masks
    without seq_idx)."""
    xd = x.double()
    wd = w.double()
    B, D, L = x.shape
    W = w.shape[1]
    H = W - 1
    xp = torch.cat([init.double(), xd], -1) if init is not None else F.pad(xd, (H, 0))
    masks = None
    if seq_idx is not None:
        sp = F.pad(seq_idx.long(), (H, 0), value=-(2 ** 40))  # positions before 0 never match
        masks = [(sp[:, k:k + L] == seq_idx.long()).unsqueeze(1) for k in range(W)]
    pre = torch.zeros(B, D, L, dtype=torch.float64, device=x.device)
    if b is not None:
        pre += b.double()[None, :, None]
    for k in range(W):
        term = wd[None, :, k, None] * xp[..., k:k + L]
        pre += term if masks is None else term * masks[k]
    return pre, xp, masks


def dpre_f64(x, w, b, dout, seq_idx=None, init=None, silu=False, magnitude=False):
    """Gradient at the pre-activation in float64, zero where seq_idx < 0; with
    the padded x and the tap masks of ``taps_f64``.

    magnitude=True returns instead the scale of the fp32 rounding error of
    dpre: |dout| * (s * (1 + |p| (1 - s)) + |b| + sum_k |w_k xx_k|) with SiLU
    (the size of silu'(p)'s factors before they cancel near its root
    p = -1.28, plus the size of p's own terms, since |silu''| <= 1/2), |dout|
    without."""
    pre, xp, masks = taps_f64(x, w, b, seq_idx, init)
    dpre = dout.double()
    if magnitude:
        dpre = dpre.abs()
    if silu:
        s = torch.sigmoid(pre)
        if magnitude:
            B, D, L = x.shape
            W = w.shape[1]
            pmag = torch.zeros_like(pre) if b is None else b.double().abs()[None, :, None].expand_as(pre).clone()
            for k in range(W):
                term = (w.double()[None, :, k, None] * xp[..., k:k + L]).abs()
                pmag += term if masks is None else term * masks[k]
            dpre = dpre * (s * (1 + pre.abs() * (1 - s)) + pmag)
        else:
            dpre = dpre * s * (1 + pre * (1 - s))
    if seq_idx is not None:
        dpre = dpre * (seq_idx >= 0).unsqueeze(1)
    return dpre, xp, masks


def weight_grads_from_dpre(dpre, xp, masks, absolute=False):
    """(dweight, dbias) sums over batch and time of dpre * xx(t+k-(W-1)) and
    dpre; with absolute=True the sums of their magnitudes (the scale of
    ``assert_reduction_close``)."""
    L = dpre.shape[-1]
    W = xp.shape[-1] - L + 1
    d = dpre.abs() if absolute else dpre
    xs = xp.abs() if absolute else xp
    dw = torch.stack([(d * xs[..., k:k + L] * (1 if masks is None else masks[k])).sum((0, 2)) for k in range(W)], 1)
    return dw, d.sum((0, 2))


def reduction_scale(x, w, b, dout, init=None, seq_idx=None, silu=False):
    """Per-element magnitude sums (S_dweight (dim, W), S_dbias (dim,)) in float64, on x's
    device: the sums of ``dpre_f64(magnitude=True) * |xx|`` over the terms of each element."""
    dmag, xp, masks = dpre_f64(x, w, b, dout, seq_idx, init, silu, magnitude=True)
    return weight_grads_from_dpre(dmag, xp, masks, absolute=True)


def scales(x, w, b, dout, *, init=None, seq_idx=None, activation=None):
    """``reduction_scale`` of test inputs, on the CPU: (S_dweight, S_dbias)."""
    cpu = (lambda t: None if t is None else t.detach().cpu())
    return reduction_scale(cpu(x), cpu(w), cpu(b), cpu(dout), init=cpu(init), seq_idx=cpu(seq_idx),
                           silu=activation in ("silu", "swish"))


def final_states_expected(x, width):
    """Last width-1 columns of x, zero padded on the left (reference _fn.py:31-50)."""
    L = x.shape[-1]
    pad = max(0, (width - 1) - L)
    tail = x[..., max(0, L - (width - 1)):]
    return F.pad(tail, (pad, 0))


def seq_pattern(name, batch, seqlen, device="cpu"):
    """seq_idx patterns of the reference's tests (test_fwd.py:316-359) plus two more."""
    if name == "single":
        s = torch.zeros(batch, seqlen, dtype=torch.int32)
    elif name == "two_equal":
        s = torch.cat([torch.zeros(batch, seqlen // 2), torch.ones(batch, seqlen - seqlen // 2)], 1)
    elif name == "varied":
        s = torch.cat([torch.zeros(batch, 10), torch.ones(batch, 25), torch.full((batch, seqlen - 35), 2)], 1)
    elif name == "with_padding":
        s = torch.cat([torch.zeros(batch, 16), torch.full((batch, 16), -1), torch.ones(batch, seqlen - 32)], 1)
    elif name == "repeat_ids":
        # an id reappears within one window: equality gating differs from run splitting here
        base = torch.tensor([0, 0, 0, 1, 0, 0, 2, 2, -1, 2, 3, 3, 3, 1, 1, 1], dtype=torch.int32)
        s = base.repeat((seqlen + 15) // 16)[:seqlen].expand(batch, seqlen)
    elif name == "random_runs":
        g = torch.Generator().manual_seed(7)
        cuts = torch.sort(torch.randperm(seqlen - 1, generator=g)[:7] + 1).values
        s = torch.zeros(seqlen)
        for i, cpos in enumerate(cuts.tolist()):
            s[cpos:] = i + 1
        s = s.expand(batch, seqlen)
    else:
        raise ValueError(name)
    return s.to(torch.int32).contiguous().to(device)


SEQ_PATTERNS = ["single", "two_equal", "varied", "with_padding", "repeat_ids", "random_runs"]
