"""Test helpers: seeded inputs, tolerances, and fp64 closed forms.

The closed forms below are formulations of the op through library routines
(grouped ``F.conv1d`` in float64, torch autograd), independent of the oracle's
loop structure. They pin the oracle; the oracle in turn is the checker for
the HIP kernels on the same seeded inputs.

Tolerances (written here once, used by every parity test):

* elementwise outputs (out, dx, dinitial_states, update out / state):
  ``allclose(rtol=1e-5, atol=1e-5)`` for fp32 and ``allclose(rtol=1e-2,
  atol=1e-2)`` for fp16/bf16 -- the parity bar of the north star.
* reductions over batch and time (dweight, dbias): the same rtol applied to
  the largest magnitude of the reference, ``|a - b| <= tol * (1 + max|ref|)``,
  because two valid fp32 summation orders of B*L terms differ by a few ulp
  of the running sum, not of each (possibly tiny) result.
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


def assert_reduction_close(actual, expected, dtype, *, name=""):
    tol = TOL[dtype]
    dev = _cmp_device(actual, expected)
    a = actual.detach().to(dev, torch.float64)
    e = expected.detach().to(dev, torch.float64)
    assert a.shape == e.shape, f"{name}: shape {tuple(a.shape)} vs {tuple(e.shape)}"
    bound = tol * (1.0 + e.abs().max().item())
    diff = (a - e).abs().max().item() if a.numel() else 0.0
    assert diff <= bound, f"{name}: max |diff| {diff:.3e} > {bound:.3e}"


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
