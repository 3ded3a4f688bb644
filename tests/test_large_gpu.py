"""Tensors of more than 2**31 elements (4.3+ GB in bf16): the kernels keep
32-bit positions inside a row or batch but 64-bit row / batch offsets, and
the launchers fall back to the 64-bit generic kernels when a batch itself
is too large. Sampled channels at the far end of each tensor are checked
against the oracle (the whole tensors would take minutes on the host).
"""

from __future__ import annotations

import pytest
import torch

import causal_conv1d_amd as cc
from _util import assert_close, assert_reduction_close, scales
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _sample(t, chans):
    return t[:, chans, :].float().cpu().to(t.dtype)


def test_rows_beyond_2_31_elements():
    B, D, L, W = 2, 8192, 140000, 4  # 2.29e9 elements per tensor, contiguous rows
    assert B * D * L > 2 ** 31
    g = torch.Generator(device=DEV).manual_seed(0)
    x = torch.randn(B, D, L, generator=g, device=DEV, dtype=torch.bfloat16)
    w = torch.randn(D, W, generator=g, device=DEV, dtype=torch.bfloat16)
    b = torch.randn(D, generator=g, device=DEV, dtype=torch.bfloat16)
    xg = x.requires_grad_()
    out = cc.causal_conv1d_fn(xg, w, b, activation="silu")
    chans = torch.tensor([0, 4097, D - 1])
    xs, ws, bs = _sample(x.detach(), chans), w[chans].cpu(), b[chans].cpu()
    assert_close(_sample(out.detach(), chans), O.causal_conv1d_fn(xs, ws, bs, activation="silu"), torch.bfloat16)
    dout = torch.randn(B, D, L, generator=g, device=DEV, dtype=torch.bfloat16)
    (dx,) = torch.autograd.grad(out, (xg,), dout)
    rdx, _, _, _ = O.causal_conv1d_bwd(xs, ws, bs, _sample(dout, chans), activation="silu")
    assert_close(_sample(dx, chans), rdx, torch.bfloat16, name="dx")
    del x, xg, out, dout, dx
    torch.cuda.empty_cache()


def test_channel_last_batch_beyond_2_31_elements():
    B, L, D, W = 1, 300000, 8192, 4  # one batch of 2.46e9 elements: 64-bit generic path
    assert L * D > 2 ** 31
    g = torch.Generator(device=DEV).manual_seed(1)
    base = torch.randn(B, L, D, generator=g, device=DEV, dtype=torch.bfloat16)
    w = torch.randn(D, W, generator=g, device=DEV, dtype=torch.bfloat16)
    x = base.transpose(1, 2)
    wg = w.clone().requires_grad_()
    out = cc.causal_conv1d_fn(x, wg, None, activation="silu")
    chans = torch.tensor([1, D // 2 + 3, D - 2])
    xs = x[:, chans, :].float().cpu().to(torch.bfloat16)
    ws = w[chans].cpu()
    assert_close(_sample(out.detach(), chans), O.causal_conv1d_fn(xs, ws, None, activation="silu"),
                 torch.bfloat16)
    dout = torch.randn(B, L, D, generator=g, device=DEV, dtype=torch.bfloat16).transpose(1, 2)
    (dw,) = torch.autograd.grad(out, (wg,), dout)
    _, rdw, _, _ = O.causal_conv1d_bwd(xs, ws, None, _sample(dout, chans), activation="silu")
    sw, _ = scales(xs, ws, None, _sample(dout, chans), activation="silu")
    assert_reduction_close(dw[chans].cpu(), rdw, torch.bfloat16, scale=sw, name="dweight")
    del base, x, out, dout
    torch.cuda.empty_cache()


def test_channel_last_fp32_batch_of_2_30_elements():
    """fp32 channel-last with 2^30 <= L * D < 2^31 elements in one batch entry: element offsets
    fit in 32 bits but byte offsets do not, so the backward must not form 32-bit byte offsets
    (positions past 2^32 / (4 D) would alias earlier rows)."""
    B, L, D, W = 1, 140000, 8192, 4
    assert 2 ** 30 <= L * D < 2 ** 31
    g = torch.Generator(device=DEV).manual_seed(2)
    base = torch.randn(B, L, D, generator=g, device=DEV, dtype=torch.float32)
    w = torch.randn(D, W, generator=g, device=DEV, dtype=torch.float32)
    x = base.transpose(1, 2)
    xg = x.detach().requires_grad_()
    wg = w.clone().requires_grad_()
    out = cc.causal_conv1d_fn(xg, wg, None, activation="silu")
    chans = torch.tensor([0, D // 2 + 1, D - 1])
    xs, ws = _sample(x, chans), w[chans].cpu()
    assert_close(_sample(out.detach(), chans), O.causal_conv1d_fn(xs, ws, None, activation="silu"),
                 torch.float32)
    dout = torch.randn(B, L, D, generator=g, device=DEV, dtype=torch.float32).transpose(1, 2)
    dx, dw = torch.autograd.grad(out, (xg, wg), dout)
    rdx, rdw, _, _ = O.causal_conv1d_bwd(xs, ws, None, _sample(dout, chans), activation="silu")
    assert_close(_sample(dx, chans), rdx, torch.float32, name="dx")
    sw, _ = scales(xs, ws, None, _sample(dout, chans), activation="silu")
    assert_reduction_close(dw[chans].cpu(), rdw, torch.float32, scale=sw, name="dweight")
    del base, x, xg, out, dout, dx
    torch.cuda.empty_cache()
