"""The benchmark configurations C1-C5 at full size.

At these sizes every output is checked against a float64 closed form
computed with torch on the GPU (shifted products and sums: the plain-torch
reference of the same op), and a sample of channels -- all batches and all
positions of each sampled channel, so dweight/dbias of those channels are
complete -- is checked against the CPU oracle on identical inputs.

  C1  (2,64,512) fp32 fwd, seed 0             -> golden fixture
  C2  (4,5120,2048) bf16 fwd+bwd, bias, SiLU
  C3a (1,8192,4096) bf16 stored channel-last, viewed (1,4096,8192), 8 packed
      sequences (seq_idx), SiLU, fwd+bwd
  C3b same layout with initial_states and return_final_states (seq_idx and
      initial/final states are mutually exclusive in the reference API, so
      C3 runs as two sub-configurations)
  C4a decode (256,5120,1) bf16, pool (512,5120,3), 256 random rows, bias, SiLU
  C4b decode (256,5120,4), circular state_len 64, cache_seqlens in [0,64)
  C5  (8,2048,16384) widths 2/3/4 x fp32/fp16/bf16, no bias, no activation, fwd+bwd
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import causal_conv1d_amd as cc
from _util import assert_close, assert_equal, assert_reduction_close, dpre_f64, taps_f64, weight_grads_from_dpre
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = Path(__file__).resolve().parent / "golden"


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _closed_form(x, w, b, seq=None, init=None, silu=False):
    """fp64 forward pieces on the GPU: (pre, out, padded x, tap masks)."""
    pre, xp, masks = taps_f64(x, w, b, seq, init)
    out = F.silu(pre) if silu else pre.clone()
    if seq is not None:
        out = out * (seq >= 0).unsqueeze(1)
    return pre, out, xp, masks


def _closed_form_bwd(x, w, b, dout, seq=None, init=None, silu=False):
    """fp64 (dx, dweight, dbias, dinit) on the GPU, plus the magnitude sums
    (S_dweight, S_dbias) that bound the dweight / dbias comparisons."""
    dpre, xp, masks = dpre_f64(x, w, b, dout, seq, init, silu)
    L = x.shape[-1]
    W = w.shape[1]
    H = W - 1
    dw, db = weight_grads_from_dpre(dpre, xp, masks)
    sw, sb = weight_grads_from_dpre(dpre, xp, masks, absolute=True)
    # dx[t] = sum_k w[W-1-k] dpre[t+k], gated on seq[t+k] == seq[t]
    dp = F.pad(dpre, (0, H))
    dx = torch.zeros_like(dpre)
    for k in range(W):
        term = w.double()[None, :, W - 1 - k, None] * dp[..., k:k + L]
        if seq is not None:
            sp = F.pad(seq.long(), (0, H), value=-(2 ** 40))
            term = term * (sp[:, k:k + L] == seq.long()).unsqueeze(1)
        dx += term
    dinit = None
    if init is not None:
        dinit = torch.stack([sum(w.double()[None, :, k] * dpre[..., i - k] for k in range(i + 1))
                             for i in range(H)], -1)
    return dx, dw, db, dinit, sw, sb


def _sample_channels(D, n=48, seed=0):
    g = _gen(seed)
    sel = torch.cat([torch.arange(min(8, D)), torch.randperm(D, generator=g)[:n]]).unique()
    return sel


def test_c1_golden_on_gpu():
    with np.load(GOLDEN / "c1_fwd_fp32.npz", allow_pickle=False) as z:
        x, w, b, want = (torch.from_numpy(z[k]) for k in ("x", "weight", "bias", "out"))
    out = cc.causal_conv1d_fn(x.to(DEV), w.to(DEV), b.to(DEV), activation="silu").cpu()
    assert_close(out, want, torch.float32)
    assert_close(out, O.causal_conv1d_fn(x, w, b, activation="silu"), torch.float32)


def test_c2_forward_backward_full_size():
    g = _gen(0)
    B, D, L, W = 4, 5120, 2048, 4
    x = torch.randn(B, D, L, generator=g).bfloat16()
    w = torch.randn(D, W, generator=g).bfloat16()
    b = torch.randn(D, generator=g).bfloat16()
    dout = torch.randn(B, D, L, generator=_gen(1)).bfloat16()
    xg, wg, bg = (t.to(DEV).requires_grad_() for t in (x, w, b))
    out = cc.causal_conv1d_fn(xg, wg, bg, activation="silu")
    out.backward(dout.to(DEV))
    # every element vs the fp64 closed form
    _, ref_out, _, _ = _closed_form(x.to(DEV), w.to(DEV), b.to(DEV), silu=True)
    assert_close(out.detach(), ref_out, torch.bfloat16, name="out")
    rdx, rdw, rdb, _, sw, sb = _closed_form_bwd(x.to(DEV), w.to(DEV), b.to(DEV), dout.to(DEV), silu=True)
    assert_close(xg.grad, rdx, torch.bfloat16, name="dx")
    assert_reduction_close(wg.grad, rdw, torch.bfloat16, scale=sw, name="dweight")
    assert_reduction_close(bg.grad, rdb, torch.bfloat16, scale=sb, name="dbias")
    # sampled channels vs the oracle (identical inputs)
    sel = _sample_channels(D)
    xs, ws, bs, gs = x[:, sel].contiguous(), w[sel].contiguous(), b[sel].contiguous(), dout[:, sel].contiguous()
    assert_close(out.detach().cpu()[:, sel], O.causal_conv1d_fn(xs, ws, bs, activation="silu"), torch.bfloat16)
    odx, odw, odb, _ = O.causal_conv1d_bwd(xs, ws, bs, gs, activation="silu")
    assert_close(xg.grad.cpu()[:, sel], odx, torch.bfloat16, name="dx vs oracle")
    assert_reduction_close(wg.grad.cpu()[sel], odw, torch.bfloat16, scale=sw.cpu()[sel], name="dweight vs oracle")
    assert_reduction_close(bg.grad.cpu()[sel], odb, torch.bfloat16, scale=sb.cpu()[sel], name="dbias vs oracle")


def _c3_inputs():
    g = _gen(0)
    L, D, W = 8192, 4096, 4
    x_store = torch.randn(1, L, D, generator=g).bfloat16()  # stored (batch, seqlen, dim)
    w = torch.randn(D, W, generator=g).bfloat16()
    cuts = torch.sort(torch.randperm(L - 1, generator=g)[:7] + 1).values
    seq = torch.zeros(1, L, dtype=torch.int32)
    for i, c in enumerate(cuts.tolist()):
        seq[:, c:] = i + 1
    init = torch.randn(1, D, W - 1, generator=g).bfloat16()
    dout_store = torch.randn(1, L, D, generator=_gen(1)).bfloat16()
    return x_store, w, seq, init, dout_store


def test_c3a_channel_last_varlen_full_size():
    x_store, w, seq, _, dout_store = _c3_inputs()
    D = w.shape[0]
    xs_g = x_store.to(DEV).requires_grad_()
    wg = w.to(DEV).requires_grad_()
    x = xs_g.transpose(1, 2)  # (1, 4096, 8192), stride (L*D, 1, D)
    assert x.stride(1) == 1
    out = cc.causal_conv1d_fn(x, wg, seq_idx=seq.to(DEV), activation="silu")
    assert out.stride() == x.stride()  # channel-last output
    dout = dout_store.to(DEV).transpose(1, 2)
    out.backward(dout)
    xv = x_store.to(DEV).transpose(1, 2)
    _, ref_out, _, _ = _closed_form(xv, w.to(DEV), None, seq.to(DEV), silu=True)
    assert_close(out.detach(), ref_out, torch.bfloat16, name="out")
    rdx, rdw, _, _, sw, _ = _closed_form_bwd(xv, w.to(DEV), None, dout, seq.to(DEV), silu=True)
    assert_close(xs_g.grad.transpose(1, 2), rdx, torch.bfloat16, name="dx")
    assert_reduction_close(wg.grad, rdw, torch.bfloat16, scale=sw, name="dweight")
    sel = _sample_channels(D)
    xcpu = x_store.transpose(1, 2)[:, sel]
    gcpu = dout_store.transpose(1, 2)[:, sel]
    assert_close(out.detach().cpu()[:, sel], O.causal_conv1d_fn(xcpu, w[sel], seq_idx=seq, activation="silu"),
                 torch.bfloat16)
    odx, odw, _, _ = O.causal_conv1d_bwd(xcpu, w[sel], None, gcpu, seq_idx=seq, activation="silu")
    assert_close(xs_g.grad.cpu().transpose(1, 2)[:, sel], odx, torch.bfloat16, name="dx vs oracle")
    assert_reduction_close(wg.grad.cpu()[sel], odw, torch.bfloat16, scale=sw.cpu()[sel], name="dweight vs oracle")


def test_c3b_channel_last_initial_final_states_full_size():
    x_store, w, _, init, dout_store = _c3_inputs()
    D = w.shape[0]
    xs_g = x_store.to(DEV).requires_grad_()
    wg = w.to(DEV).requires_grad_()
    ig = init.to(DEV).requires_grad_()
    x = xs_g.transpose(1, 2)
    out, fs = cc.causal_conv1d_fn(x, wg, initial_states=ig, return_final_states=True, activation="silu")
    assert_equal(fs.cpu(), x_store.transpose(1, 2)[..., -3:].contiguous(), name="final_states")
    out.backward(dout_store.to(DEV).transpose(1, 2))
    xv = x_store.to(DEV).transpose(1, 2)
    _, ref_out, _, _ = _closed_form(xv, w.to(DEV), None, init=init.to(DEV), silu=True)
    assert_close(out.detach(), ref_out, torch.bfloat16, name="out")
    rdx, rdw, _, rdi, sw, _ = _closed_form_bwd(xv, w.to(DEV), None, dout_store.to(DEV).transpose(1, 2),
                                               init=init.to(DEV), silu=True)
    assert_close(xs_g.grad.transpose(1, 2), rdx, torch.bfloat16, name="dx")
    assert_reduction_close(wg.grad, rdw, torch.bfloat16, scale=sw, name="dweight")
    assert_close(ig.grad, rdi, torch.bfloat16, name="dinitial_states")
    sel = _sample_channels(D)
    odx, odw, _, odi = O.causal_conv1d_bwd(x_store.transpose(1, 2)[:, sel], w[sel], None,
                                           dout_store.transpose(1, 2)[:, sel], initial_states=init[:, sel],
                                           activation="silu")
    assert_close(xs_g.grad.cpu().transpose(1, 2)[:, sel], odx, torch.bfloat16, name="dx vs oracle")
    assert_reduction_close(wg.grad.cpu()[sel], odw, torch.bfloat16, scale=sw.cpu()[sel], name="dweight vs oracle")
    assert_close(ig.grad.cpu()[:, sel], odi, torch.bfloat16, name="dinit vs oracle")


@pytest.mark.parametrize("seqlen,S,circular", [(1, 3, False), (4, 64, True)], ids=["C4a", "C4b"])
def test_c4_decode_full_size(seqlen, S, circular):
    g = _gen(0)
    B, D, W = 256, 5120, 4
    x = torch.randn(B, D, seqlen, generator=g).bfloat16()
    w = torch.randn(D, W, generator=g).bfloat16()
    b = torch.randn(D, generator=g).bfloat16()
    pool = torch.randn(512, D, S, generator=g).bfloat16()
    idx = torch.randperm(512, generator=g)[:B].to(torch.int32)
    kw = dict(activation="silu", conv_state_indices=idx)
    if circular:
        kw["cache_seqlens"] = torch.randint(0, 64, (B,), generator=g, dtype=torch.int32)
    xin = x if seqlen > 1 else x[..., 0]
    sg = pool.to(DEV)
    out = cc.causal_conv1d_update(xin.to(DEV), sg, w.to(DEV), b.to(DEV),
                                  **{k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in kw.items()})
    rs = pool.clone()
    rout = O.causal_conv1d_update(xin, rs, w, b, **kw)
    assert_close(out.cpu(), rout, torch.bfloat16, name="out")
    assert_equal(sg.cpu(), rs, name="state pool")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("width", [2, 3, 4])
def test_c5_long_sequence_full_size(dtype, width):
    B, D, L = 8, 2048, 16384
    g = torch.Generator(device=DEV).manual_seed(0)
    x = torch.randn(B, D, L, generator=g, device=DEV).to(dtype)
    w = torch.randn(D, width, generator=g, device=DEV).to(dtype)
    dout = torch.randn(B, D, L, generator=g, device=DEV).to(dtype)
    xg, wg = x.clone().requires_grad_(), w.clone().requires_grad_()
    out = cc.causal_conv1d_fn(xg, wg)
    out.backward(dout)
    _, ref_out, _, _ = _closed_form(x, w, None)
    assert_close(out.detach(), ref_out, dtype, name="out")
    del ref_out
    rdx, rdw, _, _, sw, _ = _closed_form_bwd(x, w, None, dout)
    assert_close(xg.grad, rdx, dtype, name="dx")
    assert_reduction_close(wg.grad, rdw, dtype, scale=sw, name="dweight")
    del rdx
    sel = _sample_channels(D, n=16).to(DEV)
    xs, ws, gs = (t.cpu().contiguous() for t in (x[:, sel], w[sel], dout[:, sel]))
    assert_close(out.detach()[:, sel].cpu(), O.causal_conv1d_fn(xs, ws), dtype)
    odx, odw, _, _ = O.causal_conv1d_bwd(xs, ws, None, gs)
    assert_close(xg.grad[:, sel].cpu(), odx, dtype, name="dx vs oracle")
    assert_reduction_close(wg.grad[sel].cpu(), odw, dtype, scale=sw[sel].cpu(), name="dweight vs oracle")
