"""Writes the golden fixtures under tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

The reference ships no golden vectors (its tests draw N(0,1) inputs and
compare against torch). These fixtures freeze inputs together with outputs
computed in float64 by library routines (grouped ``F.conv1d`` and torch
autograd, see ``tests/_util.py``), not by the oracle. Every array is plain
numeric data (``np.savez``, loadable with ``allow_pickle=False``).

Fixtures
  c1_fwd_fp32.npz      benchmark configuration C1: x (2,64,512), weight (64,4), bias (64),
                       N(0,1) from seed 0 in that order, SiLU -> out
  bwd_init_fp32.npz    (2,16,64) W4, bias, SiLU, initial_states, dout, dfinal_states
                       -> dx (with the final-states tail), dweight, dbias, dinitial_states
  seq_repeat_fp32.npz  (2,8,64) W4, bias, SiLU, seq_idx with ids that reappear
                       inside one window and padding -> out, dx, dweight, dbias
  update_fp32.npz      decode bursts [1,3,1,5] in linear (state_len 6) and
                       circular (state_len 5) mode -> outputs and final states
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

from _util import conv_f64, conv_seq_f64, final_states_expected, grads_f64, seq_pattern  # noqa: E402


def _np(t):
    return t.detach().cpu().numpy()


def c1_fwd():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 64, 512, generator=g)
    w = torch.randn(64, 4, generator=g)
    b = torch.randn(64, generator=g)
    out = conv_f64(x, w, b, silu=True)
    np.savez(HERE / "c1_fwd_fp32.npz", x=_np(x), weight=_np(w), bias=_np(b), out=_np(out.float()))


def bwd_init():
    g = torch.Generator().manual_seed(1)
    B, D, L, W = 2, 16, 64, 4
    x = torch.randn(B, D, L, generator=g)
    w = torch.randn(D, W, generator=g)
    b = torch.randn(D, generator=g)
    init = torch.randn(B, D, W - 1, generator=g)
    dout = torch.randn(B, D, L, generator=g)
    dfs = torch.randn(B, D, W - 1, generator=g)
    out = conv_f64(x, w, b, init, silu=True)
    dx, dw, db, dinit = grads_f64(x, w, b, dout, init=init, silu=True)
    # final_states = x[..., -(W-1):] -> its gradient lands on the same columns of dx
    dx = dx.clone()
    dx[..., -(W - 1):] += dfs.double()
    fs = final_states_expected(x, W)
    np.savez(
        HERE / "bwd_init_fp32.npz", x=_np(x), weight=_np(w), bias=_np(b), initial_states=_np(init),
        dout=_np(dout), dfinal_states=_np(dfs), out=_np(out.float()), final_states=_np(fs),
        dx=_np(dx.float()), dweight=_np(dw.float()), dbias=_np(db.float()), dinitial_states=_np(dinit.float()),
    )


def seq_repeat():
    g = torch.Generator().manual_seed(2)
    B, D, L, W = 2, 8, 64, 4
    x = torch.randn(B, D, L, generator=g)
    w = torch.randn(D, W, generator=g)
    b = torch.randn(D, generator=g)
    dout = torch.randn(B, D, L, generator=g)
    s = seq_pattern("repeat_ids", B, L)
    out = conv_seq_f64(x, w, b, s, silu=True)
    dx, dw, db, _ = grads_f64(x, w, b, dout, seq_idx=s, silu=True)
    np.savez(
        HERE / "seq_repeat_fp32.npz", x=_np(x), weight=_np(w), bias=_np(b), seq_idx=_np(s), dout=_np(dout),
        out=_np(out.float()), dx=_np(dx.float()), dweight=_np(dw.float()), dbias=_np(db.float()),
    )


def update():
    g = torch.Generator().manual_seed(3)
    B, D, W = 2, 8, 4
    H = W - 1
    bursts = [1, 3, 1, 5]
    T = sum(bursts)
    w = torch.randn(D, W, generator=g)
    b = torch.randn(D, generator=g)
    x = torch.randn(B, D, T, generator=g)
    # linear: outputs are the full conv over cat(initial state, x), read after the state
    S_lin = 6
    st_lin = torch.randn(B, D, S_lin, generator=g)
    full = torch.cat([st_lin, x], -1)
    out_lin = conv_f64(full, w, b, silu=True)[..., S_lin:]
    fin_lin = full[..., -S_lin:]
    # circular: history = the H values before the write head cs0 (mod S)
    S_cir = 5
    st_cir = torch.randn(B, D, S_cir, generator=g)
    cs0 = torch.tensor([3, 7], dtype=torch.int32)
    hist = torch.stack(
        [st_cir[i][:, [(int(cs0[i]) - H + j) % S_cir for j in range(H)]] for i in range(B)]
    )
    out_cir = conv_f64(torch.cat([hist, x], -1), w, b, silu=True)[..., H:]
    fin_cir = st_cir.clone()
    for i in range(B):
        for t in range(T):
            fin_cir[i, :, (int(cs0[i]) + t) % S_cir] = x[i, :, t]
    np.savez(
        HERE / "update_fp32.npz", weight=_np(w), bias=_np(b), x=_np(x), bursts=np.array(bursts, np.int64),
        state_linear=_np(st_lin), out_linear=_np(out_lin.float()), final_linear=_np(fin_lin),
        state_circular=_np(st_cir), cache_seqlens=_np(cs0), out_circular=_np(out_cir.float()),
        final_circular=_np(fin_cir),
    )


if __name__ == "__main__":
    c1_fwd()
    bwd_init()
    seq_repeat()
    update()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)
