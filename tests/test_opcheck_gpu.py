"""torch.library.opcheck on the package's custom ops (the boundary the
reference defines at _fn.py:82-201): each op mutates exactly the arguments its
schema declares, its fake implementation agrees with the real one, and it
dispatches through AOT autograd with dynamic shapes -- what torch.compile
relies on when it captures causal_conv1d_fn as one node."""

from __future__ import annotations

import pytest
import torch

import causal_conv1d_amd  # noqa: F401  (registers the ops)
from _util import make_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"
B, D, L, W = 2, 64, 128, 4


def _inputs(dtype):
    x, w, b, init = make_inputs(B, D, L, W, dtype=dtype, has_init=True)
    dout = make_inputs(B, D, L, W, dtype=dtype, seed=1)[0]
    dfs = make_inputs(B, D, W - 1, W, dtype=dtype, seed=2)[0]
    seq = torch.zeros(B, L, dtype=torch.int32)
    seq[:, L // 3:] = 1
    return [t.to(DEV) for t in (x, w, b, init, dout, dfs, seq)]


def _cases(dtype):
    ops = torch.ops.causal_conv1d_amd
    x, w, b, init, dout, dfs, seq = _inputs(dtype)
    out = torch.empty_like(x)
    fs = torch.empty(B, D, W - 1, dtype=dtype, device=DEV)
    dx = torch.empty_like(x)
    dw32 = torch.zeros(D, W, dtype=torch.float32, device=DEV)
    db32 = torch.zeros(D, dtype=torch.float32, device=DEV)
    dwt = torch.empty(D, W, dtype=dtype, device=DEV)
    dbt = torch.empty(D, dtype=dtype, device=DEV)
    dinit = torch.empty_like(init)
    return {
        "fwd": (ops._fwd_inplace.default, (x, w, b, None, None, out, True, None)),
        "fwd_seq_idx": (ops._fwd_inplace.default, (x, w, b, seq, None, out, True, None)),
        "fwd_states": (ops._fwd_inplace.default, (x, w, b, None, init, out, True, fs)),
        "bwd": (ops._bwd_full_inplace.default, (x, w, b, dout, None, None, dx, dw32, db32, None, True)),
        "bwd_states": (ops._bwd_full_inplace.default,
                       (x, w, b, dout, None, init, dx, dw32, db32, dinit, True, dfs)),
        "bwd_typed": (ops._bwd_typed_inplace.default,
                      (x, w, b, dout, None, None, None, dx, dwt, dbt, None, True)),
        "bwd_typed_seq_idx": (ops._bwd_typed_inplace.default,
                              (x, w, b, dout, seq, None, None, dx, dwt, dbt, None, True)),
        "bwd_typed_states": (ops._bwd_typed_inplace.default,
                             (x, w, b, dout, None, init, dfs, dx, dwt, dbt, dinit, True)),
    }


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("case", ["fwd", "fwd_seq_idx", "fwd_states", "bwd", "bwd_states", "bwd_typed",
                                  "bwd_typed_seq_idx", "bwd_typed_states"])
def test_custom_op_passes_opcheck(dtype, case):
    op, args = _cases(dtype)[case]
    torch.library.opcheck(op, args)
