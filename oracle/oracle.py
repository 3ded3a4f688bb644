"""CPU oracle for the depthwise causal conv1d path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker or the CPU
baseline. The product package (``causal_conv1d_amd``) never imports it.

Layers:

* ``fwd`` / ``bwd`` / ``update`` call the C restatement of the reference's CPU
  kernels (``oracle/cc1d_oracle.c``) on CPU tensors, with the flat argument
  tuples of ``fwd_cpu/__init__.py:139-170``, ``bwd_full_cpu/__init__.py:338-379``
  and ``update_cpu/__init__.py:162-193`` (paths under
  ``/root/reference/src/causal_conv1d_mojo``).
* ``causal_conv1d_fn`` / ``causal_conv1d_bwd`` / ``causal_conv1d_update``
  restate the Python glue around those kernels: ``_fn.py:31-50`` (final
  states), ``_fn.py:221-256`` (forward), ``_fn.py:258-332`` (backward assembly)
  and ``_update.py:117-231`` (decode).
* ``varlen_states`` restates ``causal_conv1d_varlen.py:29-61`` with explicit
  loops.

All functions take and return CPU tensors.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import torch

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "liboracle.so"

DTYPE_CODE = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}

_lib = None


def build() -> Path:
    """Compile the C oracle with its Makefile (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(_LIB_PATH))
    i64, i32, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
    lib.oracle_fwd.argtypes = [i32, i32, i32, vp, vp, vp, vp, i64, i64, i64] + [i64] * 8 + [vp, i64, i64, vp, i64, i64, i64]
    lib.oracle_fwd.restype = i32
    lib.oracle_bwd.argtypes = (
        [i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64]
        + [i64] * 11
        + [vp, i64, i64, vp, i64, i64, i64, vp, i64, i64, i64]
    )
    lib.oracle_bwd.restype = i32
    lib.oracle_update.argtypes = [i32, i32, i32, vp, vp, vp, vp, vp, i64, i64, i64, i64] + [i64] * 11 + [vp, vp]
    lib.oracle_update.restype = i32
    lib.oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
    lib.oracle_bf16_to_f32.restype = ctypes.c_float
    lib.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
    lib.oracle_f32_to_bf16.restype = ctypes.c_uint16
    lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.oracle_f16_to_f32.restype = ctypes.c_float
    lib.oracle_f32_to_f16.argtypes = [ctypes.c_float]
    lib.oracle_f32_to_f16.restype = ctypes.c_uint16
    lib.oracle_num_threads.restype = i32
    _lib = lib
    return lib


def num_threads() -> int:
    return int(_load().oracle_num_threads())


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _s(t, n):
    return list(t.stride()) if t is not None else [0] * n


def _cpu(*ts):
    for t in ts:
        if t is not None and t.device.type != "cpu":
            raise ValueError("the oracle runs on CPU tensors only")


# --------------------------------------------------------------------------
# kernel layer (C)
# --------------------------------------------------------------------------


def fwd(x, weight, bias, seq_idx, initial_states, out, apply_silu):
    """fwd_kernel_cpu (fwd_cpu/kernel.mojo:61-119). Writes ``out``."""
    _cpu(x, weight, bias, seq_idx, initial_states, out)
    if bias is not None:
        bias = bias.contiguous()  # the reference reads bias_ptr[d]
    B, D, L = x.shape
    rc = _load().oracle_fwd(
        DTYPE_CODE[x.dtype], weight.shape[1], int(bool(apply_silu)),
        _p(x), _p(weight), _p(bias), _p(out), B, D, L,
        *x.stride(), *weight.stride(), *out.stride(),
        _p(seq_idx), *_s(seq_idx, 2),
        _p(initial_states), *_s(initial_states, 3),
    )
    if rc:
        raise RuntimeError(f"oracle_fwd failed ({rc})")


def bwd(x, weight, bias, dout, seq_idx, initial_states, dx, dweight_acc, dbias_acc, dinitial_states, apply_silu):
    """bwd_kernel_cpu (bwd_full_cpu/kernel.mojo:108-314). Writes dx/dinit, adds into the fp32 accumulators."""
    _cpu(x, weight, bias, dout, seq_idx, initial_states, dx, dweight_acc, dbias_acc, dinitial_states)
    if bias is not None:
        bias = bias.contiguous()
    assert dweight_acc.dtype == torch.float32 and dweight_acc.is_contiguous()
    assert dbias_acc is None or (dbias_acc.dtype == torch.float32 and dbias_acc.is_contiguous())
    B, D, L = x.shape
    rc = _load().oracle_bwd(
        DTYPE_CODE[x.dtype], weight.shape[1], int(bool(apply_silu)),
        _p(x), _p(weight), _p(bias), _p(dout), _p(dx), _p(dweight_acc), _p(dbias_acc),
        B, D, L, *x.stride(), *weight.stride(), *dout.stride(), *dx.stride(),
        _p(seq_idx), *_s(seq_idx, 2),
        _p(initial_states), *_s(initial_states, 3),
        _p(dinitial_states), *_s(dinitial_states, 3),
    )
    if rc:
        raise RuntimeError(f"oracle_bwd failed ({rc})")


def update(x, weight, bias, conv_state, state_indices, cache_seqlens, out, apply_silu):
    """update_kernel_cpu (update_cpu/kernel.mojo:49-141). x is 3-D. Mutates conv_state, writes out."""
    _cpu(x, weight, bias, conv_state, state_indices, cache_seqlens, out)
    if bias is not None:
        bias = bias.contiguous()
    if state_indices is not None:
        state_indices = state_indices.contiguous()
    if cache_seqlens is not None:
        cache_seqlens = cache_seqlens.contiguous()
    B, D, L = x.shape
    rc = _load().oracle_update(
        DTYPE_CODE[x.dtype], weight.shape[1], int(bool(apply_silu)),
        _p(x), _p(weight), _p(bias), _p(conv_state), _p(out),
        B, D, L, conv_state.shape[2],
        *x.stride(), *weight.stride(), *conv_state.stride(), *out.stride(),
        _p(state_indices), _p(cache_seqlens),
    )
    if rc:
        raise RuntimeError(f"oracle_update failed ({rc})")


def f32_to_bf16_bits(v: float) -> int:
    return int(_load().oracle_f32_to_bf16(v))


def f32_to_f16_bits(v: float) -> int:
    return int(_load().oracle_f32_to_f16(v))


def bf16_bits_to_f32(h: int) -> float:
    return float(_load().oracle_bf16_to_f32(h))


def f16_bits_to_f32(h: int) -> float:
    return float(_load().oracle_f16_to_f32(h))


# --------------------------------------------------------------------------
# glue layer (restated Python around the kernels)
# --------------------------------------------------------------------------


def write_final_states(x, final_states_out, width):
    """_fn.py:31-50: last W-1 columns of x, left zero-padded; initial_states is ignored."""
    seqlen = x.shape[-1]
    pad_left = (width - 1) - seqlen
    if pad_left > 0:
        final_states_out[..., :pad_left].zero_()
        final_states_out[..., pad_left:].copy_(x)
    else:
        final_states_out.copy_(x[..., -(width - 1):])


def causal_conv1d_fn(x, weight, bias=None, seq_idx=None, initial_states=None,
                     return_final_states=False, final_states_out=None, activation=None):
    """Forward as the reference computes it on CPU (_fn.py:221-256 + _fn.py:82-99)."""
    apply_silu = activation in ("silu", "swish")
    B, D, L = x.shape
    W = weight.shape[1]
    out = torch.empty_like(x)
    if initial_states is not None and initial_states.stride(2) != 1:
        initial_states = initial_states.contiguous()
    if seq_idx is not None:
        seq_idx = seq_idx.contiguous()
    if out.numel() > 0:
        fwd(x, weight, bias, seq_idx, initial_states, out, apply_silu)
    if return_final_states:
        if final_states_out is None:
            final_states_out = torch.empty(B, D, W - 1, dtype=x.dtype)
        write_final_states(x, final_states_out, W)
        return out, final_states_out
    return out


def causal_conv1d_bwd(x, weight, bias, dout, seq_idx=None, initial_states=None,
                      dfinal_states=None, activation=None):
    """Backward assembly of _fn.py:258-332. Returns (dx, dweight, dbias, dinitial_states)."""
    apply_silu = activation in ("silu", "swish")
    D, W = weight.shape
    L = x.shape[-1]
    if dout.stride(-1) != 1:
        dout = dout.contiguous()
    dx = torch.empty_like(x)
    dweight_acc = torch.zeros(D, W, dtype=torch.float32)
    dbias_acc = torch.zeros(D, dtype=torch.float32) if bias is not None else None
    dinit = torch.empty_like(initial_states) if initial_states is not None else None
    if seq_idx is not None:
        seq_idx = seq_idx.contiguous()
    if x.numel() > 0:
        bwd(x, weight, bias, dout, seq_idx, initial_states, dx, dweight_acc, dbias_acc, dinit, apply_silu)
    if dfinal_states is not None:
        tail = min(W - 1, L)
        if tail > 0:
            dx[..., -tail:] += dfinal_states[..., -tail:].to(dx.dtype)
    dbias = dbias_acc.to(bias.dtype) if bias is not None else None
    return dx, dweight_acc.to(weight.dtype), dbias, dinit


def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None,
                         cache_seqlens=None, conv_state_indices=None):
    """_update.py:117-231 (validation omitted). Mutates conv_state."""
    apply_silu = activation in ("silu", "swish")
    unsqueeze = x.dim() == 2
    if unsqueeze:
        x = x.unsqueeze(-1)
    out = torch.empty_like(x)
    if x.shape[0] * x.shape[1] > 0:
        update(x, weight, bias, conv_state, conv_state_indices, cache_seqlens, out, apply_silu)
    if unsqueeze:
        out = out.squeeze(-1)
    return out


def varlen_states(x, cu_seqlens, state_len):
    """causal_conv1d_varlen.py:29-61 with explicit loops: (batch, dim, state_len), last
    ``state_len`` tokens of each packed sequence, left zero-padded."""
    _, dim = x.shape
    cu = [int(v) for v in cu_seqlens.tolist()]
    batch = len(cu) - 1
    states = torch.zeros(batch, state_len, dim, dtype=x.dtype).transpose(1, 2)
    for i in range(batch):
        end = cu[i + 1]
        start = max(cu[i], end - state_len)
        n = end - start
        for j in range(n):
            states[i, :, state_len - n + j] = x[start + j]
    return states


__all__ = [
    "build", "num_threads", "fwd", "bwd", "update", "write_final_states",
    "causal_conv1d_fn", "causal_conv1d_bwd", "causal_conv1d_update", "varlen_states",
    "DTYPE_CODE",
]
