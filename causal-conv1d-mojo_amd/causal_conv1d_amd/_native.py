"""Tensor-level wrappers over the C ABI: fill a params struct, launch on the
current HIP stream of the tensors' device.

These replace the reference's ``native_fwd`` / ``native_bwd_full`` /
``native_update`` tuple builders (``fwd/__init__.py:11-60``,
``bwd_full/__init__.py:11-73``, ``update/__init__.py:11-60``). There is one
path only: a ROCm device tensor goes to the HIP kernels; anything else
raises NotImplementedError.
"""

from __future__ import annotations

import ctypes

import torch

from causal_conv1d_amd import _lib
from causal_conv1d_amd._dtype import _DTYPE_CODE


def _require_device(x: torch.Tensor) -> None:
    if x.device.type != "cuda" or torch.version.hip is None:
        raise NotImplementedError(
            f"causal_conv1d_amd runs on ROCm GPUs (MI355X / gfx950) only; got a tensor on {x.device}"
        )


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(x: torch.Tensor) -> int:
    return torch.cuda.current_stream(x.device).cuda_stream


def _set3(arr, t: torch.Tensor | None) -> None:
    if t is not None:
        s = t.stride()
        arr[0], arr[1], arr[2] = s[0], s[1], s[2]


def _set2(arr, t: torch.Tensor | None) -> None:
    if t is not None:
        s = t.stride()
        arr[0], arr[1] = s[0], s[1]


def native_fwd(x, weight, bias, seq_idx, initial_states, out, apply_silu, final_states_out=None) -> None:
    _require_device(x)
    lib = _lib.load()
    p = _lib.FwdParams()
    p.x, p.weight, p.bias = x.data_ptr(), weight.data_ptr(), _ptr(bias)
    p.seq_idx, p.initial_states = _ptr(seq_idx), _ptr(initial_states)
    p.out, p.final_states_out = out.data_ptr(), _ptr(final_states_out)
    p.batch, p.dim, p.seqlen = x.shape
    p.width = weight.shape[1]
    _set3(p.x_stride, x)
    _set2(p.weight_stride, weight)
    p.bias_stride = bias.stride(0) if bias is not None else 0
    _set2(p.seq_idx_stride, seq_idx)
    _set3(p.initial_states_stride, initial_states)
    _set3(p.out_stride, out)
    _set3(p.final_states_stride, final_states_out)
    p.dtype = _DTYPE_CODE[x.dtype]
    p.apply_silu = int(bool(apply_silu))
    _lib.check(lib.cc1d_fwd(ctypes.byref(p), _stream(x)))


def _bwd_params(x, weight, bias, dout, seq_idx, initial_states, dx, dinitial_states, apply_silu, dfinal_states):
    p = _lib.BwdParams()
    p.x, p.weight, p.bias, p.dout = x.data_ptr(), weight.data_ptr(), _ptr(bias), dout.data_ptr()
    p.seq_idx, p.initial_states, p.dfinal_states = _ptr(seq_idx), _ptr(initial_states), _ptr(dfinal_states)
    p.dx = dx.data_ptr()
    p.dinitial_states = _ptr(dinitial_states)
    p.batch, p.dim, p.seqlen = x.shape
    p.width = weight.shape[1]
    _set3(p.x_stride, x)
    _set2(p.weight_stride, weight)
    p.bias_stride = bias.stride(0) if bias is not None else 0
    _set3(p.dout_stride, dout)
    _set2(p.seq_idx_stride, seq_idx)
    _set3(p.initial_states_stride, initial_states)
    _set3(p.dfinal_states_stride, dfinal_states)
    _set3(p.dx_stride, dx)
    _set3(p.dinitial_states_stride, dinitial_states)
    p.dtype = _DTYPE_CODE[x.dtype]
    p.apply_silu = int(bool(apply_silu))
    return p


def native_bwd(x, weight, bias, dout, seq_idx, initial_states, dx, dweight_acc, dbias_acc, dinitial_states,
               apply_silu, dfinal_states=None) -> None:
    """cc1d_bwd: adds the fp32 weight/bias-gradient sums into dweight_acc / dbias_acc."""
    _require_device(x)
    lib = _lib.load()
    p = _bwd_params(x, weight, bias, dout, seq_idx, initial_states, dx, dinitial_states, apply_silu, dfinal_states)
    p.dweight_acc, p.dbias_acc = dweight_acc.data_ptr(), _ptr(dbias_acc)
    _set2(p.dweight_acc_stride, dweight_acc)
    p.dbias_acc_stride = dbias_acc.stride(0) if dbias_acc is not None else 0
    _lib.check(lib.cc1d_bwd(ctypes.byref(p), _stream(x)))


def native_bwd_typed(x, weight, bias, dout, seq_idx, initial_states, dx, dweight, dbias, dinitial_states,
                     apply_silu, dfinal_states=None) -> None:
    """cc1d_bwd_typed: writes dweight / dbias in their dtype from a per-call fp32 workspace."""
    _require_device(x)
    lib = _lib.load()
    p = _bwd_params(x, weight, bias, dout, seq_idx, initial_states, dx, dinitial_states, apply_silu, dfinal_states)
    n = lib.cc1d_bwd_workspace_floats(ctypes.byref(p))
    if n < 0:
        _lib.check(lib.cc1d_bwd_typed(ctypes.byref(p), None, _stream(x)))
    ws = torch.empty(max(n, 1), dtype=torch.float32, device=x.device)
    g = _lib.BwdGrads()
    g.dweight, g.dbias, g.workspace = dweight.data_ptr(), _ptr(dbias), ws.data_ptr()
    _set2(g.dweight_stride, dweight)
    g.dbias_stride = dbias.stride(0) if dbias is not None else 0
    g.workspace_floats = ws.numel()
    _lib.check(lib.cc1d_bwd_typed(ctypes.byref(p), ctypes.byref(g), _stream(x)))


def native_bwd_typed_noalloc(x, weight, bias, dout, seq_idx, initial_states, dx, dweight, dbias, dinitial_states,
                             apply_silu, dfinal_states=None) -> None:
    """cc1d_bwd_typed_noalloc: as native_bwd_typed, with the library's static device scratch
    as the workspace (no allocation at all; calls that overlap on one GPU race)."""
    _require_device(x)
    lib = _lib.load()
    p = _bwd_params(x, weight, bias, dout, seq_idx, initial_states, dx, dinitial_states, apply_silu, dfinal_states)
    g = _lib.BwdGrads()
    g.dweight, g.dbias = dweight.data_ptr(), _ptr(dbias)
    _set2(g.dweight_stride, dweight)
    g.dbias_stride = dbias.stride(0) if dbias is not None else 0
    _lib.check(lib.cc1d_bwd_typed_noalloc(ctypes.byref(p), ctypes.byref(g), _stream(x)))


def native_update(x, weight, bias, conv_state, conv_state_indices, cache_seqlens, out, apply_silu) -> None:
    _require_device(x)
    lib = _lib.load()
    p = _lib.UpdateParams()
    p.x, p.weight, p.bias = x.data_ptr(), weight.data_ptr(), _ptr(bias)
    p.conv_state = conv_state.data_ptr()
    p.conv_state_indices, p.cache_seqlens = _ptr(conv_state_indices), _ptr(cache_seqlens)
    p.out = out.data_ptr()
    p.batch, p.dim, p.seqlen = x.shape
    p.width = weight.shape[1]
    p.state_len = conv_state.shape[2]
    p.state_rows = conv_state.shape[0]
    _set3(p.x_stride, x)
    _set2(p.weight_stride, weight)
    p.bias_stride = bias.stride(0) if bias is not None else 0
    _set3(p.conv_state_stride, conv_state)
    _set3(p.out_stride, out)
    p.dtype = _DTYPE_CODE[x.dtype]
    p.apply_silu = int(bool(apply_silu))
    _lib.check(lib.cc1d_update(ctypes.byref(p), _stream(x)))


def native_varlen_states(x, cu_seqlens, states) -> None:
    _require_device(x)
    lib = _lib.load()
    p = _lib.VarlenParams()
    p.x, p.cu_seqlens, p.states = x.data_ptr(), cu_seqlens.data_ptr(), states.data_ptr()
    p.total_tokens, p.dim = x.shape
    p.batch, _, p.state_len = states.shape
    _set2(p.x_stride, x)
    _set3(p.states_stride, states)
    # a bit-for-bit copy: any element type, by its size
    p.dtype = _DTYPE_CODE.get(x.dtype, 0)
    p.elem_bytes = x.element_size()
    _lib.check(lib.cc1d_varlen_states(ctypes.byref(p), _stream(x)))
