"""ctypes binding of ``libcc1d_amd.so`` (the C ABI in ``include/cc1d.h``).

The structures below mirror ``cc1d_fwd_params`` / ``cc1d_bwd_params`` /
``cc1d_bwd_grads`` / ``cc1d_update_params`` / ``cc1d_varlen_params`` field
for field. The library
is loaded on first use; a missing or stale build raises instead of falling
back to anything else.
"""

from __future__ import annotations

import ctypes
import os
import sys
from pathlib import Path

_LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libcc1d_amd.so"
ABI_VERSION = 3
# fp32 elements of the static device scratch of cc1d_bwd_typed_noalloc (CC1D_NOALLOC_WORKSPACE_FLOATS)
NOALLOC_WORKSPACE_FLOATS = 1 << 21

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_vp = ctypes.c_void_p
_i64x2 = _i64 * 2
_i64x3 = _i64 * 3


class FwdParams(ctypes.Structure):
    _fields_ = [
        ("x", _vp), ("weight", _vp), ("bias", _vp), ("seq_idx", _vp), ("initial_states", _vp),
        ("out", _vp), ("final_states_out", _vp),
        ("batch", _i64), ("dim", _i64), ("seqlen", _i64), ("width", _i64),
        ("x_stride", _i64x3), ("weight_stride", _i64x2), ("bias_stride", _i64),
        ("seq_idx_stride", _i64x2), ("initial_states_stride", _i64x3), ("out_stride", _i64x3),
        ("final_states_stride", _i64x3),
        ("dtype", _i32), ("apply_silu", _i32),
    ]


class BwdParams(ctypes.Structure):
    _fields_ = [
        ("x", _vp), ("weight", _vp), ("bias", _vp), ("dout", _vp), ("seq_idx", _vp),
        ("initial_states", _vp), ("dfinal_states", _vp),
        ("dx", _vp), ("dweight_acc", _vp), ("dbias_acc", _vp), ("dinitial_states", _vp),
        ("batch", _i64), ("dim", _i64), ("seqlen", _i64), ("width", _i64),
        ("x_stride", _i64x3), ("weight_stride", _i64x2), ("bias_stride", _i64), ("dout_stride", _i64x3),
        ("seq_idx_stride", _i64x2), ("initial_states_stride", _i64x3), ("dfinal_states_stride", _i64x3),
        ("dx_stride", _i64x3), ("dweight_acc_stride", _i64x2), ("dbias_acc_stride", _i64),
        ("dinitial_states_stride", _i64x3),
        ("dtype", _i32), ("apply_silu", _i32),
    ]


class BwdGrads(ctypes.Structure):
    _fields_ = [
        ("dweight", _vp), ("dbias", _vp), ("workspace", _vp),
        ("dweight_stride", _i64x2), ("dbias_stride", _i64), ("workspace_floats", _i64),
    ]


class UpdateParams(ctypes.Structure):
    _fields_ = [
        ("x", _vp), ("weight", _vp), ("bias", _vp), ("conv_state", _vp), ("conv_state_indices", _vp),
        ("cache_seqlens", _vp), ("out", _vp),
        ("batch", _i64), ("dim", _i64), ("seqlen", _i64), ("width", _i64), ("state_len", _i64),
        ("state_rows", _i64),
        ("x_stride", _i64x3), ("weight_stride", _i64x2), ("bias_stride", _i64),
        ("conv_state_stride", _i64x3), ("out_stride", _i64x3),
        ("dtype", _i32), ("apply_silu", _i32),
    ]


class VarlenParams(ctypes.Structure):
    _fields_ = [
        ("x", _vp), ("cu_seqlens", _vp), ("states", _vp),
        ("total_tokens", _i64), ("dim", _i64), ("batch", _i64), ("state_len", _i64),
        ("x_stride", _i64x2), ("states_stride", _i64x3),
        ("dtype", _i32), ("elem_bytes", _i32),
    ]


EXPORTED_SYMBOLS = (
    "cc1d_abi_version",
    "cc1d_strerror",
    "cc1d_fwd",
    "cc1d_bwd",
    "cc1d_bwd_workspace_floats",
    "cc1d_bwd_typed",
    "cc1d_bwd_typed_noalloc",
    "cc1d_update",
    "cc1d_varlen_states",
)

_lib = None


def library_path() -> Path:
    """The in-tree library; CC1D_AMD_LIB may name another build of it (announced on
    stderr when the library is loaded, so a stray variable cannot go unnoticed)."""
    return Path(os.environ.get("CC1D_AMD_LIB", _LIB_PATH))


def load():
    """Load and type the shared library (cached). Raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.exists():
        raise RuntimeError(
            f"causal_conv1d_amd: native library {path} is not built; "
            "run `python causal-conv1d-mojo_amd/csrc/build.py`"
        )
    if path.resolve() != _LIB_PATH.resolve():
        print(f"causal_conv1d_amd: loading {path} (CC1D_AMD_LIB), not the in-tree {_LIB_PATH}",
              file=sys.stderr, flush=True)
    lib = ctypes.CDLL(str(path))
    lib.cc1d_abi_version.restype = ctypes.c_int
    lib.cc1d_abi_version.argtypes = []
    lib.cc1d_strerror.restype = ctypes.c_char_p
    lib.cc1d_strerror.argtypes = [ctypes.c_int]
    for name, st in (("cc1d_fwd", FwdParams), ("cc1d_bwd", BwdParams), ("cc1d_update", UpdateParams),
                     ("cc1d_varlen_states", VarlenParams)):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.POINTER(st), _vp]
    lib.cc1d_bwd_workspace_floats.restype = ctypes.c_int64
    lib.cc1d_bwd_workspace_floats.argtypes = [ctypes.POINTER(BwdParams)]
    for name in ("cc1d_bwd_typed", "cc1d_bwd_typed_noalloc"):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.POINTER(BwdParams), ctypes.POINTER(BwdGrads), _vp]
    got = lib.cc1d_abi_version()
    if got != ABI_VERSION:
        raise RuntimeError(f"causal_conv1d_amd: ABI version mismatch (library {got}, bindings {ABI_VERSION})")
    _lib = lib
    return lib


def check(status: int) -> None:
    if status != 0:
        msg = load().cc1d_strerror(status).decode()
        raise RuntimeError(f"causal_conv1d_amd native call failed: {msg} (status {status})")
