"""C-ABI checks that need no GPU.

* ``libcc1d_amd.so`` loads and exports every function ``include/cc1d.h``
  declares;
* the ctypes structures of ``causal_conv1d_amd._lib`` have the size and
  field offsets that gcc computes from the header;
* argument validation returns the documented status codes before any HIP
  call (NULL params, bad dtype / width / shape, mutually exclusive inputs,
  short conv_state) and zero-size problems return CC1D_OK without work.
"""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from causal_conv1d_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "cc1d.h"

OK, ERR_NULL, ERR_DTYPE, ERR_WIDTH, ERR_SHAPE, ERR_EXCL, ERR_STATE = 0, 1, 2, 3, 4, 5, 6


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def _declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(cc1d_\w+)\s*\(", text, re.M)))


def test_header_declares_the_bound_entry_points():
    assert _declared_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.library_path())], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (cc1d_\w+)$", out, re.M))
    for name in _declared_functions():
        assert name in exported, f"{name} not exported"
        assert getattr(lib, name) is not None


def test_abi_version_and_strerror(lib):
    assert lib.cc1d_abi_version() == _lib.ABI_VERSION == 3
    for code in range(0, 9):
        msg = lib.cc1d_strerror(code).decode()
        assert msg and msg != "unknown status"
    assert lib.cc1d_strerror(99).decode() == "unknown status"


STRUCTS = {
    "cc1d_fwd_params": _lib.FwdParams,
    "cc1d_bwd_params": _lib.BwdParams,
    "cc1d_bwd_grads": _lib.BwdGrads,
    "cc1d_update_params": _lib.UpdateParams,
    "cc1d_varlen_params": _lib.VarlenParams,
}


def test_struct_layout_matches_header(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "cc1d.h"', "int main(void) {"]
    for cname, st in STRUCTS.items():
        lines.append(f'printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for fname, _ in st._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    got = {}
    for ln in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        s, f, v = ln.split()
        got[(s, f)] = int(v)
    for cname, st in STRUCTS.items():
        assert got[(cname, "sizeof")] == ctypes.sizeof(st), cname
        for fname, _ in st._fields_:
            assert got[(cname, fname)] == getattr(st, fname).offset, f"{cname}.{fname}"


def _fwd(**kw):
    p = _lib.FwdParams()
    p.batch, p.dim, p.seqlen, p.width, p.dtype = 1, 8, 16, 4, 1
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def test_fwd_validation_codes(lib):
    call = lambda p: lib.cc1d_fwd(ctypes.byref(p), None)  # noqa: E731
    assert lib.cc1d_fwd(None, None) == ERR_NULL
    assert call(_fwd(dtype=3)) == ERR_DTYPE
    assert call(_fwd(width=1)) == ERR_WIDTH
    assert call(_fwd(width=10)) == ERR_WIDTH
    assert call(_fwd(seqlen=-1)) == ERR_SHAPE
    assert call(_fwd(seq_idx=16, initial_states=16)) == ERR_EXCL
    assert call(_fwd(seq_idx=16, final_states_out=16)) == ERR_EXCL
    assert call(_fwd()) == ERR_NULL  # x / weight / out missing
    assert call(_fwd(batch=0)) == OK  # zero-size: nothing to do
    assert call(_fwd(dim=0)) == OK
    assert call(_fwd(seqlen=0)) == OK  # no final_states requested


def test_bwd_validation_codes(lib):
    def call(**kw):
        p = _lib.BwdParams()
        p.batch, p.dim, p.seqlen, p.width, p.dtype = 1, 8, 16, 4, 1
        for k, v in kw.items():
            setattr(p, k, v)
        return lib.cc1d_bwd(ctypes.byref(p), None)

    assert lib.cc1d_bwd(None, None) == ERR_NULL
    assert call(dtype=-1) == ERR_DTYPE
    assert call(width=11) == ERR_WIDTH
    assert call(seq_idx=16, initial_states=16, dinitial_states=16) == ERR_EXCL
    assert call(seq_idx=16, dfinal_states=16) == ERR_EXCL
    assert call(seq_idx=16, dinitial_states=16) == ERR_EXCL
    assert call(initial_states=16) == ERR_NULL  # dinitial_states missing
    assert call() == ERR_NULL
    assert call(batch=0) == OK
    assert call(seqlen=0) == OK


def test_bwd_typed_validation_codes(lib):
    def params(**kw):
        p = _lib.BwdParams()
        p.batch, p.dim, p.seqlen, p.width, p.dtype = 1, 8, 16, 4, 1
        for k, v in kw.items():
            setattr(p, k, v)
        return p

    def call(grads=True, gkw=None, **kw):
        g = _lib.BwdGrads()
        for k, v in (gkw or {}).items():
            setattr(g, k, v)
        return lib.cc1d_bwd_typed(ctypes.byref(params(**kw)), ctypes.byref(g) if grads else None, None)

    assert lib.cc1d_bwd_typed(None, None, None) == ERR_NULL
    assert call(grads=False) == ERR_NULL
    assert call(dtype=-1) == ERR_DTYPE
    assert call(width=11) == ERR_WIDTH
    assert call(seq_idx=16, dfinal_states=16) == ERR_EXCL
    assert call(seq_idx=16, dinitial_states=16) == ERR_EXCL
    assert call(initial_states=16) == ERR_NULL  # dinitial_states missing
    assert call() == ERR_NULL  # dweight missing
    assert call(gkw=dict(dweight=16)) == ERR_NULL  # x, dout, dx, workspace missing
    assert call(dim=0) == OK
    # workspace size: -1 for invalid params, 0 when there is nothing to sum, else positive
    assert lib.cc1d_bwd_workspace_floats(None) == -1
    assert lib.cc1d_bwd_workspace_floats(ctypes.byref(params(width=11))) == -1
    assert lib.cc1d_bwd_workspace_floats(ctypes.byref(params(seqlen=0))) == 0
    assert lib.cc1d_bwd_workspace_floats(ctypes.byref(params())) > 0


def test_update_validation_codes(lib):
    def call(**kw):
        p = _lib.UpdateParams()
        p.batch, p.dim, p.seqlen, p.width, p.state_len, p.state_rows, p.dtype = 2, 8, 1, 4, 3, 2, 1
        for k, v in kw.items():
            setattr(p, k, v)
        return lib.cc1d_update(ctypes.byref(p), None)

    assert lib.cc1d_update(None, None) == ERR_NULL
    assert call(state_len=2) == ERR_STATE
    assert call(state_rows=1) == ERR_SHAPE  # no indices: one row per batch entry
    assert call(width=10) == ERR_WIDTH
    assert call() == ERR_NULL
    assert call(seqlen=0) == OK
    assert call(batch=0, state_rows=0) == OK


def test_varlen_validation_codes(lib):
    def call(**kw):
        p = _lib.VarlenParams()
        p.total_tokens, p.dim, p.batch, p.state_len, p.dtype = 10, 8, 2, 3, 1
        for k, v in kw.items():
            setattr(p, k, v)
        return lib.cc1d_varlen_states(ctypes.byref(p), None)

    assert lib.cc1d_varlen_states(None, None) == ERR_NULL
    assert call(dtype=7) == ERR_DTYPE
    # an element size overrides the dtype code; only 1, 2, 4, 8 and 16 bytes
    for e in (3, 5, 32, -1):
        assert call(elem_bytes=e) == ERR_DTYPE
    assert call(dtype=7, elem_bytes=8) == ERR_NULL  # valid up to the missing pointers
    assert call(state_len=-1) == ERR_SHAPE
    assert call() == ERR_NULL
    assert call(batch=0) == OK


def _workspace_floats(lib, B, D, L, dtype, channel_last=False, W=4, offsets=(0, 0, 0), seq_stride=None):
    p = _lib.BwdParams()
    fake = 1 << 20  # never dereferenced: the size is computed on the host
    p.x, p.dout, p.dx = (ctypes.c_void_p(fake + o) for o in offsets)  # byte offsets
    p.weight = ctypes.c_void_p(fake)
    if seq_stride is not None:  # seq_idx (B, L) int32 with this time stride
        p.seq_idx = ctypes.c_void_p(fake)
        p.seq_idx_stride[:] = (L * seq_stride, seq_stride)
    p.batch, p.dim, p.seqlen, p.width = B, D, L, W
    strides = (D * L, 1, D) if channel_last else (D * L, L, 1)
    p.x_stride[:] = p.dout_stride[:] = p.dx_stride[:] = strides
    p.weight_stride[:] = (W, 1)
    p.dtype, p.apply_silu = dtype, 1
    return lib.cc1d_bwd_workspace_floats(ctypes.byref(p))


def test_workspace_sizes_of_the_benchmark_configurations(lib):
    """The typed backward's workspace at the benchmark configurations, every one within the
    allocation-free entry point's static scratch."""
    sizes = {
        "C2": _workspace_floats(lib, 4, 5120, 2048, 1),
        "C3": _workspace_floats(lib, 1, 4096, 8192, 1, channel_last=True),
        "C5 bf16": _workspace_floats(lib, 8, 2048, 16384, 1),
        "C5 fp32": _workspace_floats(lib, 8, 2048, 16384, 2),
    }
    assert sizes == {"C2": 102_400, "C3": 163_840, "C5 bf16": 655_360, "C5 fp32": 1_310_720}
    assert max(sizes.values()) <= _lib.NOALLOC_WORKSPACE_FLOATS == 2_097_152


def test_ragged_rows_keep_the_row_kernel(lib):
    """Rows whose length is not a multiple of the 16-byte vector, or that start off a 16-byte
    boundary, are planned as row segments (one record of W + 1 floats per segment of 64 lanes
    x VPT vectors, spanning ceil((L + EPV - 1) / EPV) vectors); the generic kernel would take
    64-step chunks. dout or dx at another offset modulo 16 bytes falls back to it."""
    B, D, W = 1, 64, 4

    def rows(L, epv, aligned=False, B=B, D=D):
        nvec = L // epv if aligned else -(-(L + epv - 1) // epv)
        per = -(-nvec // 64)
        # one segment of 4 rather than two of 2 when the grid keeps 2048 wavefronts
        vpt = 4 if per >= 4 or (per == 3 and B * D >= 2048) else (2 if per >= 2 else 1)
        if vpt == 4 and -(-nvec // 128) * 128 * 100 <= -(-nvec // 256) * 256 * 85:
            vpt = 2  # the last 4-vector segment would be mostly empty
        return B * D * -(-nvec // (64 * vpt)) * (W + 1)

    def generic(L):
        return B * D * -(-L // 64) * (W + 1)

    bf16, fp32 = 1, 2
    assert _workspace_floats(lib, B, D, 2048, bf16) == rows(2048, 8, aligned=True) == 320
    assert _workspace_floats(lib, B, D, 2047, bf16) == rows(2047, 8) == 960  # 257 vectors: 3 of 128
    assert _workspace_floats(lib, B, D, 1001, bf16) == rows(1001, 8) == 320
    assert _workspace_floats(lib, B, D, 1031, bf16) == rows(1031, 8) == 640  # 130 vectors, 64 rows: 2 of 128
    assert _workspace_floats(lib, 4, 5120, 1536, bf16) == rows(1536, 8, True, 4, 5120) == 102_400  # 1 of 256
    assert _workspace_floats(lib, B, D, 7, bf16) == rows(7, 8) == 320
    assert _workspace_floats(lib, B, D, 2047, fp32) == rows(2047, 4) == 1600
    # a base one element past a 16-byte boundary, x / dout / dx alike
    assert _workspace_floats(lib, B, D, 2048, bf16, offsets=(2, 2, 2)) == rows(2048, 8) == 960
    assert _workspace_floats(lib, B, D, 2048, fp32, offsets=(4, 4, 4)) == rows(2048, 4) == 1600
    # dout at another offset inside its vector than x: the generic kernel
    assert _workspace_floats(lib, B, D, 2047, bf16, offsets=(0, 2, 0)) == generic(2047) == 10240
    assert _workspace_floats(lib, B, D, 2048, bf16, offsets=(2, 2, 4)) == generic(2048) == 10240
    # seq_idx: unit time stride keeps the row kernel; the ragged id loads need it, others go generic
    assert _workspace_floats(lib, B, D, 2047, bf16, seq_stride=1) == rows(2047, 8) == 960
    assert _workspace_floats(lib, B, D, 2047, bf16, seq_stride=2) == generic(2047) == 10240
