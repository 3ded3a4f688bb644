"""Python API surface and argument validation (no GPU needed).

Mirrors the reference's validation tests (tests/test_fwd.py:146-152,
209-219, 294-310, 386-401, 461-474; tests/test_update.py:246-251;
tests/test_imports.py) -- same exception types and message fragments --
and checks that a valid call on a non-ROCm device raises instead of
running anything on the CPU.
"""

from __future__ import annotations

import ast
import importlib.util
import inspect
import shutil
import sys
from pathlib import Path

import pytest
import torch

import causal_conv1d_amd as cc
from causal_conv1d_amd import reference


def test_public_names_and_version():
    for name in ("causal_conv1d_fn", "causal_conv1d_ref", "causal_conv1d_update", "causal_conv1d_update_ref",
                 "causal_conv1d_varlen_states", "causal_conv1d_varlen_states_ref"):
        assert callable(getattr(cc, name))
    assert set(cc.__all__) >= {"causal_conv1d_fn", "causal_conv1d_update"}
    assert isinstance(cc.__version__, str)
    assert cc.causal_conv1d_varlen_states is cc.causal_conv1d_varlen_states_ref


def _sig(fn):
    args = ast.parse(inspect.getsource(fn).split("\n", 1)[0] + "\n    pass").body[0].args
    return [a.arg for a in args.args], [ast.unparse(d) for d in args.defaults]


def test_signatures_match_the_reference():
    # parameter names / defaults of src/causal_conv1d_mojo/_fn.py:335-344,
    # _update.py:24-32, causal_conv1d_varlen.py:29-31
    sig = inspect.signature(cc.causal_conv1d_fn)
    assert list(sig.parameters) == ["x", "weight", "bias", "seq_idx", "initial_states", "return_final_states",
                                    "final_states_out", "activation"]
    assert [p.default for p in list(sig.parameters.values())[2:]] == [None, None, None, False, None, None]
    sig = inspect.signature(cc.causal_conv1d_update)
    assert list(sig.parameters) == ["x", "conv_state", "weight", "bias", "activation", "cache_seqlens",
                                    "conv_state_indices"]
    assert list(inspect.signature(cc.causal_conv1d_varlen_states).parameters) == ["x", "cu_seqlens", "state_len"]
    assert list(inspect.signature(cc.causal_conv1d_ref).parameters) == [
        "x", "weight", "bias", "initial_states", "return_final_states", "final_states_out", "activation"]
    assert list(inspect.signature(cc.causal_conv1d_update_ref).parameters) == [
        "x", "conv_state", "weight", "bias", "activation", "cache_seqlens"]


def test_custom_ops_registered():
    assert hasattr(torch.ops.causal_conv1d_amd, "_fwd_inplace")
    assert hasattr(torch.ops.causal_conv1d_amd, "_bwd_full_inplace")
    schema = str(torch.ops.causal_conv1d_amd._bwd_full_inplace.default._schema)
    for arg in ("Tensor(a6!) dx", "Tensor(a7!) dweight_acc", "Tensor(a8!)? dbias_acc"):
        assert arg in schema


# ---------------------------------------------------------------- causal_conv1d_fn


def test_width_invalid_raises():
    x = torch.randn(1, 8, 16, dtype=torch.float16)
    with pytest.raises(NotImplementedError, match="width must be in 2..9"):
        cc.causal_conv1d_fn(x, torch.randn(8, 10, dtype=torch.float16))
    x = torch.randn(2, 64, 128)
    with pytest.raises(NotImplementedError, match="width must be in 2..5"):
        cc.causal_conv1d_fn(x, torch.randn(64, 6))


def test_activation_and_dtype_validation():
    x = torch.randn(1, 8, 16)
    w = torch.randn(8, 4)
    with pytest.raises(NotImplementedError, match="activation"):
        cc.causal_conv1d_fn(x, w, activation="relu")
    with pytest.raises(NotImplementedError, match="unsupported dtype"):
        cc.causal_conv1d_fn(x.double(), w.double())
    with pytest.raises(NotImplementedError, match="weight.dtype"):
        cc.causal_conv1d_fn(x, w.half())
    with pytest.raises(NotImplementedError, match="bias.dtype"):
        cc.causal_conv1d_fn(x, w, torch.randn(8).half())


def test_final_states_out_requires_return_final_states():
    x = torch.randn(1, 8, 16, dtype=torch.float16)
    w = torch.randn(8, 4, dtype=torch.float16)
    with pytest.raises(ValueError, match="return_final_states=True"):
        cc.causal_conv1d_fn(x, w, return_final_states=False, final_states_out=torch.empty(1, 8, 3, dtype=torch.float16))


def test_seq_idx_mutual_exclusion_and_validation():
    x = torch.randn(1, 8, 16, dtype=torch.float16)
    w = torch.randn(8, 4, dtype=torch.float16)
    s = torch.zeros(1, 16, dtype=torch.int32)
    with pytest.raises(ValueError, match="mutually exclusive"):
        cc.causal_conv1d_fn(x, w, seq_idx=s, return_final_states=True)
    with pytest.raises(ValueError, match="mutually exclusive"):
        cc.causal_conv1d_fn(x, w, seq_idx=s, initial_states=torch.randn(1, 8, 3, dtype=torch.float16))
    with pytest.raises(ValueError, match="seq_idx.dtype must be int32"):
        cc.causal_conv1d_fn(x, w, seq_idx=s.long())
    with pytest.raises(ValueError, match="seq_idx shape"):
        cc.causal_conv1d_fn(x, w, seq_idx=torch.zeros(1, 15, dtype=torch.int32))


def test_initial_and_final_states_shape_validation():
    x = torch.randn(2, 8, 16, dtype=torch.float16)
    w = torch.randn(8, 4, dtype=torch.float16)
    with pytest.raises(ValueError, match="initial_states shape"):
        cc.causal_conv1d_fn(x, w, initial_states=torch.randn(2, 8, 4, dtype=torch.float16))
    with pytest.raises(ValueError, match="initial_states.dtype"):
        cc.causal_conv1d_fn(x, w, initial_states=torch.randn(2, 8, 3))
    with pytest.raises(ValueError, match="final_states_out shape"):
        cc.causal_conv1d_fn(x, w, return_final_states=True, final_states_out=torch.empty(2, 8, 2, dtype=torch.float16))
    with pytest.raises(ValueError, match="weight shape"):
        cc.causal_conv1d_fn(x, torch.randn(7, 4, dtype=torch.float16))


def test_cpu_tensors_are_refused_not_computed():
    x = torch.randn(1, 8, 16)
    w = torch.randn(8, 4)
    with pytest.raises(NotImplementedError, match="ROCm"):
        cc.causal_conv1d_fn(x, w)
    with pytest.raises(NotImplementedError, match="ROCm"):
        cc.causal_conv1d_update(torch.randn(1, 8), torch.zeros(1, 8, 3), w)
    with pytest.raises(NotImplementedError, match="ROCm"):
        cc.causal_conv1d_varlen_states(torch.randn(4, 8), torch.tensor([0, 4], dtype=torch.int32), 2)


# ---------------------------------------------------------------- causal_conv1d_update


def test_update_state_too_small_raises():
    x = torch.randn(1, 8, 1, dtype=torch.float16)
    with pytest.raises(ValueError, match="must be >="):
        cc.causal_conv1d_update(x, torch.zeros(1, 8, 2, dtype=torch.float16), torch.randn(8, 4, dtype=torch.float16))


def test_update_validation():
    x = torch.randn(2, 8, dtype=torch.float16)
    st = torch.zeros(2, 8, 3, dtype=torch.float16)
    w = torch.randn(8, 4, dtype=torch.float16)
    with pytest.raises(NotImplementedError, match="width must be in 2..9"):
        cc.causal_conv1d_update(x, st, torch.randn(8, 10, dtype=torch.float16))
    with pytest.raises(NotImplementedError, match="conv_state.dtype"):
        cc.causal_conv1d_update(x, st.float(), w)
    with pytest.raises(ValueError, match="conv_state shape"):
        cc.causal_conv1d_update(x, torch.zeros(3, 8, 3, dtype=torch.float16), w)
    with pytest.raises(ValueError, match="cache_seqlens.dtype must be int32"):
        cc.causal_conv1d_update(x, st, w, cache_seqlens=torch.zeros(2, dtype=torch.int64))
    with pytest.raises(ValueError, match="conv_state_indices shape"):
        cc.causal_conv1d_update(x, st, w, conv_state_indices=torch.zeros(3, dtype=torch.int32))
    with pytest.raises(ValueError, match="conv_state_indices.dtype must be int32"):
        cc.causal_conv1d_update(x, st, w, conv_state_indices=torch.zeros(2, dtype=torch.int64))


# ---------------------------------------------------------------- reference functions


@pytest.mark.parametrize("width", [2, 4])
def test_reference_functions_are_plain_torch(width):
    """causal_conv1d_ref / causal_conv1d_update_ref run anywhere (they are API, not the product)."""
    x = torch.randn(2, 8, 12)
    w = torch.randn(8, width)
    b = torch.randn(8)
    out, fs = reference.causal_conv1d_ref(x, w, b, activation="silu", return_final_states=True)
    expect = torch.nn.functional.silu(
        torch.nn.functional.conv1d(torch.nn.functional.pad(x, (width - 1, 0)), w.unsqueeze(1), b, groups=8))
    torch.testing.assert_close(out, expect)
    torch.testing.assert_close(fs, x[..., -(width - 1):])
    st = torch.zeros(2, 8, width - 1)
    dec = torch.stack([reference.causal_conv1d_update_ref(x[..., t], st, w, b, activation="silu")
                       for t in range(12)], -1)
    torch.testing.assert_close(dec, out)


PACKAGE_SOURCES = sorted((Path(__file__).resolve().parent.parent / "causal-conv1d-mojo_amd").rglob("*.py"))


@pytest.mark.parametrize("path", PACKAGE_SOURCES, ids=lambda p: p.name)
def test_modules_do_not_import_the_oracle(path):
    """No module of the package (nor the build script or the compat shim) imports the test oracle:
    checked on the syntax tree, so every import form counts, and on the text."""
    text = path.read_text()
    assert "oracle" not in text, f"{path.name} mentions the oracle"
    for node in ast.walk(ast.parse(text)):
        if isinstance(node, ast.Import):
            assert not any(a.name.split(".")[0] == "oracle" for a in node.names)
        elif isinstance(node, ast.ImportFrom):
            assert (node.module or "").split(".")[0] != "oracle"


COMPAT = Path(__file__).resolve().parent.parent / "causal-conv1d-mojo_amd" / "compat"


def test_compat_namespace_reexports_the_package():
    """``import causal_conv1d`` (compat/src/causal_conv1d/__init__.py:24-48): same five names."""
    sys.path.insert(0, str(COMPAT))
    try:
        sys.modules.pop("causal_conv1d", None)
        import causal_conv1d
    finally:
        sys.path.remove(str(COMPAT))
    assert sorted(causal_conv1d.__all__) == sorted(["__version__", "causal_conv1d_fn", "causal_conv1d_ref",
                                                    "causal_conv1d_update", "causal_conv1d_update_ref"])
    for name in causal_conv1d.__all__:
        assert getattr(causal_conv1d, name) is getattr(cc, name)
    assert not hasattr(causal_conv1d, "causal_conv1d_varlen_states")


def test_compat_namespace_refuses_a_mixed_install(tmp_path):
    """Upstream's interface module beside the shim's __init__ means two installs share the directory."""
    pkg = tmp_path / "causal_conv1d"
    pkg.mkdir()
    shutil.copy(COMPAT / "causal_conv1d" / "__init__.py", pkg / "__init__.py")
    (pkg / "causal_conv1d_interface.py").write_text("")
    spec = importlib.util.spec_from_file_location("causal_conv1d_mixed", pkg / "__init__.py")
    with pytest.raises(ImportError, match="causal_conv1d"):
        spec.loader.exec_module(importlib.util.module_from_spec(spec))
