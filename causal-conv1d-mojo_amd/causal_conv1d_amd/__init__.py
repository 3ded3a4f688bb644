"""Depthwise causal conv1d for AMD Instinct MI355X (gfx950).

Drop-in for the public API of ``causal_conv1d_mojo``
(``src/causal_conv1d_mojo/__init__.py:39-60``): the same six names with the
same signatures. ``causal_conv1d_fn`` (forward + autograd backward),
``causal_conv1d_update`` (decode) and ``causal_conv1d_varlen_states`` run
hand-written HIP kernels from ``_lib/libcc1d_amd.so`` through its C ABI
(``include/cc1d.h``) on the current HIP stream; they accept ROCm device
tensors only and raise ``NotImplementedError`` for any other device.
``causal_conv1d_ref`` / ``causal_conv1d_update_ref`` are plain-torch
formulations kept for API parity.
"""

from __future__ import annotations

from causal_conv1d_amd._fn import causal_conv1d_fn
from causal_conv1d_amd._update import causal_conv1d_update
from causal_conv1d_amd.causal_conv1d_varlen import (
    causal_conv1d_varlen_states,
    causal_conv1d_varlen_states_ref,
)
from causal_conv1d_amd.reference import causal_conv1d_ref, causal_conv1d_update_ref

__version__ = "1.6.1"

__all__ = [
    "causal_conv1d_fn",
    "causal_conv1d_ref",
    "causal_conv1d_update",
    "causal_conv1d_update_ref",
    "causal_conv1d_varlen_states",
    "causal_conv1d_varlen_states_ref",
]
