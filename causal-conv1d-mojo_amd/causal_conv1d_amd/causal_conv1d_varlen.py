"""``causal_conv1d_varlen_states``: last ``state_len`` tokens of each packed
sequence, as the decode ``conv_state`` layout.

Drop-in for ``src/causal_conv1d_mojo/causal_conv1d_varlen.py:29-67`` (same
signature, same output shape / dtype / strides, same ``_ref`` alias). The
reference loops over the batch in Python with one strided torch copy per
sequence; here one HIP gather kernel writes the whole ``(batch, dim,
state_len)`` result, zero padding included. Like the reference's copy it
works for any element type: the kernel moves 1-, 2-, 4-, 8- or 16-byte
elements bit for bit.
"""

from __future__ import annotations

import torch

from causal_conv1d_amd._native import native_varlen_states


def causal_conv1d_varlen_states(x: torch.Tensor, cu_seqlens: torch.Tensor, state_len: int) -> torch.Tensor:
    """
    x: (total_tokens, dim) packed batch of token activations.
    cu_seqlens: (batch + 1,) cumulative sequence lengths starting at 0, sorted non-decreasing.
    state_len: trailing tokens kept per sequence; shorter sequences are left zero-padded.

    Returns states: (batch, dim, state_len), dtype/device of x, allocated as
    (batch, state_len, dim) and transposed (unit stride along dim).
    """
    if x.dim() != 2:
        raise ValueError(f"x shape {tuple(x.shape)}: expected (total_tokens, dim)")
    if cu_seqlens.dim() != 1 or cu_seqlens.shape[0] < 1:
        raise ValueError(f"cu_seqlens shape {tuple(cu_seqlens.shape)}: expected (batch + 1,)")
    if x.element_size() not in (1, 2, 4, 8, 16):
        raise NotImplementedError(f"unsupported dtype {x.dtype}: elements of {x.element_size()} bytes")
    if state_len < 0:
        raise ValueError(f"state_len must be >= 0 (got {state_len})")
    _, dim = x.shape
    batch = cu_seqlens.shape[0] - 1
    if cu_seqlens.dtype != torch.int32 or cu_seqlens.device != x.device or not cu_seqlens.is_contiguous():
        cu_seqlens = cu_seqlens.to(device=x.device, dtype=torch.int32).contiguous()
    states = torch.empty(batch, state_len, dim, dtype=x.dtype, device=x.device).transpose(1, 2)
    native_varlen_states(x, cu_seqlens, states)
    return states


causal_conv1d_varlen_states_ref = causal_conv1d_varlen_states
