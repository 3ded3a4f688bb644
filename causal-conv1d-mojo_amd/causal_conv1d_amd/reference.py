"""Pure-PyTorch reference implementations, exported under the reference's
public names ``causal_conv1d_ref`` / ``causal_conv1d_update_ref``
(``src/causal_conv1d_mojo/reference.py:21-121``).

They are the plain-torch formulation of the op (grouped ``F.conv1d``, computed
in the weight dtype) for callers that want a checker or a device-agnostic
fallback of their own. The package's kernels never call them.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def causal_conv1d_ref(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    initial_states: torch.Tensor | None = None,
    return_final_states: bool = False,
    final_states_out: torch.Tensor | None = None,
    activation: str | None = None,
) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
    """
    x: (batch, dim, seqlen); weight: (dim, width); bias: (dim,)
    initial_states / final_states_out: (batch, dim, width - 1)

    Causal depthwise conv: out[..., t] = bias + sum_k weight[:, k] * xx[..., t + k - (width-1)],
    where xx is x preceded by initial_states (or zeros). Final states are the last
    width-1 columns of cat(initial_states, x) (zero padded on the left when shorter).
    """
    if activation not in (None, "silu", "swish"):
        raise NotImplementedError("activation must be None, silu, or swish")
    dtype_in = x.dtype
    seqlen = x.shape[-1]
    dim, width = weight.shape
    xw = x.to(weight.dtype)
    if initial_states is not None:
        xw = torch.cat([initial_states.to(weight.dtype), xw], dim=-1)
        padded = xw
    else:
        padded = F.pad(xw, (width - 1, 0))
    out = F.conv1d(padded, weight.unsqueeze(1), bias, groups=dim)[..., :seqlen]
    if activation is not None:
        out = F.silu(out)
    out = out.to(dtype_in)
    if not return_final_states:
        return out
    history = xw[..., -(width - 1):] if width > 1 else xw[..., :0]
    final_states = F.pad(history, (width - 1 - history.shape[-1], 0)).to(dtype_in)
    if final_states_out is not None:
        final_states_out.copy_(final_states)
        final_states = final_states_out
    return out, final_states


def causal_conv1d_update_ref(
    x: torch.Tensor,
    conv_state: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    activation: str | None = None,
    cache_seqlens: torch.Tensor | None = None,
) -> torch.Tensor:
    """
    x: (batch, dim) or (batch, dim, seqlen); conv_state: (batch, dim, state_len), mutated.
    cache_seqlens: (batch,) int32 or None; when given, conv_state is a circular
    buffer written at (cache_seqlens + i) % state_len.
    """
    if activation not in (None, "silu", "swish"):
        raise NotImplementedError("activation must be None, silu, or swish")
    dtype_in = x.dtype
    squeeze = x.dim() == 2
    if squeeze:
        x = x.unsqueeze(-1)
    batch, dim, seqlen = x.shape
    width = weight.shape[1]
    state_len = conv_state.shape[-1]
    if conv_state.shape != (batch, dim, state_len) or weight.shape != (dim, width):
        raise ValueError("shape mismatch between x, conv_state and weight")
    if cache_seqlens is None:
        full = torch.cat([conv_state, x], dim=-1).to(weight.dtype)
        conv_state.copy_(full[..., -state_len:])
    else:
        head = cache_seqlens.to(torch.long).unsqueeze(1)
        hist_pos = torch.remainder(head + torch.arange(-(width - 1), 0, device=x.device), state_len)
        history = conv_state.gather(2, hist_pos.unsqueeze(1).expand(batch, dim, width - 1))
        full = torch.cat([history, x], dim=-1).to(weight.dtype)
        write_pos = torch.remainder(head + torch.arange(seqlen, device=x.device), state_len)
        conv_state.scatter_(2, write_pos.unsqueeze(1).expand(batch, dim, seqlen), x)
    # windows of `width` consecutive values; the last `seqlen` windows are the outputs
    windows = full.unfold(-1, width, 1)[:, :, -seqlen:]
    out = (windows * weight.unsqueeze(1)).sum(-1)
    if bias is not None:
        out = out + bias.unsqueeze(-1)
    if activation is not None:
        out = F.silu(out)
    out = out.to(dtype_in)
    return out.squeeze(-1) if squeeze else out
