"""``causal_conv1d_fn``: forward + autograd backward on MI355X.

Drop-in for the reference's ``causal_conv1d_fn`` (``src/causal_conv1d_mojo/_fn.py:335-520``):
same signature, same argument checks in the same order with the same
exception types and message fragments, same custom-op boundary
(``_fwd_inplace`` / ``_bwd_full_inplace``, ``_fn.py:82-201``) and the same
autograd contract (``_fn.py:204-332``).

Differences in *where* work happens (results are the same):

* ``final_states_out`` is written by the forward kernel itself instead of a
  separate torch copy (``_fn.py:31-50`` semantics, including the zero left
  pad that ignores ``initial_states``).
* the ``dfinal_states`` tail add of the backward (``_fn.py:308-315``) is done
  inside the backward kernel with the same two roundings (dx rounded to the
  dtype, then the sum rounded again).
* the autograd backward gets dweight / dbias in their dtype from
  ``_bwd_typed_inplace`` (one kernel writes fp32 partial sums, one kernel adds
  them per channel in a fixed order and rounds once) instead of zero-filled
  fp32 accumulators, atomics and two casts; the sums are fp32 as in the
  reference, and the same inputs give the same bits on every run.
* ``dout`` keeps its layout when it already matches ``x`` (the kernels read
  any strides); only a mismatching layout is copied once.
* widths 6..9 with autograd are accepted at any seqlen (the reference needs
  seqlen % 1024 == 0 there, ``_fn.py:415-423``).
"""

from __future__ import annotations

import torch

from causal_conv1d_amd._dtype import _DTYPE_CODE
from causal_conv1d_amd._native import native_bwd, native_bwd_typed, native_fwd


def _fwd_inplace_impl(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    seq_idx: torch.Tensor | None,
    initial_states: torch.Tensor | None,
    out: torch.Tensor,
    apply_silu: bool,
    final_states_out: torch.Tensor | None,
) -> None:
    native_fwd(x, weight, bias, seq_idx, initial_states, out, apply_silu, final_states_out)


def _fwd_inplace_fake(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    seq_idx: torch.Tensor | None,
    initial_states: torch.Tensor | None,
    out: torch.Tensor,
    apply_silu: bool,
    final_states_out: torch.Tensor | None,
) -> None:
    return None


_fwd_inplace = torch.library.custom_op(
    "causal_conv1d_amd::_fwd_inplace",
    mutates_args=("out", "final_states_out"),
)(_fwd_inplace_impl)
_fwd_inplace.register_fake(_fwd_inplace_fake)


def _bwd_full_inplace_impl(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    dout: torch.Tensor,
    seq_idx: torch.Tensor | None,
    initial_states: torch.Tensor | None,
    dx: torch.Tensor,
    dweight_acc: torch.Tensor,
    dbias_acc: torch.Tensor | None,
    dinitial_states: torch.Tensor | None,
    apply_silu: bool,
    dfinal_states: torch.Tensor | None = None,
) -> None:
    native_bwd(
        x, weight, bias, dout, seq_idx, initial_states, dx, dweight_acc, dbias_acc,
        dinitial_states, apply_silu, dfinal_states,
    )


def _bwd_full_inplace_fake(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    dout: torch.Tensor,
    seq_idx: torch.Tensor | None,
    initial_states: torch.Tensor | None,
    dx: torch.Tensor,
    dweight_acc: torch.Tensor,
    dbias_acc: torch.Tensor | None,
    dinitial_states: torch.Tensor | None,
    apply_silu: bool,
    dfinal_states: torch.Tensor | None = None,
) -> None:
    return None


_bwd_full_inplace = torch.library.custom_op(
    "causal_conv1d_amd::_bwd_full_inplace",
    mutates_args=("dx", "dweight_acc", "dbias_acc", "dinitial_states"),
)(_bwd_full_inplace_impl)
_bwd_full_inplace.register_fake(_bwd_full_inplace_fake)


def _bwd_typed_inplace_impl(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    dout: torch.Tensor,
    seq_idx: torch.Tensor | None,
    initial_states: torch.Tensor | None,
    dfinal_states: torch.Tensor | None,
    dx: torch.Tensor,
    dweight: torch.Tensor,
    dbias: torch.Tensor | None,
    dinitial_states: torch.Tensor | None,
    apply_silu: bool,
) -> None:
    native_bwd_typed(
        x, weight, bias, dout, seq_idx, initial_states, dx, dweight, dbias, dinitial_states, apply_silu,
        dfinal_states,
    )


def _bwd_typed_inplace_fake(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    dout: torch.Tensor,
    seq_idx: torch.Tensor | None,
    initial_states: torch.Tensor | None,
    dfinal_states: torch.Tensor | None,
    dx: torch.Tensor,
    dweight: torch.Tensor,
    dbias: torch.Tensor | None,
    dinitial_states: torch.Tensor | None,
    apply_silu: bool,
) -> None:
    return None


# The autograd backward's op: the same kernel as _bwd_full_inplace, but the
# weight/bias gradients come back in their dtype from one extra reduction
# kernel, instead of two zero-fills, fp32 atomics and two casts.
_bwd_typed_inplace = torch.library.custom_op(
    "causal_conv1d_amd::_bwd_typed_inplace",
    mutates_args=("dx", "dweight", "dbias", "dinitial_states"),
)(_bwd_typed_inplace_impl)
_bwd_typed_inplace.register_fake(_bwd_typed_inplace_fake)


def _match_layout(t: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    """Return ``t`` with the memory layout of ``like`` (a copy only if needed)."""
    if t.stride() == like.stride():
        return t
    if like.stride(-1) == 1:
        return t if t.stride(-1) == 1 else t.contiguous()
    return torch.empty_like(like).copy_(t)


class _CausalConv1dFn(torch.autograd.Function):
    """Autograd op (``_fn.py:204-332``): saves x/weight/bias/seq_idx/initial_states,
    recomputes the pre-activation in the fused backward kernel."""

    @staticmethod
    def forward(
        ctx,
        x: torch.Tensor,
        weight: torch.Tensor,
        bias: torch.Tensor | None,
        seq_idx: torch.Tensor | None,
        initial_states: torch.Tensor | None,
        apply_silu: bool,
        final_states_out: torch.Tensor | None,
    ):
        out = torch.empty_like(x)
        torch.ops.causal_conv1d_amd._fwd_inplace(
            x, weight, bias, seq_idx, initial_states, out, apply_silu, final_states_out
        )
        ctx.save_for_backward(x, weight, bias, seq_idx, initial_states)
        ctx.apply_silu = apply_silu
        ctx.has_bias = bias is not None
        ctx.return_final_states = final_states_out is not None
        if final_states_out is not None:
            return out, final_states_out
        return out

    @staticmethod
    def backward(ctx, *grad_outputs):
        dout = grad_outputs[0]
        dfinal_states = grad_outputs[1] if ctx.return_final_states else None
        x, weight, bias, seq_idx, initial_states = ctx.saved_tensors
        D, W = weight.shape
        dout = _match_layout(dout, x)
        dx = torch.empty_like(x)
        # fp32 sums rounded once to the parameter dtype, as the reference's
        # accumulators + casts (_fn.py:276-292,317-320)
        dweight = torch.empty(D, W, dtype=weight.dtype, device=x.device)
        dbias = torch.empty(D, dtype=bias.dtype, device=x.device) if ctx.has_bias else None
        dinitial_states = torch.empty_like(initial_states) if initial_states is not None else None
        if dfinal_states is not None and dfinal_states.dtype != x.dtype:
            dfinal_states = dfinal_states.to(x.dtype)
        torch.ops.causal_conv1d_amd._bwd_typed_inplace(
            x, weight, bias, dout, seq_idx, initial_states, dfinal_states, dx, dweight, dbias,
            dinitial_states, ctx.apply_silu,
        )
        return dx, dweight, dbias, None, dinitial_states, None, None


def causal_conv1d_fn(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    seq_idx: torch.Tensor | None = None,
    initial_states: torch.Tensor | None = None,
    return_final_states: bool = False,
    final_states_out: torch.Tensor | None = None,
    activation: str | None = None,
) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
    """
    x: (batch, dim, seqlen)
    weight: (dim, width)
    bias: (dim,)
    seq_idx: (batch, seqlen)
    initial_states: (batch, dim, width - 1)
    final_states_out: (batch, dim, width - 1), to be written to
    activation: either None or "silu" or "swish"

    out: (batch, dim, seqlen)
    """
    if activation not in (None, "silu", "swish"):
        raise NotImplementedError("only activation in {None, 'silu', 'swish'} is supported")
    if x.dtype not in _DTYPE_CODE:
        raise NotImplementedError(f"unsupported dtype {x.dtype}; only fp16/bf16/fp32 are supported")
    if weight.dtype != x.dtype:
        raise NotImplementedError(f"weight.dtype ({weight.dtype}) must match x.dtype ({x.dtype})")
    if bias is not None and bias.dtype != x.dtype:
        raise NotImplementedError(f"bias.dtype ({bias.dtype}) must match x.dtype ({x.dtype})")
    if x.dim() != 3 or weight.dim() != 2:
        raise ValueError(
            f"expected x of shape (batch, dim, seqlen) and weight of shape (dim, width); "
            f"got x {tuple(x.shape)}, weight {tuple(weight.shape)}"
        )
    width = weight.shape[1]
    max_width = 5 if x.dtype == torch.float32 else 9
    if width < 2 or width > max_width:
        dtype_name = "fp32" if x.dtype == torch.float32 else "fp16/bf16"
        raise NotImplementedError(f"width must be in 2..{max_width} for {dtype_name} (got {width})")
    if x.device != weight.device or (bias is not None and x.device != bias.device):
        raise NotImplementedError(
            f"x, weight, bias must all be on the same device "
            f"(got x={x.device}, weight={weight.device}, "
            f"bias={'None' if bias is None else bias.device})"
        )
    if final_states_out is not None and not return_final_states:
        raise ValueError("final_states_out is only meaningful when return_final_states=True")

    batch, dim, seqlen = x.shape
    if weight.shape[0] != dim:
        raise ValueError(f"weight shape {tuple(weight.shape)} != expected ({dim}, width)")
    if bias is not None and tuple(bias.shape) != (dim,):
        raise ValueError(f"bias shape {tuple(bias.shape)} != expected {(dim,)}")

    if seq_idx is not None:
        if return_final_states:
            raise ValueError(
                "seq_idx and return_final_states are mutually exclusive "
                "(packed sequences have no single 'last W-1 cols')"
            )
        if initial_states is not None:
            raise ValueError("seq_idx and initial_states are mutually exclusive")
        if seq_idx.shape != (batch, seqlen):
            raise ValueError(f"seq_idx shape {tuple(seq_idx.shape)} != expected {(batch, seqlen)}")
        if seq_idx.dtype != torch.int32:
            raise ValueError(f"seq_idx.dtype must be int32 (got {seq_idx.dtype})")
        if seq_idx.device != x.device:
            raise ValueError(f"seq_idx.device ({seq_idx.device}) must match x.device ({x.device})")
        if not seq_idx.is_contiguous():
            seq_idx = seq_idx.contiguous()

    if initial_states is not None:
        if initial_states.shape != (batch, dim, width - 1):
            raise ValueError(
                f"initial_states shape {tuple(initial_states.shape)} != expected {(batch, dim, width - 1)}"
            )
        if initial_states.dtype != x.dtype:
            raise ValueError(f"initial_states.dtype ({initial_states.dtype}) must match x.dtype ({x.dtype})")
        if initial_states.device != x.device:
            raise ValueError(
                f"initial_states.device ({initial_states.device}) must match x.device ({x.device})"
            )

    if return_final_states:
        if final_states_out is None:
            final_states_out = torch.empty(batch, dim, width - 1, dtype=x.dtype, device=x.device)
        else:
            if final_states_out.shape != (batch, dim, width - 1):
                raise ValueError(
                    f"final_states_out shape {tuple(final_states_out.shape)} "
                    f"!= expected {(batch, dim, width - 1)}"
                )
            if final_states_out.dtype != x.dtype:
                raise ValueError(
                    f"final_states_out.dtype ({final_states_out.dtype}) must match x.dtype ({x.dtype})"
                )
            if final_states_out.device != x.device:
                raise ValueError(
                    f"final_states_out.device ({final_states_out.device}) must match x.device ({x.device})"
                )

    apply_silu = activation in ("silu", "swish")
    return _CausalConv1dFn.apply(x, weight, bias, seq_idx, initial_states, apply_silu, final_states_out)
