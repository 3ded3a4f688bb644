"""GPU parity for causal_conv1d_varlen_states (one HIP gather kernel) against
the reference's known answers (tests/test_varlen.py:25-72) and the oracle's
loop restatement of causal_conv1d_varlen.py:29-61."""

from __future__ import annotations

import pytest
import torch

import causal_conv1d_amd as cc
from _util import assert_equal
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _packed(cu, dim, dtype):
    x = torch.arange(cu[-1] * dim, dtype=dtype).reshape(cu[-1], dim)
    return x, torch.tensor(cu, dtype=torch.int32)


def test_basic_known_answer():
    x, cu = _packed([0, 5, 7, 11], 2, torch.float32)
    out = cc.causal_conv1d_varlen_states(x.to(DEV), cu.to(DEV), state_len=3).cpu()
    assert out.shape == (3, 2, 3) and out.dtype == torch.float32
    assert torch.equal(out[0], x[2:5].T)
    assert torch.equal(out[1, :, 0], torch.zeros(2)) and torch.equal(out[1, :, 1:], x[5:7].T)
    assert torch.equal(out[2], x[8:11].T)


def test_zero_length_sequence():
    x, cu = _packed([0, 3, 3, 5], 4, torch.float32)
    out = cc.causal_conv1d_varlen_states(x.to(DEV), cu.to(DEV), state_len=2).cpu()
    assert torch.equal(out[1], torch.zeros(4, 2))


def test_state_longer_than_all_sequences():
    x, cu = _packed([0, 2, 4], 3, torch.float16)
    out = cc.causal_conv1d_varlen_states(x.to(DEV), cu.to(DEV), state_len=8).cpu()
    assert torch.equal(out[0, :, :6], torch.zeros(3, 6, dtype=torch.float16))
    assert torch.equal(out[0, :, 6:], x[0:2].T)
    assert torch.equal(out[1, :, 6:], x[2:4].T)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_random_packing_matches_oracle_and_layout(dtype):
    g = torch.Generator().manual_seed(0)
    cu = torch.tensor([0, 17, 17, 32, 80, 81], dtype=torch.int32)
    x = torch.randn(81, 64, generator=g).to(dtype)
    out = cc.causal_conv1d_varlen_states(x.to(DEV), cu.to(DEV), 10)
    assert out.stride() == (10 * 64, 1, 64)  # allocated (batch, state_len, dim), transposed
    assert_equal(out.cpu(), O.varlen_states(x, cu, 10))


@pytest.mark.parametrize("dtype", [torch.float64, torch.int64, torch.int32, torch.int16, torch.int8, torch.uint8,
                                   torch.bool, torch.complex64, torch.complex128],
                         ids=lambda d: str(d).replace("torch.", ""))
def test_any_element_type_is_copied_bit_for_bit(dtype):
    """The reference's version is a torch copy, so it accepts every dtype
    (causal_conv1d_varlen.py:49-60); the gather moves raw 1/2/4/8/16-byte elements."""
    g = torch.Generator().manual_seed(2)
    cu = torch.tensor([0, 3, 3, 11, 12, 40], dtype=torch.int32)
    if dtype.is_complex:
        x = torch.randn(40, 24, generator=g, dtype=dtype)
    elif dtype == torch.bool:
        x = torch.randint(0, 2, (40, 24), generator=g).bool()
    elif dtype.is_floating_point:
        x = torch.randn(40, 24, generator=g, dtype=dtype)
    else:
        x = torch.randint(-100 if dtype != torch.uint8 else 0, 100, (40, 24), generator=g).to(dtype)
    out = cc.causal_conv1d_varlen_states(x.to(DEV), cu.to(DEV), 5)
    assert out.dtype == dtype and out.stride() == (5 * 24, 1, 24)
    assert torch.equal(out.cpu(), O.varlen_states(x, cu, 5))


def test_ref_alias():
    assert cc.causal_conv1d_varlen_states is cc.causal_conv1d_varlen_states_ref


def test_prefill_states_feed_decode():
    """varlen states of a packed prefill are the decode conv_state: decoding the
    next token from them equals the forward over the whole sequence."""
    g = torch.Generator().manual_seed(1)
    D, W = 32, 4
    lens = [5, 9, 2]
    cu = torch.tensor([0, 5, 14, 16], dtype=torch.int32)
    w = torch.randn(D, W, generator=g).bfloat16()
    seqs = [torch.randn(n + 1, D, generator=g).bfloat16() for n in lens]  # n prefill tokens + 1 decode token
    packed = torch.cat([s[:-1] for s in seqs])
    states = cc.causal_conv1d_varlen_states(packed.to(DEV), cu.to(DEV), W - 1)
    nxt = torch.stack([s[-1] for s in seqs]).to(DEV)
    dec = cc.causal_conv1d_update(nxt, states.contiguous(), w.to(DEV), activation="silu").cpu()
    for i, s in enumerate(seqs):
        full = cc.causal_conv1d_fn(s.T.unsqueeze(0).contiguous().to(DEV), w.to(DEV), activation="silu").cpu()
        assert_equal(dec[i], full[0, :, -1])
