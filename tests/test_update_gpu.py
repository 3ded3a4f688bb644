"""GPU decode-update parity: causal_conv1d_update on MI355X vs the oracle
(update_cpu/kernel.mojo restated) on the same inputs and the same initial
state; both the outputs and the mutated conv_state are compared.

Coverage follows the reference's tests/test_update.py: single token with
state_len = W-1, short bursts, decode loop == full forward (bit-exact for
fp16/bf16), circular buffer incl. cache_seqlens >= state_len, circular decode
loop, conv_state_indices pools, padding rows (-1, -2, INT32_MIN, out of pool), plus the benchmark decode
shapes at reduced batch and out-of-pool indices.
"""

from __future__ import annotations

import pytest
import torch

import causal_conv1d_amd as cc
from _util import DTYPE_IDS, DTYPES, assert_close, assert_equal, make_inputs
from causal_conv1d_amd._native import native_update
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(x, state, w, b=None, **kw):
    sg = state.to(DEV)
    out = cc.causal_conv1d_update(x.to(DEV), sg, w.to(DEV), None if b is None else b.to(DEV),
                                  **{k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in kw.items()})
    torch.cuda.synchronize()
    rs = state.clone()
    ref = O.causal_conv1d_update(x, rs, w, b, **kw)
    return out.cpu(), sg.cpu(), ref, rs


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4, 5, 9])
@pytest.mark.parametrize("activation", [None, "silu"])
@pytest.mark.parametrize("has_bias", [True, False], ids=["bias", "nobias"])
# 1400: 11 channel groups of 128 bf16 channels, the last one partial, in workgroups of 4 groups
@pytest.mark.parametrize("dim", [16, 40, 1400, 2048])
def test_single_token(dtype, width, activation, has_bias, dim):
    x, w, b, _ = make_inputs(3, dim, 1, width, dtype=dtype, has_bias=has_bias)
    state = make_inputs(3, dim, width - 1, width, dtype=dtype, seed=1)[0]
    out, st, rout, rst = _run(x[..., 0], state, w, b, activation=activation)
    assert out.shape == (3, dim)
    assert_close(out, rout, dtype, name="out")
    assert_equal(st, rst, name="state")


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4])
@pytest.mark.parametrize("seqlen,state_extra", [(3, 4), (1, 4), (6, 0), (8, 2), (2, 0)])
def test_short_burst_linear(dtype, width, seqlen, state_extra):
    x, w, b, _ = make_inputs(2, 8, seqlen, width, dtype=dtype)
    state = make_inputs(2, 8, width - 1 + state_extra, width, dtype=dtype, seed=1)[0]
    out, st, rout, rst = _run(x, state, w, b, activation="silu")
    assert_close(out, rout, dtype)
    assert_equal(st, rst, name="state")


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("has_bias", [True, False], ids=["bias", "nobias"])
def test_decode_loop_matches_full_forward_bit_exact(dtype, has_bias):
    x, w, b, _ = make_inputs(2, 16, 24, 4, dtype=dtype, has_bias=has_bias)
    xg, wg = x.to(DEV), w.to(DEV)
    bg = b.to(DEV) if b is not None else None
    full = cc.causal_conv1d_fn(xg, wg, bg, activation="silu")
    state = torch.zeros(2, 16, 3, dtype=dtype, device=DEV)
    dec = torch.cat([cc.causal_conv1d_update(xg[:, :, t:t + 1], state, wg, bg, activation="silu")
                     for t in range(24)], -1)
    # forward and update share the tap loop and epilogue: identical bits (reference
    # test_update.py:70-96 allows 1e-6 for fp32; this build is exact for all dtypes)
    assert_equal(dec.cpu(), full.cpu())


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4])
@pytest.mark.parametrize("activation", [None, "silu"])
@pytest.mark.parametrize("seqlen", [1, 3, 9])
def test_circular_buffer(dtype, width, activation, seqlen):
    S = width + 5
    x, w, b, _ = make_inputs(2, 16, seqlen, width, dtype=dtype)
    state = make_inputs(2, 16, S, width, dtype=dtype, seed=1)[0]
    cs = torch.tensor([S // 2, S + 3], dtype=torch.int32)
    out, st, rout, rst = _run(x, state, w, b, activation=activation, cache_seqlens=cs)
    assert_close(out, rout, dtype)
    assert_equal(st, rst, name="state")


def test_circular_negative_head_uses_floored_modulo():
    x, w, b, _ = make_inputs(2, 8, 2, 4, dtype=torch.float32)
    state = torch.randn(2, 8, 6)
    cs = torch.tensor([-1, -13], dtype=torch.int32)
    out, st, rout, rst = _run(x, state, w, b, activation="silu", cache_seqlens=cs)
    assert_close(out, rout, torch.float32)
    assert_equal(st, rst)


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
def test_circular_decode_loop(dtype):
    x, w, _, _ = make_inputs(1, 8, 16, 4, dtype=dtype)
    xg, wg = x.to(DEV), w.to(DEV)
    full = cc.causal_conv1d_fn(xg, wg, activation="silu")
    state = torch.zeros(1, 8, 3, dtype=dtype, device=DEV)
    dec = [cc.causal_conv1d_update(xg[:, :, t:t + 1], state, wg, activation="silu",
                                   cache_seqlens=torch.tensor([t], dtype=torch.int32, device=DEV))
           for t in range(16)]
    assert_equal(torch.cat(dec, -1).cpu(), full.cpu())


def _chunk_cases():
    """Circular updates on state lines of whole 16-byte chunks (the chunked kernel): every
    window offset inside a chunk, windows that cross a chunk or wrap past the line end."""
    for dtype, did in zip(DTYPES, DTYPE_IDS):
        epv = 16 // torch.tensor([], dtype=dtype).element_size()
        for width in ([2, 4, 5] if dtype == torch.float32 else [2, 4, 5, 9]):
            for seqlen in sorted({1, 2, epv + 1 - (width - 1)} - {0}):
                if seqlen < 1 or width - 1 + seqlen > epv + 1:
                    continue
                for S in (2 * epv, 3 * epv, 64):
                    yield pytest.param(dtype, width, seqlen, S, id=f"{did}-w{width}-L{seqlen}-S{S}")


@pytest.mark.parametrize("dtype,width,seqlen,S", list(_chunk_cases()))
def test_circular_chunked_lines(dtype, width, seqlen, S):
    B, D = S + 4, 48
    x, w, b, _ = make_inputs(B, D, seqlen, width, dtype=dtype)
    pool = make_inputs(B + 3, D, S, width, dtype=dtype, seed=1)[0]
    g = torch.Generator().manual_seed(3)
    idx = torch.randperm(B + 3, generator=g)[:B].to(torch.int32)
    idx[5] = -1  # one padding entry
    # every head position of the line (plus >= S and negative heads), so every offset in a chunk
    cs = torch.cat([torch.arange(S), torch.tensor([S, 2 * S + 1, -1, -S - 2])]).to(torch.int32)[:B]
    out, st, rout, rst = _run(x, pool, w, b, activation="silu", cache_seqlens=cs, conv_state_indices=idx)
    assert_close(out, rout, dtype)
    assert torch.all(out[5] == 0)
    assert_equal(st, rst, name="pool")


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("circular", [False, True])
@pytest.mark.parametrize("dim", [16, 64, 512])  # 512: whole wavefronts per batch entry (scalar index reads)
def test_conv_state_indices_pool(dtype, circular, dim):
    x, w, b, _ = make_inputs(3, dim, 1, 4, dtype=dtype)
    S = 3 if not circular else 7
    pool = make_inputs(5, dim, S, 4, dtype=dtype, seed=1)[0]
    idx = torch.tensor([3, 0, 4], dtype=torch.int32)
    kw = dict(activation="silu", conv_state_indices=idx)
    if circular:
        kw["cache_seqlens"] = torch.tensor([2, 9, 0], dtype=torch.int32)
    out, st, rout, rst = _run(x[..., 0], pool, w, b, **kw)
    assert_close(out, rout, dtype)
    assert_equal(st, rst, name="pool")
    for r in (1, 2):
        assert_equal(st[r], pool[r], name=f"untouched row {r}")


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("dim", [8, 64, 1024])  # 1024: whole wavefronts per batch entry (scalar index reads)
@pytest.mark.parametrize("circular", [False, True])
def test_padding_and_out_of_pool_rows(dtype, dim, circular):
    # every negative index is padding (-1, -2, INT32_MIN), and so is an index >= the pool size
    idx = torch.tensor([0, -1, 2, 4, -2, -(2 ** 31), 3, 9], dtype=torch.int32)
    B = idx.numel()
    x, w, b, _ = make_inputs(B, dim, 1, 4, dtype=dtype)
    S = 16 if circular else 3  # 16: whole 16-byte chunks per state line (the chunked circular kernel)
    pool = make_inputs(4, dim, S, 4, dtype=dtype, seed=1)[0]
    cs = torch.tensor([1, 5, 6, 0, 2, 3, 19, 4], dtype=torch.int32) if circular else None
    sg = pool.to(DEV)
    # through the C ABI with an output prefilled with NaN, so a padding entry that is not written shows
    og = torch.full((B, dim, 1), float("nan"), dtype=dtype, device=DEV)
    native_update(x.to(DEV), w.to(DEV), b.to(DEV), sg, idx.to(DEV), None if cs is None else cs.to(DEV), og, True)
    out = og[..., 0].cpu()
    pad = torch.tensor([1, 3, 4, 5, 7])
    assert torch.all(out[pad] == 0)
    st = sg.cpu()
    assert_equal(st[1], pool[1])
    real = torch.tensor([0, 2, 6])
    rs = pool[idx[real].long()].clone()
    kw = dict(activation="silu")
    if circular:
        kw["cache_seqlens"] = cs[real]
    rout = O.causal_conv1d_update(x[real, :, 0], rs, w, b, **kw)
    assert_close(out[real], rout, dtype)
    assert_equal(st[idx[real].long()], rs)
    # the public API gives the same
    sg2 = pool.to(DEV)
    kw2 = dict(activation="silu", conv_state_indices=idx.to(DEV))
    if circular:
        kw2["cache_seqlens"] = cs.to(DEV)
    out2 = cc.causal_conv1d_update(x[..., 0].to(DEV), sg2, w.to(DEV), b.to(DEV), **kw2).cpu()
    assert_equal(out2, out)
    assert_equal(sg2.cpu(), st)


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("width", [2, 3, 4, 5])
@pytest.mark.parametrize("dim", [136, 200])  # whole 16-byte vectors, a partial last channel group
def test_odd_batch_offset_indices(dtype, width, dim):
    """Two batch entries per wavefront with an odd batch (the last wavefront's second entry is
    past the end), indices read from a view at a 4-byte (not 8-byte) aligned address, and a
    channel group that ends inside a wavefront (both dims take the direct decode kernel)."""
    B, P = 7, 9
    full = torch.tensor([99, 3, 0, -1, 8, 5, -3, 1], dtype=torch.int32)
    idx = full.to(DEV)[1:]  # storage offset of one int32
    assert idx.data_ptr() % 8 == 4
    x, w, b, _ = make_inputs(B, dim, 1, width, dtype=dtype)
    pool = make_inputs(P, dim, width - 1, width, dtype=dtype, seed=1)[0]
    sg = pool.to(DEV)
    og = torch.full((B, dim, 1), float("nan"), dtype=dtype, device=DEV)
    native_update(x.to(DEV), w.to(DEV), b.to(DEV), sg, idx, None, og, True)
    out, st = og[..., 0].cpu(), sg.cpu()
    ids = full[1:]
    real = (ids >= 0).nonzero().flatten()
    assert torch.all(out[(ids < 0).nonzero().flatten()] == 0)
    rs = pool[ids[real].long()].clone()
    rout = O.causal_conv1d_update(x[real, :, 0], rs, w, b, activation="silu")
    assert_close(out[real], rout, dtype)
    assert_equal(st[ids[real].long()], rs)
    untouched = [r for r in range(P) if r not in ids.tolist()]
    assert_equal(st[untouched], pool[untouched])


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("batch", [1, 7])
def test_odd_batch_without_indices_exact_state(dtype, batch):
    """Batch entry b updates state row b; with an odd batch the last wavefront's second entry
    lies past the batch and must neither store nor read beyond the last state row (the state
    tensor here has exactly `batch` rows)."""
    D, W = 264, 4
    x, w, b, _ = make_inputs(batch, D, 1, W, dtype=dtype)
    state = make_inputs(batch, D, W - 1, W, dtype=dtype, seed=1)[0]
    sg = state.to(DEV)
    og = torch.full((batch, D, 1), float("nan"), dtype=dtype, device=DEV)
    native_update(x.to(DEV), w.to(DEV), b.to(DEV), sg, None, None, og, True)
    rs = state.clone()
    rout = O.causal_conv1d_update(x[:, :, 0], rs, w, b, activation="silu")
    assert_close(og[..., 0].cpu(), rout, dtype)
    assert_equal(sg.cpu(), rs)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_strided_inputs(dtype):
    # x as a column slice, state with padded channel stride, transposed weight
    g = torch.Generator().manual_seed(0)
    xb = torch.randn(2, 32, 3, generator=g).to(dtype)
    x = xb[:, :, 1]
    sb = torch.randn(2, 32, 8, generator=g).to(dtype)
    w = torch.randn(4, 32, generator=g).to(dtype).t()
    b = torch.randn(32, generator=g).to(dtype)
    sg = sb.to(DEV)
    out = cc.causal_conv1d_update(xb.to(DEV)[:, :, 1], sg[:, :, 2:7], torch.randn(4, 32).to(dtype).to(DEV).t()
                                  .copy_(w.to(DEV)), b.to(DEV), activation="silu").cpu()
    rs = sb.clone()
    rout = O.causal_conv1d_update(x, rs[:, :, 2:7], w, b, activation="silu")
    assert_close(out, rout, dtype)
    assert_equal(sg.cpu(), rs)


@pytest.mark.parametrize("seqlen,S,circular", [(1, 3, False), (4, 64, True)])
def test_baseline_decode_shapes_reduced(seqlen, S, circular):
    """Benchmark configuration C4 with batch 32 (full size runs in tests/test_configs_gpu.py)."""
    g = torch.Generator().manual_seed(0)
    B, D, W = 32, 5120, 4
    x = torch.randn(B, D, seqlen, generator=g).bfloat16()
    w = torch.randn(D, W, generator=g).bfloat16()
    b = torch.randn(D, generator=g).bfloat16()
    pool = torch.randn(64, D, S, generator=g).bfloat16()
    idx = torch.randperm(64, generator=g)[:B].to(torch.int32)
    kw = dict(activation="silu", conv_state_indices=idx)
    if circular:
        kw["cache_seqlens"] = torch.randint(0, 64, (B,), generator=g, dtype=torch.int32)
    out, st, rout, rst = _run(x if seqlen > 1 else x[..., 0], pool, w, b, **kw)
    assert_close(out, rout, torch.bfloat16)
    assert_equal(st, rst)
