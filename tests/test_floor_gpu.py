"""The bandwidth floors bench.py times beside the decode kernels
(csrc/bench/cc1d_floor.hip) move exactly the bytes they claim: every
16-byte vector they are meant to read is read and written back with its bits
flipped, and nothing else is touched. A floor that skipped work would
understate the bound the kernels are compared with."""

from __future__ import annotations

import pytest
import torch

from bench import Floors

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _flip(t):
    """What the floors write: every dword of the tensor's bytes XOR 1."""
    v = t.contiguous().reshape(-1).view(torch.int32)
    return (v ^ 1).view(t.dtype).view(t.shape)


@pytest.fixture(scope="module")
def floors():
    return Floors()


def test_copy_floor(floors):
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (4096 * 4 + 12,), dtype=torch.int32, device=DEV)
    dst = torch.zeros_like(src)
    floors.copy(torch, src[:4096 * 4], dst[:4096 * 4])
    torch.cuda.synchronize()
    assert torch.equal(dst[:4096 * 4], src[:4096 * 4] ^ 1)
    assert torch.all(dst[4096 * 4:] == 0)


@pytest.mark.parametrize("dim", [5120, 1000 * 8])
def test_rows_floor(floors, dim):
    B, P, S = 6, 9, 3
    g = torch.Generator(device=DEV).manual_seed(0)
    x = torch.randn(B, dim, generator=g, device=DEV).bfloat16()
    out = torch.zeros_like(x)
    pool = torch.randn(P, dim, S, generator=g, device=DEV).bfloat16()
    idx = torch.tensor([4, 0, 8, 2, 7, 5], dtype=torch.int32, device=DEV)
    before = pool.clone()
    floors.rows(torch, x, out, pool, idx, S)
    torch.cuda.synchronize()
    assert torch.equal(out, _flip(x))
    for r in range(P):
        want = _flip(before[r]) if r in idx.tolist() else before[r]
        assert torch.equal(pool[r], want), f"pool row {r}"


@pytest.mark.parametrize("nchunks,gran", [(1, 1), (2, 1), (1, 4), (2, 4), (2, 8)])
def test_chunks_floor(floors, nchunks, gran):
    B, D, S, L, P = 5, 48, 64, 4, 7
    g = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn(B, D, L, generator=g, device=DEV).bfloat16()
    out = torch.zeros_like(x)
    pool = torch.randn(P, D, S, generator=g, device=DEV).bfloat16()
    idx = torch.tensor([6, 1, 3, 0, 4], dtype=torch.int32, device=DEV)
    cs = torch.tensor([0, 7, 63, -1, 20], dtype=torch.int32, device=DEV)
    before = pool.clone()
    floors.chunks(torch, x, out, pool, idx, cs, nchunks, gran)
    torch.cuda.synchronize()
    assert torch.equal(out, _flip(x))
    line_chunks = S * 2 // 16
    want = before.clone().view(P, D, line_chunks, 8)
    for b, (r, c) in enumerate(zip(idx.tolist(), cs.tolist())):
        k = c % line_chunks
        if gran == 1:
            ks = [(k + j) % line_chunks for j in range(nchunks)]
        else:  # the whole granules holding chunks k .. k + nchunks - 1
            two = gran < line_chunks and k % gran + nchunks > gran
            ks = [(k - k % gran + j) % line_chunks for j in range(2 * gran if two else gran)]
        for kk in ks:
            want[r, :, kk] = _flip(want[r, :, kk])
    assert torch.equal(pool, want.view(P, D, S))


@pytest.mark.parametrize("seg", [256, 1024, 4096])
def test_tiles_floor(floors, seg):
    rows, width = 128, 2048  # bf16 rows of 4 KB
    g = torch.Generator(device=DEV).manual_seed(2)
    x = torch.randn(rows + 3, width, generator=g, device=DEV).bfloat16()
    d = torch.randn(rows + 3, width, generator=g, device=DEV).bfloat16()
    out = torch.zeros_like(x)
    floors.tiles(torch, x[:rows], d[:rows], out[:rows], seg)
    torch.cuda.synchronize()
    want = x[:rows].view(torch.int32) ^ d[:rows].view(torch.int32) ^ 1  # bit patterns (some are NaNs)
    assert torch.equal(out[:rows].view(torch.int32), want)
    assert torch.all(out[rows:].view(torch.int16) == 0)


def test_walk_floor(floors):
    rows, width = 2048, 384  # bf16 rows of 768 bytes: 3 slices, 2 blocks of 8 runs per slice
    g = torch.Generator(device=DEV).manual_seed(3)
    x = torch.randn(rows + 5, width, generator=g, device=DEV).bfloat16()
    d = torch.randn(rows + 5, width, generator=g, device=DEV).bfloat16()
    out = torch.zeros_like(x)
    floors.walk(torch, x[:rows], d[:rows], out[:rows])
    torch.cuda.synchronize()
    want = x[:rows].view(torch.int32) ^ d[:rows].view(torch.int32) ^ 1
    assert torch.equal(out[:rows].view(torch.int32), want)
    assert torch.all(out[rows:].view(torch.int16) == 0)
