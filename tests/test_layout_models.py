"""CPU models of the kernels' data layouts (the reference's fake-backend technique,
kernels/gemm/qgemm_test.go:122,225: model the contract of code the test machine cannot run and check its
layout plumbing everywhere; the kernels themselves are tested on the GPU).

Each model follows the index arithmetic of one kernel and checks a property that kernel relies on:
- gemm_mfma.hpp: the LDS chunk swizzle of the DMA ring pairs the same 16-byte k chunk of A and B in every
  MFMA fragment, and the 16 rows a ds_read_b128 phase reads fall on 16 distinct 16-byte bank groups;
- gemv_bf16.hip reduce_store: the reduce-scatter butterfly gives every sum bit-identical to a full butterfly,
  and exactly one store lane holds each sum;
- gemv_bf16.hip gemv_dma_kernel: the staged x blocks meet the weight bytes of the same k in the FMAs.
"""
import numpy as np
import pytest

LANES = np.arange(64)


def swz(r):
    return (r >> 1) & 7


def dma_ring_tile(rows):
    """Which global 16-byte chunk of its 128-byte k-tile row each LDS position holds after the DMA of
    gemm_kernel: one instruction covers rows R..R+7; lane l writes position l % 8 of row R + l // 8 and fetches
    chunk (l % 8) ^ swz(R + l // 8)."""
    lds = np.full((rows, 8), -1)
    for base in range(0, rows, 8):
        for lane in LANES:
            r, p = base + lane // 8, lane % 8
            lds[r, p] = p ^ swz(r)
    return lds


@pytest.mark.parametrize("bm", [32, 64, 128, 192, 256])
def test_gemm_swizzle_pairs_k_chunks(bm):
    """Fragment read of half s, MFMA row block i, wave row offset wm·WM: lane (fr = lane % 16, fg = lane // 16)
    reads LDS position ((s·4 + fg) ^ swz(fr)) of row wm·WM + 16i + fr and must find k chunk s·4 + fg of that row,
    for A and B alike, so both operands of an MFMA carry the same k."""
    lds = dma_ring_tile(bm)
    assert (lds >= 0).all() and all(sorted(lds[r]) == list(range(8)) for r in range(bm))
    for wm_off in range(0, bm, 16):
        for s in range(2):
            for lane in LANES:
                fr, fg = lane % 16, lane // 16
                row = wm_off + fr
                assert lds[row, (s * 4 + fg) ^ swz(fr)] == s * 4 + fg


@pytest.mark.parametrize("bm", [32, 128, 256])
def test_gemm_swizzle_spreads_banks(bm):
    """The 16 lanes of one ds_read_b128 phase (same fg, rows fr = 0..15 of a 16-row block) read 16 distinct
    16-byte bank groups of the 256-byte bank line (LDS rows are 128 bytes, unpadded)."""
    for base in range(0, bm, 16):
        for s in range(2):
            for fg in range(4):
                groups = {((base + fr) * 128 + (((s * 4 + fg) ^ swz(fr)) << 4)) // 16 % 16 for fr in range(16)}
                assert len(groups) == 16


def full_butterfly(col):
    """One sum over 64 lanes: u += u[lane ^ off] for off = 32 .. 1, in float32."""
    u = col.astype(np.float32).copy()
    for off in (32, 16, 8, 4, 2, 1):
        u = (u + u[LANES ^ off]).astype(np.float32)
    assert (u == u[0]).all() or np.isnan(u).all()
    return u[0]


def reduce_scatter(acc):
    """gemv_bf16.hip reduce_store for V = R·MM sums: while a lane holds more than one sum, each step at lane
    distance off halves them (the lane keeps the upper half if its bit off is set, else the lower half, and adds
    its partner's copy of that half); then full steps. Returns the per-lane values and sum index j."""
    v = acc.astype(np.float32).copy()
    V = v.shape[1]
    j = np.zeros(64, np.int64)
    c = V
    for off in (32, 16, 8, 4, 2, 1):
        if c > 1:
            up = (LANES & off) != 0
            c //= 2
            new = v.copy()
            for i in range(c):
                keep = np.where(up, v[:, i + c], v[:, i])
                give = np.where(up, v[:, i], v[:, i + c])
                new[:, i] = (keep + give[LANES ^ off]).astype(np.float32)
            v = new
            j = 2 * j + up
        else:
            v[:, 0] = (v[:, 0] + v[LANES ^ off, 0]).astype(np.float32)
    return v[:, 0], j


@pytest.mark.parametrize("V", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("seed", range(4))
def test_gemv_reduce_scatter_is_a_full_butterfly(V, seed):
    """Every sum the reduce-scatter forms is bit-identical to the full butterfly of its 64 lane partials, and
    the store lanes (lane & (64 / V − 1) == 0) hold each sum exactly once."""
    rng = np.random.default_rng(seed * 31 + V)
    acc = (rng.normal(0, 1, (64, V)) * rng.choice([1e-3, 1.0, 1e3], (64, V))).astype(np.float32)
    got, j = reduce_scatter(acc)
    splits = V.bit_length() - 1
    store = (LANES & ((64 >> splits) - 1)) == 0
    assert sorted(j[store]) == list(range(V))
    for lane in LANES[store]:
        assert got[lane].tobytes() == full_butterfly(acc[:, j[lane]]).tobytes(), f"V={V} sum {j[lane]}"


@pytest.mark.parametrize("mm,chunks,k", [(1, 4, 2048), (4, 4, 2044), (8, 4, 1536), (4, 11, 5632)])
def test_dma_gemv_x_blocks_meet_weight_k(mm, chunks, k):
    """gemv_dma_kernel: x block (m, c, h) holds x[m][512c + 8l + 4h .. +3] in lane l's 16 bytes (zero for k
    past K); lane l's 16 weight bytes of unit chunk c are the 8 bf16 at k = 512c + 8l .. +7, the FMA pairs
    x element e (block h = e / 4, element e % 4) with weight element e (low half of dword e / 2 for even e).
    Summing those products over lanes and chunks gives x·w exactly (float64, integer-valued data)."""
    rng = np.random.default_rng(mm * 100 + chunks)
    kp = chunks * 512
    x = rng.integers(-8, 9, (mm, k)).astype(np.float64)
    w = rng.integers(-8, 9, (3, k)).astype(np.float64)
    wpad = np.zeros((3, kp))
    wpad[:, :k] = w
    blocks = np.zeros((mm, chunks, 2, 64, 4))
    for m in range(mm):
        for c in range(chunks):
            for h in range(2):
                for lane in LANES:
                    kk = c * 512 + lane * 8 + h * 4
                    if kk + 4 <= k:
                        blocks[m, c, h, lane] = x[m, kk:kk + 4]
    acc = np.zeros((3, mm, 64))
    for row in range(3):
        for c in range(chunks):
            for lane in LANES:
                wl = wpad[row, c * 512 + lane * 8:c * 512 + lane * 8 + 8]
                for e in range(8):
                    acc[row, :, lane] += blocks[:, c, e >> 2, lane, e & 3] * wl[e]
    assert np.array_equal(acc.sum(axis=2), w @ x.T)
