"""CPU checks of the row order of the gate|up GEMM with the fused SwiGLU epilogue (mxfp8.fused_swiglu_rows), on
which the epilogue's register layout rests: output tile t = 128 columns holds gate columns 64t.. then up
columns 64t.., and inside every 32-row block the weight row at MFMA row a is pi_col(a), so that in the
32x32 accumulator layout (lane l, register i -> MFMA row (i/4)*8 + (l/32)*4 + i%4) each lane holds the 16
contiguous columns (l/32)*16 + 0..15 of its token."""
import torch

import mxfp8


def _pi_col(a):
    return ((a >> 2) & 1) * 16 + (a >> 3) * 4 + (a & 3)


def test_fused_rows_is_a_permutation_in_tile_halves():
    for n in (128, 640, 3584, 6144):
        p = mxfp8.fused_swiglu_rows(n)
        assert sorted(p.tolist()) == list(range(2 * n))
        for t in (0, n // 64 - 1):
            tile = p[128 * t:128 * t + 128]
            assert bool(((tile[:64] >= 64 * t) & (tile[:64] < 64 * t + 64)).all())          # gate rows
            assert bool(((tile[64:] >= n + 64 * t) & (tile[64:] < n + 64 * t + 64)).all())  # matching up rows
            assert torch.equal(tile[64:] - n, tile[:64])


def test_each_lane_holds_16_contiguous_columns():
    n, t, half, blk = 6144, 7, 1, 1
    p = mxfp8.fused_swiglu_rows(n)
    base = 128 * t + 64 * half + 32 * blk
    for lane in range(64):
        cols = [int(p[base + (i // 4) * 8 + (lane // 32) * 4 + i % 4]) for i in range(16)]
        first = half * n + 64 * t + 32 * blk + (lane // 32) * 16
        assert cols == list(range(first, first + 16)), lane
    assert [_pi_col(a) for a in range(32)] == [int(x) - (64 * t + 32 * blk) for x in p[128 * t + 32 * blk:128 * t + 32 * blk + 32]]
