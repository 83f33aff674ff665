"""Pins the CPU oracle of the MX quantizer (oracle/mx_oracle.c, oracle/mx.py) against what mathematics and
independent implementations fix, since the reference ships no test vectors for this path.

- E8M0 exponent: the reference's own route (fp32 division by 448, round up to a power of two, satfinite;
  mxfp8.py:61-63) vs the integer closed form vs exact rational arithmetic, for every bf16 amax.
- E4M3 encode: the oracle's nearest-value search vs torch's float8_e4m3fn cast (an independent RNE
  implementation), for every bf16 value; decode table vs torch.
- Known-answer blocks (zero, -0, 448·2^k, RNE ties, padded rows, NaN).
- Blocked layout: index formula (mxfp8.py:74) vs torchao's reshape construction vs inverse.
- Invariants used by the weight preparation (mxfp8.py:472-484, 410-415) and the column-slice store
  (fused_mlp.py:160-162).
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import mx

ALL_BF16 = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)


def _exact_e8m0(bits):
    """clamp(ceil(log2(amax / 448)) + 127, 0, 254) in exact rational arithmetic; NaN -> 255, inf -> 254."""
    E, m = (bits >> 23) & 0xFF, bits & 0x7FFFFF
    if E == 255:
        return 255 if m else 254
    if E == 0 and m == 0:
        return 0
    if E == 0:
        amax = Fraction(m, 1 << 23) * Fraction(2) ** -126
    else:
        amax = (1 + Fraction(m, 1 << 23)) * Fraction(2) ** (E - 127)
    q = amax / 448
    c = q.numerator.bit_length() - q.denominator.bit_length()
    while Fraction(2) ** c < q:
        c += 1
    while Fraction(2) ** (c - 1) >= q:
        c -= 1
    return min(max(c + 127, 0), 254)


def test_e8m0_all_bf16_three_ways():
    bad = []
    for h in range(0, 0x8000):  # every non-negative bf16 pattern incl. subnormals, inf, NaN
        bits = h << 16
        amax = np.array([bits], np.uint32).view(np.float32)[0]
        a = mx.e8m0_ieee(amax)
        b = mx.e8m0_closed(bits)
        c = _exact_e8m0(bits)
        if not (a == b == c):
            bad.append((hex(h), a, b, c))
    assert not bad, bad[:10]


def test_e8m0_fp32_closed_form_random():
    # the closed form also holds for arbitrary fp32 amax (not only bf16-valued ones)
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 0x7F800000, size=20000, dtype=np.uint32)
    for b in bits:
        a = np.array([b], np.uint32).view(np.float32)[0]
        assert mx.e8m0_ieee(a) == mx.e8m0_closed(int(b)) == _exact_e8m0(int(b))


def test_e4m3_encode_all_bf16_vs_torch():
    v = ALL_BF16.float()
    fin = torch.isfinite(v) & (v.abs() <= 448)
    ref = v[fin].to(torch.float8_e4m3fn).view(torch.uint8)
    got = torch.tensor([mx.e4m3_rne(float(t)) for t in v[fin]], dtype=torch.uint8)
    mism = (got != ref).nonzero().flatten()
    assert mism.numel() == 0, [(float(v[fin][i]), int(got[i]), int(ref[i])) for i in mism[:10]]
    # beyond the clamp every magnitude saturates to the top code (the reference clamps to +-448 first)
    assert mx.e4m3_rne(1e6) == 0x7E and mx.e4m3_rne(-1e6) == 0xFE and mx.e4m3_rne(float("nan")) == 0x7F


def test_e4m3_encode_random_fp32_vs_torch():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(20000) * np.exp2(rng.integers(-14, 9, 20000))).astype(np.float32)
    x = np.clip(x, -448, 448)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([mx.e4m3_rne(float(t)) for t in x], np.uint8)
    assert np.array_equal(got, ref)


def test_e4m3_decode_table_vs_torch():
    lut = mx.e4m3_lut()
    ref = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(lut), nan)
    assert np.array_equal(lut[~nan], ref[~nan])


def _block(vals):
    x = torch.zeros((1, 128), dtype=torch.float32)
    x[0, :32] = torch.tensor(vals, dtype=torch.float32)
    return x.to(torch.bfloat16)


def _scale0(s):
    return int(s[mx.blocked_offset(0, 0, 1)])


@pytest.mark.parametrize("k", list(range(-20, 21)))
def test_kat_boundary_448(k):
    vals = [0.5 * 2.0 ** k] * 32
    vals[7] = 448.0 * 2.0 ** k
    vals[9] = -448.0 * 2.0 ** k
    q, s = mx.quant(_block(vals))
    assert _scale0(s) == 127 + k
    assert int(q[0, 7]) == 0x7E and int(q[0, 9]) == 0xFE
    assert int(q[0, 0]) == 0x30  # 0.5


def test_kat_table():
    # all +0.0 -> scale 0, codes 0x00; all -0.0 -> scale 0, codes 0x80
    q, s = mx.quant(_block([0.0] * 32))
    assert _scale0(s) == 0 and int(q[0, :32].max()) == 0
    q, s = mx.quant(_block([-0.0] * 32))
    assert _scale0(s) == 0 and bool((q[0, :32] == 0x80).all())
    # amax 450 -> 128 (450/448 > 1); amax 448 -> 127; amax 1.0 -> 119
    for amax, e in ((450.0, 128), (448.0, 127), (1.0, 119), (2.0 ** -120, 0), (3.0e38, 247)):
        _, s = mx.quant(_block([amax] + [0.0] * 31))
        assert _scale0(s) == e, (amax, _scale0(s), e)
    # RNE ties at scale 1 (amax 448): 17 -> 0x58, 19 -> 0x5A, 2^-10 -> 0x00, 3*2^-10 -> 0x02, -17 -> 0xD8
    q, s = mx.quant(_block([448.0, 17.0, 19.0, 2.0 ** -10, 3 * 2.0 ** -10, -17.0] + [0.0] * 26))
    assert _scale0(s) == 127
    assert [int(c) for c in q[0, :6]] == [0x7E, 0x58, 0x5A, 0x00, 0x02, 0xD8]
    # NaN block: scale 0xFF, codes 0x7F (documented choice); other blocks of the row unaffected
    x = _block([1.0] * 32).float()
    x[0, 3] = float("nan")
    x[0, 32:64] = 1.0
    q, s = mx.quant(x.to(torch.bfloat16))
    assert _scale0(s) == 255 and bool((q[0, :32] == 0x7F).all())
    assert int(s[mx.blocked_offset(0, 1, 1)]) == 119 and int(q[0, 32]) == 0x78  # 1.0 * 2^8
    # +inf: satfinite scale 254, inf -> 0x7E, finite elements scaled by 2^-127
    q, s = mx.quant(_block([float("inf"), 2.0 ** 127] + [0.0] * 30))
    assert _scale0(s) == 254 and int(q[0, 0]) == 0x7E and int(q[0, 1]) == 0x38


def test_kat_padded_rows_zero():
    x = torch.randn(130, 256).to(torch.bfloat16)
    q, s = mx.quant(x)
    assert s.numel() == 2 * 2 * 512
    for i in range(130, 256):
        for b in range(8):
            assert int(s[mx.blocked_offset(i, b, 2)]) == 0


@pytest.mark.parametrize("R,C", [(1, 128), (127, 256), (128, 128), (300, 384), (513, 1024)])
def test_blocked_layout_formula_vs_torchao(R, C):
    g = torch.Generator().manual_seed(R * 7 + C)
    sc = torch.randint(1, 255, (R, C // 32), generator=g, dtype=torch.uint8)
    flat = mx.to_blocked_torchao(sc)
    i = torch.arange(R).view(-1, 1)
    b = torch.arange(C // 32).view(1, -1)
    mine = torch.zeros_like(flat)
    mine[mx.blocked_offset(i, b, C // 128).reshape(-1)] = sc.reshape(-1)
    assert torch.equal(flat, mine)
    assert torch.equal(mx.from_blocked(flat, R, C // 32), sc)


def test_quant_scales_match_torchao_layout_of_rowwise_scales():
    x = (torch.randn(200, 512) * torch.exp2(torch.randint(-8, 8, (200, 1)).float())).to(torch.bfloat16)
    q, s = mx.quant(x)
    rowwise = torch.zeros(200, 16, dtype=torch.uint8)
    xf = x.float().view(200, 16, 32)
    for i in range(200):
        for b in range(16):
            rowwise[i, b] = mx.e8m0_ieee(float(xf[i, b].abs().max()))
    assert torch.equal(s, mx.to_blocked_torchao(rowwise))


def test_quant_error_bound_and_rceil_range():
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(256, 1024, generator=g) * torch.exp2(torch.randint(-30, 30, (256, 32), generator=g).float()
                                                           ).repeat_interleave(32, 1)).to(torch.bfloat16)
    q, s = mx.quant(x)
    d = mx.dequant(q, s, 256, 1024)
    xf = x.float()
    e = mx.from_blocked(s, 256, 32).float()
    blk = xf.view(256, 32, 32)
    amax = blk.abs().amax(-1)
    scaled_amax = amax * torch.exp2(127 - e)
    nz = amax > 0
    # RCEIL: the block maximum lands in (224, 448] after scaling
    assert bool(((scaled_amax > 224) & (scaled_amax <= 448))[nz].all())
    # RNE error bound: half a step of the E4M3 grid at the element's binade (relative 2^-4), or half the
    # subnormal step 2^-10 (absolute, in scaled units)
    step = torch.maximum(blk.abs() * 2.0 ** -4, torch.exp2(e - 127 - 10).unsqueeze(-1))
    assert bool(((d.view(256, 32, 32) - blk).abs() <= step * 1.0000001).all())


def test_quant_exact_when_representable():
    g = torch.Generator().manual_seed(9)
    codes = torch.randint(0, 0x7F, (64, 256), generator=g, dtype=torch.uint8)  # finite codes incl. subnormal
    codes[:, ::32] = 0x7E  # each block's max is 448 -> scale byte = exponent chosen below
    vals = codes.view(torch.float8_e4m3fn).float()
    sgn = torch.where(torch.rand(64, 256, generator=g) < 0.5, -1.0, 1.0)
    k = torch.randint(-40, 40, (64, 8), generator=g)
    x = (vals * sgn * torch.exp2(k.float()).repeat_interleave(32, 1)).to(torch.bfloat16)
    q, s = mx.quant(x)
    assert torch.equal(mx.from_blocked(s, 64, 8).long(), k + 127)
    assert torch.equal(mx.dequant(q, s, 64, 256), x.float())


def test_weight_prep_invariants():
    g = torch.Generator().manual_seed(3)
    N, K = 384, 256
    Wg = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    Wu = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    w, ws = mx.quant(torch.cat([Wg, Wu]))
    qg, sg = mx.quant(Wg)
    qu, su = mx.quant(Wu)
    # forward scales are ordered by tile row: the first half is gate's (mxfp8.py:480-482)
    assert torch.equal(w[:N], qg) and torch.equal(w[N:], qu)
    assert torch.equal(ws[:ws.numel() // 2], sg) and torch.equal(ws[ws.numel() // 2:], su)
    # transposed operand: a column slice of quant(W_guᵀ) with its tiles cut out equals quant(W_gateᵀ)
    # (mxfp8.py:410-415)
    wt, wts = mx.quant_t(torch.cat([Wg, Wu]))
    qgt, sgt = mx.quant_t(Wg)
    s3 = wts.view(K // 128, 2 * N // 128, 512)
    assert torch.equal(wt[:, :N], qgt)
    assert torch.equal(s3[:, :N // 128].reshape(-1), sgt)


def test_column_slice_store_matches_separate_quant():
    g = torch.Generator().manual_seed(4)
    T, N = 200, 256
    dg = torch.randn(T, N, generator=g).to(torch.bfloat16)
    du = torch.randn(T, N, generator=g).to(torch.bfloat16)
    q = torch.zeros(T, 2 * N, dtype=torch.uint8)
    s = torch.full((mx.scale_bytes(T, 2 * N),), 0xAA, dtype=torch.uint8)
    mx.quant_into(dg, q, s, 0, 2 * N // 128)
    mx.quant_into(du, q, s, N, 2 * N // 128)
    q2, s2 = mx.quant(torch.cat([dg, du], 1))
    assert torch.equal(q, q2) and torch.equal(s, s2)


def test_tiled_layout_is_the_gemm_lds_image():
    # The MX-tiled layout must hold, for each 16-row x 64-code slice, exactly the 1 KB the GEMM's row-major DMA
    # leaves in LDS: lane i of that DMA reads row i // 4 of the slice, logical 16-byte chunk
    # (i % 4) ^ ((i // 16) % 4), and lands at byte 16 i.  Checked slice by slice on a ragged shape, plus the
    # inverse and padding.
    rng = np.random.default_rng(7)
    R, K = 45, 192
    q = rng.integers(0, 256, size=(R, K), dtype=np.uint8)
    t = mx.to_tiled(q)
    Rp = 48
    assert t.size == Rp * K
    qp = np.zeros((Rp, K), np.uint8)
    qp[:R] = q
    for rg in range(Rp // 16):
        for kb in range(K // 64):
            blk = t[(rg * (K // 64) + kb) * 1024:(rg * (K // 64) + kb + 1) * 1024]
            for i in range(64):
                row = rg * 16 + i // 4
                c = (i % 4) ^ ((i // 16) % 4)
                assert np.array_equal(blk[16 * i:16 * i + 16], qp[row, kb * 64 + 16 * c:kb * 64 + 16 * c + 16])
    assert np.array_equal(mx.from_tiled(t, R, K), q)
    assert not t.reshape(Rp // 16, K // 64, 16, 64)[-1, :, R - 32:].any()  # rows 45..47 are zero padding


def test_ft_layout_matches_lane_order():
    # the fused-tile layout (gu, dhm between the GEMM and the fused kernels), built element by element from its
    # definition: in block (rb, cb), lane l = r%32 + 32*lg holds columns 16*lg + 0..15 of row r; the block
    # stores all lanes' first 8 columns (8 per lane, lane order), then all lanes' last 8
    R, C = 45, 96
    x = np.arange(R * C, dtype=np.int64).reshape(R, C) + 1
    t = mx.to_ft(x)
    Rp = 64
    want = np.zeros(Rp * C, np.int64)
    pos = 0
    for rb in range(Rp // 32):
        for cb in range(C // 32):
            for half in range(2):
                for lane in range(64):
                    r, lg = rb * 32 + lane % 32, lane // 32
                    for e in range(8):
                        c = cb * 32 + lg * 16 + half * 8 + e
                        want[pos] = x[r, c] if r < R else 0
                        pos += 1
    assert pos == Rp * C and np.array_equal(t, want)
    assert np.array_equal(mx.from_ft(t, R, C), x)
