"""Pins oracle/lora.py (the CPU restatement of /root/reference/scripts/mxfp8.py:89-293) against what the
arithmetic fixes, independently of the formula: B = 0 and scale = 0 reduce to a bf16 residual add; products of small
integers are exact; a known-answer element where rounding y + s·p once and then adding x differs from a single
rounding of x + y + s·p; for the backward, one-hot inputs that select single entries (a transposed operand or a
swapped role of B and xa fails them), exact integer products, and a known-answer element where rounding the product
before the scale differs from rounding after it."""
import torch

from oracle import lora


def _bf(t):
    return t.to(torch.bfloat16)


def test_zero_b_and_zero_scale_reduce_to_the_residual_add():
    g = torch.Generator().manual_seed(1)
    x, y = _bf(torch.randn(64, 256, generator=g)), _bf(torch.randn(64, 256, generator=g))
    xa, B = _bf(torch.randn(64, 16, generator=g)), _bf(torch.randn(256, 16, generator=g))
    want = (x.float() + y.float()).to(torch.bfloat16)
    assert torch.equal(lora.res_lora(x, y, xa, torch.zeros_like(B), 2.0), want)
    assert torch.equal(lora.res_lora(x, y, xa, B, 0.0), want)


def test_exact_integer_products():
    # xa, B in {-2..2}: every product and sum is an integer below 2^8, exact in bf16, fp32 and float64
    g = torch.Generator().manual_seed(2)
    xa = _bf(torch.randint(-2, 3, (32, 16), generator=g).float())
    B = _bf(torch.randint(-2, 3, (128, 16), generator=g).float())
    x = _bf(torch.randint(-8, 9, (32, 128), generator=g).float())
    y = _bf(torch.randint(-8, 9, (32, 128), generator=g).float())
    p = (xa.long() @ B.long().t())
    want = (x.long() + y.long() + 2 * p).float()
    assert (want.abs() < 256).all()
    assert torch.equal(lora.res_lora(x, y, xa, B, 2.0).float(), want)


def test_two_roundings_known_answer():
    # bf16 spacing at 1 is u = 2^-7.  y = 1, s·p = xa·B = 2^-3 · 3·2^-7 = 0.375 u, x = 2^-9 = 0.25 u:
    #   the reference rounds t = bf16(1 + 0.375 u) = 1, then bf16(x + t) = bf16(1 + 0.25 u) = 1;
    #   a single rounding of x + y + s·p = 1 + 0.625 u would give 1 + u.
    x = torch.full((1, 128), 2.0 ** -9, dtype=torch.bfloat16)
    y = torch.ones(1, 128, dtype=torch.bfloat16)
    xa = torch.zeros(1, 16, dtype=torch.bfloat16)
    xa[0, 0] = 2.0 ** -3
    B = torch.zeros(128, 16, dtype=torch.bfloat16)
    B[:, 0] = 3 * 2.0 ** -7
    out = lora.res_lora(x, y, xa, B, 1.0)
    assert (out.float() == 1.0).all(), out[0, :4]
    single = (x.double() + y.double() + xa.double() @ B.double().t()).to(torch.bfloat16)
    assert (single.float() == 1.0 + 2.0 ** -7).all()


def test_lora_bwd_one_hot_selects_entries():
    # dy = e_(t0, n0): d(xa)[t0, :] = scale · B[n0, :] and dB[n0, :] = scale · xa[t0, :], zero elsewhere
    g = torch.Generator().manual_seed(3)
    T, N, r = 40, 256, 16
    xa = _bf(torch.randn(T, r, generator=g))
    B = _bf(torch.randn(N, r, generator=g))
    dy = torch.zeros(T, N, dtype=torch.bfloat16)
    t0, n0 = 7, 200
    dy[t0, n0] = 1.0
    dxa, dB = lora.lora_bwd(dy, xa, B, 2.0)
    want_dxa = torch.zeros(T, r)
    want_dxa[t0] = 2.0 * B[n0].float()
    want_dB = torch.zeros(N, r)
    want_dB[n0] = 2.0 * xa[t0].float()
    assert torch.equal(dxa.float(), want_dxa) and dxa.dtype == torch.bfloat16
    assert torch.equal(dB, want_dB) and dB.dtype == torch.float32


def test_lora_bwd_exact_integer_products_and_zeros():
    g = torch.Generator().manual_seed(4)
    T, N, r = 48, 384, 32
    dy = _bf(torch.randint(-2, 3, (T, N), generator=g).float())
    xa = _bf(torch.randint(-2, 3, (T, r), generator=g).float())
    B = _bf(torch.randint(-1, 2, (N, r), generator=g).float())
    dxa, dB = lora.lora_bwd(dy, xa, B, 0.5)
    pd = dy.long() @ B.long()          # halves of integers below 2^7 have at most 8 significant bits: exact bf16
    pb = dy.long().t() @ xa.long()     # fp32 exact
    assert torch.equal(dB, 0.5 * pb.float())
    exact = 0.5 * pd.double()
    rep = exact.abs() < 128
    assert rep.double().mean().item() > 0.99
    assert torch.equal(dxa.double()[rep], exact[rep])
    z_dxa, z_dB = lora.lora_bwd(dy, xa, torch.zeros_like(B), 3.0)
    assert int(torch.count_nonzero(z_dxa)) == 0 and int(torch.count_nonzero(lora.lora_bwd(dy, xa, B, 0.0)[1])) == 0
    assert int(torch.count_nonzero(lora.lora_bwd(dy, torch.zeros_like(xa), B, 1.0)[1])) == 0


def test_lora_bwd_scale_before_rounding_known_answer():
    # dy row = (1, 2^-8, 0, ...), B[:2, 0] = 1: the fp32 product is 1 + 2^-8 (bf16 would round it to 1, a tie to
    # even).  The reference scales in fp32 before the one bf16 rounding: bf16(3 (1 + 2^-8)) = bf16(3.01171875)
    # = 3 + 2^-6 (spacing 2^-6 at 3); rounding before the scale would give 3 · 1 = 3.
    dy = torch.zeros(1, 128, dtype=torch.bfloat16)
    dy[0, 0], dy[0, 1] = 1.0, 2.0 ** -8
    B = torch.zeros(128, 16, dtype=torch.bfloat16)
    B[0, 0] = B[1, 0] = 1.0
    xa = torch.zeros(1, 16, dtype=torch.bfloat16)
    dxa, _ = lora.lora_bwd(dy, xa, B, 3.0)
    assert dxa[0, 0].item() == 3.0 + 2.0 ** -6
    assert (dy.float() @ B.float()).to(torch.bfloat16)[0, 0].item() * 3.0 == 3.0


def test_lora_bwd_transpose_relation():
    # dB(dy, xa) is d(xa)'s product with the roles swapped: scale · dyᵀ·xa = (scale · xaᵀ·dy)ᵀ, computed here by
    # calling the oracle on (dyᵀ, ., xa) where its "dy @ B" is dyᵀ @ xa
    g = torch.Generator().manual_seed(5)
    T, N, r = 64, 128, 16
    dy, xa = _bf(torch.randn(T, N, generator=g)), _bf(torch.randn(T, r, generator=g))
    B = _bf(torch.randn(N, r, generator=g))
    _, dB = lora.lora_bwd(dy, xa, B, 1.0)
    via_dxa, _ = lora.lora_bwd(dy.t().contiguous(), torch.zeros(N, r, dtype=torch.bfloat16), xa, 1.0)
    assert torch.equal(dB.to(torch.bfloat16), via_dxa)
