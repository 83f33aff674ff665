"""GPU checks of the rank-r LoRA kernels around the fused MLP (libmxfp8_mlp.so: mxfp8_lora_prep, mxfp8_lora_nt,
mxfp8_lora_tn, mxfp8_mlp_bwd_finish) against float64 references with the reference's rounding points
(/root/reference/scripts/fused_mlp.py:272-277, :311-333): every product is a bf16 GEMM with fp32 accumulation
(one rounding of the sum, then one more after a scale).  The kernels sum in another fp32 order, so results may
sit one bf16 step apart where the exact sum lies near a rounding boundary; the bar is at most one bf16 step
everywhere and exact equality for at least 99% of the elements.  The bf16 casts of the weights are exact
(round to nearest even, as Tensor.to)."""
import pytest
import torch

import _native
import fused_linear
import fused_mlp

pytestmark = pytest.mark.gpu


def _bf16_step_ok(got, ref_f64, absum):
    """got: bf16-valued tensor; ref: the exact float64 value the bf16 result rounds; absum: Σ |terms| of each
    element.  Bar: within one bf16 step of bf16(ref) plus the fp32 accumulation slack 2^-20 Σ |terms| (a sum
    that cancels to a tiny value carries fp32 rounding of its large terms, in any summation order)."""
    got = got.float().cpu().double()
    ref = ref_f64.cpu()
    rounded = ref.float().to(torch.bfloat16).double()
    mag = torch.maximum(rounded.abs(), got.abs()).clamp_min(1e-30)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)
    d = (got - rounded).abs()
    assert bool((d <= ulp * 1.0001 + 2.0 ** -20 * absum.cpu()).all()), d.max().item()
    frac = (got == rounded).double().mean().item()
    assert frac >= 0.99, frac
    return frac


@pytest.mark.parametrize("R,K,N", [(16, 1024, 3584), (32, 2048, 6144)])
def test_prep_casts_and_transposes(R, K, N, gpu):
    g = torch.Generator().manual_seed(R + K)
    Ag, Au = torch.randn(R, K, generator=g), torch.randn(R, K, generator=g)
    Bg, Bu = torch.randn(N, R, generator=g), torch.randn(N, R, generator=g)
    Ad, Bd = torch.randn(R, N, generator=g), torch.randn(K, R, generator=g)
    fused_linear.new_step()
    lw = fused_mlp._prep(*(t.to(gpu) for t in (Ag, Bg, Au, Bu, Ad, Bd)), torch.bfloat16)
    b = lambda t: t.to(torch.bfloat16)  # noqa: E731
    ref = dict(S=b(torch.cat([Ag, Au])), ST=b(torch.cat([Ag, Au]).t()), bg=b(Bg), bu=b(Bu), bgT=b(Bg.t()),
               buT=b(Bu.t()), ad=b(Ad), adT=b(Ad.t()), bd=b(Bd), bdT=b(Bd.t()))
    for k, v in ref.items():
        assert torch.equal(getattr(lw, k).cpu(), v.contiguous()), k


@pytest.mark.parametrize("T,K,rp,scale", [(10752, 2048, 32, 1.0), (300, 1024, 16, 2.0), (77, 2048, 64, 0.75)])
def test_lora_nt(T, K, rp, scale, gpu):
    g = torch.Generator().manual_seed(T + rp)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(rp, K, generator=g) * 0.02).to(torch.bfloat16)
    out = torch.empty(T, rp, dtype=torch.bfloat16, device=gpu)
    tpad = -(-T // 128) * 128
    outT = torch.full((rp, tpad), 7.0, dtype=torch.bfloat16, device=gpu)
    _native.lora_nt(x.to(gpu), w.to(gpu), out, scale=scale, outT=outT)
    exact = x.double() @ w.double().t()
    absum = x.double().abs() @ w.double().abs().t()
    if scale == 1.0:
        _bf16_step_ok(out, exact, absum)
    else:
        # out = bf16(bf16(exact) * scale); with the first rounding at most one step off, compare the second
        first = exact.float().to(torch.bfloat16).double()
        _bf16_step_ok(out, first * scale, absum * abs(scale) + first.abs() * abs(scale) * 2.0 ** -7)
    assert torch.equal(outT[:, :T].cpu(), out.t().cpu()) and int(torch.count_nonzero(outT[:, T:])) == 0


@pytest.mark.parametrize("T,K,rp,scale,transpose", [(10752, 2048, 16, 2.0, True), (10752, 2048, 32, 1.0, False),
                                                    (333, 1024, 64, 1.0, False), (31, 256, 16, 1.0, True)])
def test_lora_tn(T, K, rp, scale, transpose, gpu):
    g = torch.Generator().manual_seed(T + K + rp)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16)
    p = torch.randn(T, rp, generator=g).to(torch.bfloat16)
    out = torch.empty((K, rp) if transpose else (rp, K), dtype=torch.float32, device=gpu)
    part = torch.empty(_native.lora_tn_chunks(T, K) * rp * K, dtype=torch.float32, device=gpu)
    _native.lora_tn(x.to(gpu), p.to(gpu), out, part, scale=scale, transpose=transpose)
    exact = p.double().t() @ x.double()  # [rp, K]
    absum = p.double().abs().t() @ x.double().abs()
    got = out.t() if transpose else out
    assert bool((got.cpu() == got.cpu().to(torch.bfloat16).float()).all())  # bf16 values held in fp32
    _bf16_step_ok(got if scale == 1.0 else got / scale, exact, absum)  # scale 2: exact second rounding
    # the same twice (fixed chunk order)
    out2 = torch.empty_like(out)
    _native.lora_tn(x.to(gpu), p.to(gpu), out2, part, scale=scale, transpose=transpose)
    assert torch.equal(out, out2)
    # bf16 output
    outb = torch.empty((K, rp) if transpose else (rp, K), dtype=torch.bfloat16, device=gpu)
    _native.lora_tn(x.to(gpu), p.to(gpu), outb, part, scale=scale, transpose=transpose)
    assert torch.equal(outb.float(), out)


def test_bwd_finish_matches_reference_reduction(gpu):
    g = torch.Generator().manual_seed(3)
    ncg, nsb, T, N, R, s_g, s_u = 5, 3, 300, 512, 16, 2.0, 0.5
    dxa_p = torch.randn(ncg, T, 3 * R, generator=g)
    dbg_p, dbu_p = torch.randn(nsb, N, R, generator=g), torch.randn(nsb, N, R, generator=g)
    dad_p = torch.randn(nsb, R, N, generator=g)
    dxa = torch.empty(T, 2 * R, dtype=torch.bfloat16, device=gpu)
    xsd = torch.empty(T, R, dtype=torch.bfloat16, device=gpu)
    dbg, dbu = torch.empty(N, R, device=gpu), torch.empty(N, R, device=gpu)
    dad = torch.empty(R, N, device=gpu)
    _native.mlp_bwd_finish(dxa_p.to(gpu), dbg_p.to(gpu), dbu_p.to(gpu), dad_p.to(gpu), T, N, R, s_g, s_u, dxa, xsd,
                           dbg, dbu, dad)

    def ordered(p):
        v = p[0].clone()
        for c in range(1, p.shape[0]):
            v += p[c]
        return v
    sx = ordered(dxa_p)
    ref_dxa = torch.cat([sx[:, :R] * s_g, sx[:, R:2 * R] * s_u], 1).to(torch.bfloat16)
    assert torch.equal(dxa.cpu(), ref_dxa) and torch.equal(xsd.cpu(), sx[:, 2 * R:].to(torch.bfloat16))
    assert torch.equal(dbg.cpu(), ordered(dbg_p) * s_g) and torch.equal(dbu.cpu(), ordered(dbu_p) * s_u)
    assert torch.equal(dad.cpu(), ordered(dad_p))


@pytest.mark.parametrize("T,K,rp,scale", [(300, 1024, 32, 1.0), (4096, 2048, 16, 2.0), (1, 128, 16, 1.0),
                                          (8896, 2048, 32, 1.0)])
def test_quant_lora_matches_quantizer_and_product(T, K, rp, scale, gpu):
    # one read of x: codes and scales bit-identical to mxfp8_quant_tiled; out / outT as lora_nt's contract
    import mxfp8
    from oracle import mx
    g = torch.Generator().manual_seed(T + K + rp)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(rp, K, generator=g) * 0.02).to(torch.bfloat16)
    q, s, out, outT = mxfp8.mx_quant_lora(x.to(gpu), w.to(gpu), scale=scale)
    qr, sr = mxfp8.mx_quant_tiled(x.to(gpu))
    live = lambda qq: mx.from_tiled(qq.view(torch.uint8).cpu().numpy().reshape(-1), T, K)  # noqa: E731
    import numpy as np
    assert np.array_equal(live(q), live(qr))
    assert torch.equal(s.view(torch.uint8), sr.view(torch.uint8))
    exact = x.double() @ w.double().t()
    absum = x.double().abs() @ w.double().abs().t()
    if scale != 1.0:
        exact = exact.float().to(torch.bfloat16).double() * scale
        absum = absum * scale
    _bf16_step_ok(out, exact, absum)
    tpad = -(-T // 128) * 128
    assert outT.shape == (rp, tpad) and torch.equal(outT[:, :T].t().cpu(), out.cpu())
    assert int(torch.count_nonzero(outT[:, T:])) == 0
