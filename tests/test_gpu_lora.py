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


@pytest.mark.parametrize("T,K,rp,scale", [(10752, 2048, 32, 1.0), (300, 1024, 16, 2.0), (77, 2048, 64, 0.75),
                                          (45, 384, 64, 1.0), (130, 192, 16, 2.0)])
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
                                                    (333, 1024, 64, 1.0, False), (31, 256, 16, 1.0, True),
                                                    (49200, 2048, 32, 1.0, False)])  # > 192 MB: one step in flight
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
                                          (8896, 2048, 32, 1.0), (520, 1280, 32, 1.0), (130, 3072, 16, 2.0),
                                          (1100, 2048, 64, 1.0), (130, 3072, 64, 2.0), (1, 128, 64, 1.0),
                                          (260, 256, 32, 1.0), (129, 384, 16, 2.0)])
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


@pytest.mark.parametrize("T,K,rp", [(300, 256, 32), (129, 2048, 16), (77, 384, 64)])
def test_quant_lora_special_blocks(T, K, rp, gpu):
    """Codes and scale bytes of blocks that are zero, -0, inf, NaN, at the E4M3 saturation boundary (448 * 2^k) or
    huge, at rows of every 32-row block of a scale tile and in the first and last K steps (the scale words leave one
    step late, the last ones after the loop): byte for byte mxfp8_quant_tiled's."""
    import numpy as np
    import mxfp8
    from oracle import mx
    g = torch.Generator().manual_seed(T * K + rp)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16)
    xi = x.view(torch.int16)
    for row, col in ((0, 0), (33, K - 32), (66, 32), (T - 1, K - 64)):
        row = min(row, T - 1)
        xi[row, col:col + 32] = 0
    xi[min(5, T - 1), K - 96:K - 64] = -32768  # -0.0
    xi[min(40, T - 1), 64:96] = 0x7F80  # +inf
    xi[min(70, T - 1), K - 32:K] = 0x7FC0  # NaN
    xi[min(100, T - 1), 0:32] = -128  # -inf (0xFF80)
    x[min(9, T - 1), 96:128] = 448.0 * 2.0 ** -7
    x[min(10, T - 1), K - 128:K - 96] = torch.randn(32, generator=g).to(torch.bfloat16) * 3e38
    w = (torch.randn(rp, K, generator=g) * 0.02).to(torch.bfloat16)
    q, s, _, _ = mxfp8.mx_quant_lora(x.to(gpu), w.to(gpu))
    qr, sr = mxfp8.mx_quant_tiled(x.to(gpu))
    live = lambda qq: mx.from_tiled(qq.view(torch.uint8).cpu().numpy().reshape(-1), T, K)  # noqa: E731
    assert np.array_equal(live(q), live(qr))
    assert torch.equal(s.view(torch.uint8), sr.view(torch.uint8))


@pytest.mark.parametrize("T,N,r,scale", [(300, 2048, 16, 2.0), (4096, 1024, 32, 0.5), (1, 128, 16, 1.0),
                                         (10752, 2048, 16, 2.0)])
def test_res_lora_matches_oracle(T, N, r, scale, gpu):
    # out = bf16(x + bf16(y + scale · xa·Bᵀ)) (mxfp8.py:265-293): the GPU sums the r products in the MFMA's order,
    # so an element may sit one bf16 step from the oracle where y + scale·p lies near a rounding boundary
    import mxfp8
    from oracle import lora
    g = torch.Generator().manual_seed(T + N + r)
    x = torch.randn(T, N, generator=g).to(torch.bfloat16)
    y = torch.randn(T, N, generator=g).to(torch.bfloat16)
    xa_full = torch.randn(T, r + 8, generator=g).to(torch.bfloat16)  # a column slice: row stride r + 8
    xa = xa_full[:, 4:4 + r]
    B = (torch.randn(N, r, generator=g) * 0.1).to(torch.bfloat16)
    want = lora.res_lora(x, y, xa, B, scale)
    xa_d = xa_full.to(gpu)[:, 4:4 + r]
    got = mxfp8.res_lora(x.to(gpu), y.to(gpu), xa_d, B.to(gpu), scale).cpu()
    # the intermediate t = bf16(y + scale·p) may land on a bf16 neighbour of the oracle's; the result must be the
    # second rounding bf16(x + t) of one of those three values (under cancellation one step of t can exceed one
    # step of the output), and equal the oracle's almost everywhere
    t = (y.float() + scale * (xa.double() @ B.double().t()).float()).to(torch.bfloat16)
    bits = t.view(torch.int16)
    cands = [(x.float() + (bits + k).view(torch.bfloat16).float()).to(torch.bfloat16) for k in (-1, 0, 1)]
    ok = (got == cands[0]) | (got == cands[1]) | (got == cands[2])
    assert bool(ok.all()), (got[~ok][:4], want[~ok][:4])
    assert torch.equal(cands[1], want)
    assert (got == want).double().mean().item() >= 0.99


@pytest.mark.parametrize("T,N,r,off,mode", [(300, 1024, 16, 1, "both"), (1, 128, 16, 0, "both"),
                                            (4096, 2048, 32, 2, "both"), (777, 384, 16, 0, "quant"),
                                            (2000, 512, 32, 0, "lora"), (10752, 4096, 16, 0, "both"),
                                            (1500, 128, 32, 3, "both")])
def test_lora_bwd_matches_oracle(T, N, r, off, mode, gpu):
    # one read of dy (mxfp8.py:202-262): codes and scales at column tile `off` of a wider q, byte for byte the
    # oracle quantizer's; d(xa) within one bf16 step of the oracle (the GPU adds the N products in another fp32
    # order); dB within fp32 summation slack; other columns of q / s / the d(xa) destination untouched
    import mxfp8
    from oracle import lora, mx
    g = torch.Generator().manual_seed(T + N + r + off)
    dy = torch.randn(T, N, generator=g).to(torch.bfloat16)
    xS = torch.randn(T, 3 * r, generator=g).to(torch.bfloat16)  # xa = the middle r columns (row stride 3r)
    B = (torch.randn(N, r, generator=g) * 0.05).to(torch.bfloat16)
    scale = 0.5
    do_q, has_lora = mode != "lora", mode != "quant"
    width = (off + N // 128 + 1) * 128
    q = torch.zeros(T, width, dtype=torch.uint8, device=gpu) if do_q else None
    s = torch.zeros(mxfp8.scale_numel(T, width), dtype=torch.uint8, device=gpu) if do_q else None
    xS_d = xS.to(gpu)
    dS = torch.zeros(T, 2 * r, dtype=torch.bfloat16, device=gpu)
    db = mxfp8.lora_bwd(dy.to(gpu), xS_d[:, r:2 * r] if has_lora else None, B.to(gpu) if has_lora else None,
                        scale, q, s, off, dS[:, r:] if has_lora else None)
    if do_q:
        qr = torch.zeros(T, width, dtype=torch.uint8)
        sr = torch.zeros(mx.scale_bytes(T, width), dtype=torch.uint8)
        mx.quant_into(dy, qr, sr, off * 128, width // 128)
        assert torch.equal(q.cpu(), qr) and torch.equal(s.cpu(), sr)
    if not has_lora:
        assert db is None
        return
    want_dxa, want_db = lora.lora_bwd(dy, xS[:, r:2 * r], B, scale)
    got = dS.cpu()
    assert int(torch.count_nonzero(got[:, :r])) == 0
    exact = scale * (dy.double() @ B.double())
    absum = scale * (dy.double().abs() @ B.double().abs())
    _bf16_step_ok(got[:, r:], exact, absum)
    assert (got[:, r:] == want_dxa).double().mean().item() >= 0.99
    absum_b = scale * (dy.double().abs().t() @ xS[:, r:2 * r].double().abs())
    d = (db.cpu().double() - want_db.double()).abs()
    assert bool((d <= 2.0 ** -16 * absum_b + 1e-30).all()), (d / absum_b.clamp_min(1e-30)).max().item()
    db2 = mxfp8.lora_bwd(dy.to(gpu), xS_d[:, r:2 * r], B.to(gpu), scale, None, None, 0, dS[:, r:])
    assert torch.equal(db2, db)  # deterministic: fixed-order partial sums


def test_lora_bwd_quant_matches_mx_quant(gpu):
    # quantization alone into a q of the same width: the bytes of mxfp8.mx_quant(dy)
    import mxfp8
    g = torch.Generator().manual_seed(9)
    dy = (torch.randn(1000, 768, generator=g) * 3).to(torch.bfloat16).to(gpu)
    q = torch.empty(1000, 768, dtype=mxfp8.F8, device=gpu)
    s = torch.empty(mxfp8.scale_numel(1000, 768), dtype=torch.uint8, device=gpu)
    assert mxfp8.lora_bwd(dy, q=q, s=s) is None
    qr, sr = mxfp8.mx_quant(dy)
    assert torch.equal(q.view(torch.uint8), qr.view(torch.uint8)) and torch.equal(s, sr.view(torch.uint8))


@pytest.mark.parametrize("mode", ["both", "quant"])
def test_lora_bwd_codes_on_edge_blocks(mode, gpu):
    # configuration 5's upstream gradient (Student-t with x100 channels, +-0 blocks, 448·2^k maxima, RNE ties)
    # plus NaN and inf blocks: codes and scale words byte for byte the oracle's, at a column-tile offset
    import mxfp8
    import workloads
    from oracle import mx
    dy = workloads.make_inputs(5, T=700, x=False)["dy"].clone()  # [700, 2048]
    dy[5, 64:96] = float("nan")
    dy[6, 128:160] = float("inf")
    dy[7, 0:32] = -float("inf")
    dy[699, 2016:2048] = float("nan")
    T, N, off = dy.shape[0], dy.shape[1], 1
    width = (off + N // 128) * 128
    q = torch.zeros(T, width, dtype=torch.uint8, device=gpu)
    s = torch.zeros(mxfp8.scale_numel(T, width), dtype=torch.uint8, device=gpu)
    g = torch.Generator().manual_seed(3)
    xa = torch.randn(T, 16, generator=g).to(torch.bfloat16).to(gpu) if mode == "both" else None
    B = (torch.randn(N, 16, generator=g) * 0.05).to(torch.bfloat16).to(gpu) if mode == "both" else None
    dxa = torch.empty(T, 16, dtype=torch.bfloat16, device=gpu) if mode == "both" else None
    mxfp8.lora_bwd(dy.to(gpu), xa, B, 1.0, q, s, off, dxa)
    qr = torch.zeros(T, width, dtype=torch.uint8)
    sr = torch.zeros(mx.scale_bytes(T, width), dtype=torch.uint8)
    mx.quant_into(dy, qr, sr, off * 128, width // 128)
    assert torch.equal(s.cpu(), sr)
    assert torch.equal(q.cpu(), qr)


def test_pack_bf16_matches_torch(gpu):
    """mxfp8_pack_bf16 against torch: fp32 and bf16 sources (row-strided views too), straight and transposed
    destinations, zero fills, and more jobs than one launch's table takes (two launches)."""
    g = torch.Generator().manual_seed(3)
    srcs = [(torch.randn(48, 256, generator=g) * 3).to(gpu),
            torch.randn(16, 2048, generator=g).to(torch.bfloat16).to(gpu),
            torch.randn(64, 96, generator=g).to(gpu)[:, 16:80],   # row stride 96
            (torch.randn(3072, 16, generator=g) * 1e-3).to(gpu)]
    srcs[0][0, :4] = torch.tensor([float("inf"), -float("inf"), 65504.0, 1e-40])
    jobs, want = [], []
    for k in range(12):  # 12 x 3 = 36 jobs
        src = srcs[k % len(srcs)]
        r, c = src.shape
        straight = torch.full((r, c + 8), 7.0, dtype=torch.bfloat16, device=gpu)[:, :c]
        trans = torch.full((c, r + 8), 7.0, dtype=torch.bfloat16, device=gpu)[:, :r]
        zero = torch.full((r, c), 7.0, dtype=torch.bfloat16, device=gpu)
        jobs += [(src, straight, False), (src, trans, True), (None, zero, False)]
        want += [(straight, src.to(torch.bfloat16)), (trans, src.to(torch.bfloat16).t()), (zero, torch.zeros_like(zero))]
    _native.pack_bf16(jobs)
    torch.cuda.synchronize()
    for got, ref in want:
        assert torch.equal(got.view(torch.int16), ref.contiguous().view(torch.int16))


@pytest.mark.parametrize("T,Ns,R,with_q", [(1000, (2048, 512, 512), 16, True), (300, (128, 256), 32, True),
                                           (777, (512, 384, 128), 16, False)])
def test_lora_bwd_batch_matches_per_layer(T, Ns, R, with_q, gpu):
    """mxfp8_lora_bwd_batch (the layers of a group in one launch) against mxfp8_lora_bwd per layer: codes, scales
    and d(xa) bit-identical (same products, same column-chunk order), dB within fp32 rounding (other row chunks)."""
    import mxfp8
    g = torch.Generator().manual_seed(T + sum(Ns) + R)
    dys = [(torch.randn(T, n, generator=g) * 0.1).to(torch.bfloat16).to(gpu) for n in Ns]
    xas = [(torch.randn(T, R, generator=g)).to(torch.bfloat16).to(gpu) for _ in Ns]
    Bs = [(torch.randn(n, R, generator=g) * 0.05).to(torch.bfloat16).to(gpu) for n in Ns]
    scales = [2.0, 0.5, 1.0][:len(Ns)]
    n_tot = sum(Ns)
    offs = [sum(Ns[:k]) // 128 for k in range(len(Ns))]
    out = []
    for batched in (False, True):
        q = torch.full((T, n_tot), 0x55, dtype=torch.uint8, device=gpu).view(mxfp8.F8) if with_q else None
        s = torch.full((mxfp8.scale_numel(T, n_tot),), 0x55, dtype=torch.uint8, device=gpu) if with_q else None
        dxas = [torch.full((T, R), 3.0, dtype=torch.bfloat16, device=gpu) for _ in Ns]
        if batched:
            dbs = mxfp8.lora_bwd_batch(dys, xas, Bs, scales, dxas, q=q, s=s, col_tile_offs=offs)
        else:
            dbs = [mxfp8.lora_bwd(dy, xa, B, sc, q=q, s=s, col_tile_off=off, dxa_out=dxa)
                   for dy, xa, B, sc, dxa, off in zip(dys, xas, Bs, scales, dxas, offs)]
        torch.cuda.synchronize()
        out.append((q, s, dxas, dbs))
    (q0, s0, dx0, db0), (q1, s1, dx1, db1) = out
    if with_q:
        assert torch.equal(q0.view(torch.uint8), q1.view(torch.uint8)) and torch.equal(s0, s1)
    for a, b in zip(dx0, dx1):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    for a, b in zip(db0, db1):
        err = ((a.double() - b.double()).abs().max() / b.double().abs().max()).item()
        assert err <= 1e-5, err


@pytest.mark.parametrize("T,K,rp,C,scale", [(10752, 2048, 16, 32, 2.0), (300, 1024, 32, 64, 1.0), (1, 128, 16, 16, 1.0),
                                            (129, 256, 64, 32, 0.5), (8896, 2048, 16, 32, 2.0)])
def test_quant_lora_tp_matches_separate_launches(T, K, rp, C, scale, gpu):
    """mxfp8_quant_lora_tp (the quantizer, its rank-rp product and the zero-padded transpose of another [T, C] tensor
    from one launch) against mxfp8_quant_lora and mxfp8_transpose_pad run apart: every output byte identical."""
    import numpy as np

    import mxfp8
    from oracle import mx
    g = torch.Generator().manual_seed(T + K + rp + C)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16).to(gpu)
    w = (torch.randn(rp, K, generator=g) * 0.02).to(torch.bfloat16).to(gpu)
    tx = torch.randn(T, C, generator=g).to(torch.bfloat16).to(gpu)
    q, s, out, outT = mxfp8.mx_quant_lora(x, w, scale=scale)
    tpad = -(-T // 128) * 128
    txT = torch.empty((C, tpad), dtype=torch.bfloat16, device=gpu)
    _native.transpose_pad(tx, txT)
    q2, s2, out2, outT2, txT2 = mxfp8.mx_quant_lora_tp(x, w, tx, scale=scale)
    live = lambda qq: mx.from_tiled(qq.view(torch.uint8).cpu().numpy().reshape(-1), T, K)  # noqa: E731
    assert np.array_equal(live(q), live(q2))
    assert torch.equal(s.view(torch.uint8), s2.view(torch.uint8))
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))
    assert torch.equal(outT.view(torch.int16), outT2.view(torch.int16))
    assert torch.equal(txT.view(torch.int16), txT2.view(torch.int16))
    assert torch.equal(txT2[:, :T].t(), tx) and int(torch.count_nonzero(txT2[:, T:])) == 0


@pytest.mark.parametrize("T,K", [(10752, 2048), (300, 1024), (1, 128), (8896, 2048)])
def test_lora_tn_batch_matches_single_calls(T, K, gpu):
    """mxfp8_lora_tn_batch (the backward's dB_d and dA reductions in one launch, their chunk sums in one more)
    against two mxfp8_lora_tn calls with the same chunking: bit-identical outputs, fp32 and bf16 holders, both
    orientations, a scale and none."""
    g = torch.Generator().manual_seed(T + K)
    x0 = torch.randn(T, K, generator=g).to(torch.bfloat16).to(gpu)
    p0 = (torch.randn(T, 16, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    x1 = torch.randn(T, K, generator=g).to(torch.bfloat16).to(gpu)
    p1 = (torch.randn(T, 32, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    chunks = _native.lora_tn_chunks(T, K)
    for dt0, dt1 in ((torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32)):
        a0 = torch.empty((K, 16), dtype=dt0, device=gpu)
        a1 = torch.empty((32, K), dtype=dt1, device=gpu)
        _native.lora_tn(x0, p0, a0, torch.empty(chunks * 16 * K, device=gpu), scale=2.0, transpose=True)
        _native.lora_tn(x1, p1, a1, torch.empty(chunks * 32 * K, device=gpu), scale=1.0, transpose=False)
        b0 = torch.empty_like(a0)
        b1 = torch.empty_like(a1)
        _native.lora_tn_batch([(x0, p0, b0, 2.0, True), (x1, p1, b1, 1.0, False)],
                              torch.empty(chunks * 48 * K, device=gpu))
        torch.cuda.synchronize()
        assert torch.equal(a0, b0) and torch.equal(a1, b1), (dt0, dt1)


@pytest.mark.parametrize("T,K", [(10752, 2048), (300, 1024), (1, 128), (50000, 2048)])
def test_lora_tn_batch_rank_64_matches_single_calls(T, K, gpu):
    """mxfp8_lora_tn_batch with a rank-64 job (the grouped linears' dA at q|k|v, whose dS is padded to 64 columns)
    beside ranks 16 and 32, against mxfp8_lora_tn per job with the same chunking: bit-identical outputs.  At
    T = 50000 each x holds 205 MB, past the size that takes the two-step register ring."""
    g = torch.Generator().manual_seed(T + K + 64)
    rps = (64, 16, 32)
    xs = [torch.randn(T, K, generator=g).to(torch.bfloat16).to(gpu) for _ in rps]
    ps = [(torch.randn(T, rp, generator=g) * 0.1).to(torch.bfloat16).to(gpu) for rp in rps]
    chunks = _native.lora_tn_chunks(T, K)
    want, got = [], []
    for j, (x, p, rp) in enumerate(zip(xs, ps, rps)):
        shape = (K, rp) if j == 1 else (rp, K)
        want.append(torch.empty(shape, dtype=torch.float32, device=gpu))
        got.append(torch.full(shape, float("nan"), dtype=torch.float32, device=gpu))
        _native.lora_tn(x, p, want[j], torch.empty(chunks * rp * K, device=gpu), scale=2.0 if j == 1 else 1.0,
                        transpose=j == 1)
    _native.lora_tn_batch([(x, p, o, 2.0 if j == 1 else 1.0, j == 1) for j, (x, p, o) in enumerate(zip(xs, ps, got))],
                          torch.full((chunks * sum(rps) * K,), float("nan"), device=gpu))
    torch.cuda.synchronize()
    for j, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), j
