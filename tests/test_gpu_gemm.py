"""GPU parity of the MX GEMM (libmxfp8_mlp.so mxfp8_gemm_nt via mxfp8.mx_mm) against the oracle's
dequantize -> matmul -> bf16 (the torch._scaled_mm contract, fused_mlp.py:279/283/309/329).

Tolerances: the BASELINE bar is max|Δ| / max|ref| <= 2e-2.  Both sides form the same exact products and sum
them in fp32 in different orders, so a tighter elementwise bound also holds and is asserted: one bf16 rounding
step of the reference value (2^-8 relative) plus fp32 reordering slack (1e-3 of max|ref|)."""
import pytest
import torch

import _native
import mxfp8
from oracle import mlp as omlp
from oracle import mx

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _ref_gemm_f64(qa, sa, qb, sb, M, N, K):
    a = mx.dequant(qa.view(torch.uint8).cpu(), sa.view(torch.uint8).cpu(), M, K).double()
    b = mx.dequant(qb.view(torch.uint8).cpu(), sb.view(torch.uint8).cpu(), N, K).double()
    return a @ b.t()


def _assert_close(got, ref):
    got = got.float().cpu().double()
    err = (got - ref).abs()
    scale = ref.abs().max().item()
    assert err.max().item() <= TOL * scale, (err.max().item(), scale)
    bound = ref.abs() * 2.0 ** -8 + 1e-3 * scale
    bad = (err > bound).nonzero()
    assert bad.numel() == 0, (bad[:5].tolist(), err.max().item())


@pytest.mark.parametrize("wide", [0, 4])
@pytest.mark.parametrize("M,N,K", [(256, 256, 128), (300, 384, 256), (1, 128, 128), (513, 640, 1152),
                                   (256, 7168, 1024), (1000, 1024, 3584)])
def test_gemm_random(M, N, K, wide, gpu):
    g = torch.Generator().manual_seed(M * 31 + N * 7 + K)
    a = (torch.randn(M, K, generator=g) * torch.exp2(torch.randint(-6, 6, (M, 1), generator=g).float()))
    b = torch.randn(N, K, generator=g) * 0.02
    qa, sa = mxfp8.mx_quant(a.to(torch.bfloat16).to(gpu))
    qb, sb = mxfp8.mx_quant(b.to(torch.bfloat16).to(gpu))
    c = mxfp8.mx_mm(qa, sa, qb, sb, layout=wide)
    _assert_close(c, _ref_gemm_f64(qa, sa, qb, sb, M, N, K))


def test_gemm_matches_oracle_bf16(gpu):
    # against the oracle's own fp32-accumulated bf16 result (what the fused-MLP oracle uses)
    g = torch.Generator().manual_seed(5)
    M, N, K = 384, 512, 2048
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    b = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    qa, sa = mx.quant(a)
    qb, sb = mx.quant(b)
    ref = omlp.mx_gemm(qa, sa, qb, sb, M, N, K).float()
    c = mxfp8.mx_mm(qa.view(torch.float8_e4m3fn).to(gpu), sa.to(gpu), qb.view(torch.float8_e4m3fn).to(gpu),
                    sb.to(gpu)).float().cpu()
    ulp = (ref.abs() * 2.0 ** -7).clamp_min(1e-30)
    assert ((c - ref).abs() <= ulp + 1e-3 * ref.abs().max()).all()


def test_gemm_strided_weight_half(gpu):
    # B operand as a column half of W_guᵀ [K, 2N] (row stride 2N): mx_wt's gate/up view (mxfp8.py:410-415)
    g = torch.Generator().manual_seed(9)
    T, K, N = 256, 256, 384
    w = (torch.randn(2 * N, K, generator=g) * 0.02).to(torch.bfloat16)
    dy = torch.randn(T, N, generator=g).to(torch.bfloat16).to(gpu)
    q, s, qt, st = mxfp8.quant_both(w.to(gpu))
    import types
    hold = types.SimpleNamespace(n=N, half_t=[None, None], w=q, ws=s, wt=qt, wts=st)

    class _Lin:
        pass

    lin = _Lin()
    lin._mx_gu = (hold, 1)
    qd, sd = mxfp8.mx_quant(dy)
    wt, wts = mxfp8.mx_wt(lin)
    assert wt.stride(0) == 2 * N
    dx = mxfp8.mx_mm(qd, sd, wt, wts)
    qtr, str_ = mx.quant_t(w[N:])
    _assert_close(dx, _ref_gemm_f64(qd, sd, qtr, str_, T, K, N))


@pytest.mark.parametrize("r", [16, 32, 48, 64])
def test_gemm_lora_epilogue(r, gpu):
    # C = bf16(bf16(A·Bᵀ) + alpha · P·Qᵀ): the y.addmm_(xsd, bdᵀ, alpha=s_d) of fused_mlp.py:284.  P and Q are the
    # first r columns of 64-wide buffers whose other columns hold NaN: the epilogue must read exactly r columns
    g = torch.Generator().manual_seed(r)
    M, N, K = 300, 1024, 512
    a = torch.randn(M, K, generator=g).to(torch.bfloat16).to(gpu)
    b = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(gpu)
    P = torch.randn(M, r, generator=g).to(torch.bfloat16)
    Q = (torch.randn(N, r, generator=g) * 0.5).to(torch.bfloat16)
    Pw = torch.full((M, 64), float("nan"), dtype=torch.bfloat16)
    Qw = torch.full((N, 64), float("nan"), dtype=torch.bfloat16)
    Pw[:, :r], Qw[:, :r] = P, Q
    qa, sa = mxfp8.mx_quant(a)
    qb, sb = mxfp8.mx_quant(b)
    c0 = mxfp8.mx_mm(qa, sa, qb, sb)
    c = mxfp8.mx_mm(qa, sa, qb, sb, lora=(Pw.to(gpu)[:, :r], Qw.to(gpu)[:, :r]), alpha=2.0)
    assert bool(torch.isfinite(c).all())
    ref = (c0.float().cpu() + 2.0 * (P.float() @ Q.float().t())).to(torch.bfloat16).float()
    err = (c.float().cpu() - ref).abs()
    assert (err <= ref.abs() * 2.0 ** -7 + 1e-4).all(), err.max()


def _operands(M, N, K, seed, gpu):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16).to(gpu)
    b = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(gpu)
    return mxfp8.mx_quant(a) + mxfp8.mx_quant(b)


@pytest.mark.parametrize("M,N,K", [(256, 7168, 1024), (1000, 1024, 3584), (10752, 2048, 6144)])
def test_gemm_split_tail(M, N, K, gpu):
    # 8-wave shape: tail tiles split along K (the workspace plan) against every tile run whole: the same exact
    # products summed in another fp32 order, so at most one bf16 step apart; repeated split runs are
    # bit-identical (pieces are added in part order, whatever order they finish in) and leave the counters at
    # zero; the default 4-wave shape never splits and matches the whole 8-wave run bit for bit
    import _native
    assert _native.load().mxfp8_gemm_workspace_size(M, N, K) > 0
    qa, sa, qb, sb = _operands(M, N, K, M + N + K, gpu)
    whole = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    _native.gemm_nt(qa, sa, K, qb, sb, K, M, N, K, whole, split=False, layout=_native.GEMM_WIDE)
    assert torch.equal(mxfp8.mx_mm(qa, sa, qb, sb), whole)
    c1, c2 = mxfp8.mx_mm(qa, sa, qb, sb, layout=4), mxfp8.mx_mm(qa, sa, qb, sb, layout=4)
    assert torch.equal(c1, c2)
    ws, _ = _native.gemm_workspace(M, N, K, c1.device)
    assert int(torch.count_nonzero(ws[:4096])) == 0
    w, s = whole.float(), c1.float()
    assert bool(((w - s).abs() <= w.abs() * 2.0 ** -7 + 1e-6 * w.abs().max()).all())
    if M * N <= 1 << 21:
        _assert_close(c1, _ref_gemm_f64(qa, sa, qb, sb, M, N, K))


def test_gemm_split_lora_epilogue(gpu):
    # the rank-r epilogue runs once, in the piece that finishes a split tile
    M, N, K, r = 512, 1024, 2048, 32
    qa, sa, qb, sb = _operands(M, N, K, 77, gpu)
    g = torch.Generator().manual_seed(78)
    P = torch.randn(M, r, generator=g).to(torch.bfloat16)
    Q = (torch.randn(N, r, generator=g) * 0.5).to(torch.bfloat16)
    import _native
    assert _native.load().mxfp8_gemm_workspace_size(M, N, K) > 0
    c0 = mxfp8.mx_mm(qa, sa, qb, sb, layout=4)
    c = mxfp8.mx_mm(qa, sa, qb, sb, lora=(P.to(gpu), Q.to(gpu)), alpha=2.0, layout=4)
    ref = (c0.float().cpu() + 2.0 * (P.float() @ Q.float().t())).to(torch.bfloat16).float()
    err = (c.float().cpu() - ref).abs()
    assert (err <= ref.abs() * 2.0 ** -7 + 1e-4).all(), err.max()


@pytest.mark.parametrize("M,N,K", [(300, 384, 512), (1000, 1024, 3584), (4096, 2048, 1024)])
def test_gemm_tiled_operands_bit_identical(M, N, K, gpu):
    # MX-tiled A and/or B leave the same bytes in LDS as row-major operands: identical results, bit for bit
    qa, sa, qb, sb = _operands(M, N, K, 3 * M + N, gpu)
    ref = mxfp8.mx_mm(qa, sa, qb, sb)
    ta, tb = mxfp8.tile_codes(qa), mxfp8.tile_codes(qb)
    for layout, a, b in ((1, ta, qb), (2, qa, tb), (3, ta, tb), (5, ta, qb), (6, qa, tb), (7, ta, tb)):
        c = mxfp8.mx_mm(a, sa, b, sb, layout=layout, m=M)
        if layout & 4:  # the 8-wave shape may split tail tiles along K: compare with its own whole run
            import _native
            w = torch.empty_like(c)
            _native.gemm_nt(qa, sa, K, qb, sb, K, M, N, K, w, layout=4)
            assert torch.equal(c, w), layout
        else:
            assert torch.equal(c, ref), layout
    # and with the rank-r epilogue
    g = torch.Generator().manual_seed(M)
    P = torch.randn(M, 16, generator=g).to(torch.bfloat16).to(gpu)
    Q = torch.randn(N, 16, generator=g).to(torch.bfloat16).to(gpu)
    assert torch.equal(mxfp8.mx_mm(ta, sa, tb, sb, lora=(P, Q), alpha=2.0, layout=3, m=M),
                       mxfp8.mx_mm(qa, sa, qb, sb, lora=(P, Q), alpha=2.0))


@pytest.mark.parametrize("M,N,K,r", [(300, 384, 512, 0), (1000, 1024, 3584, 16), (64, 12288, 2048, 0)])
def test_gemm_ft_output(M, N, K, r, gpu):
    # C in the fused-tile layout holds exactly the row-major result, rearranged (oracle.mx.to_ft)
    import numpy as np
    qa, sa, qb, sb = _operands(M, N, K, 5 * M + N, gpu)
    lora = None
    if r:
        g = torch.Generator().manual_seed(N)
        lora = (torch.randn(M, r, generator=g).to(torch.bfloat16).to(gpu),
                torch.randn(N, r, generator=g).to(torch.bfloat16).to(gpu))
    ref = mxfp8.mx_mm(qa, sa, qb, sb, lora=lora, alpha=2.0)
    ta, tb = mxfp8.tile_codes(qa), mxfp8.tile_codes(qb)
    for layout, a, b in ((8, qa, qb), (11, ta, tb)):
        c = mxfp8.mx_mm(a, sa, b, sb, lora=lora, alpha=2.0, layout=layout, m=M)
        assert c.shape == (mxfp8.ft_rows(M), N)
        want = mx.to_ft(ref.view(torch.uint16).cpu().numpy())
        got = c.view(torch.uint16).cpu().numpy().reshape(-1)
        # compare the elements of rows < M (the padding rows are not written)
        live = mx.from_ft(np.arange(want.size), mxfp8.ft_rows(M), N)[:M].reshape(-1)
        assert np.array_equal(got[live], want[live]), layout


@pytest.mark.parametrize("M,N,K,layout,rank", [(10752, 6144, 2048, 8, 0), (1000, 640, 384, 8, 0), (333, 2048, 1024, 0, 16),
                                               (700, 640, 384, 0, 32), (512, 1024, 256, 12, 0)])
def test_b_pi_layout_matches_row_order(M, N, K, layout, rank, gpu):
    """MXFP8_GEMM_B_PI (B rows in the pi_col order of mxfp8.fused_dgrad_rows, 16-byte stores) gives C bit for
    bit equal to the GEMM with B in row order, in the row-major and FT output layouts, with and without the rank-r
    epilogue and in the 8-wave shape."""
    g = torch.Generator().manual_seed(M + N + K)
    a = (torch.randn(M, K, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    b = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(gpu)
    perm = mxfp8.fused_dgrad_rows(N, gpu)
    qa, sa = mxfp8.mx_quant_tiled(a)
    qb, sb = mxfp8.mx_quant_tiled(b)
    qp, sp = mxfp8.mx_quant_tiled(b[perm].contiguous())
    lora = lora_p = None
    if rank:
        P = (torch.randn(M, rank, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
        Q = (torch.randn(N, rank, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
        lora = lora_p = (P, Q)  # Q stays in row order
    rows = mxfp8.ft_rows(M) if layout & 8 else M  # rows past M are not written: start both from zeros
    ref = mxfp8.mx_mm(qa, sa, qb, sb, out=torch.zeros((rows, N), dtype=torch.bfloat16, device=gpu), lora=lora,
                      alpha=0.5, layout=3 | layout, m=M)
    got = mxfp8.mx_mm(qa, sa, qp, sp, out=torch.zeros((rows, N), dtype=torch.bfloat16, device=gpu), lora=lora_p,
                      alpha=0.5, layout=3 | layout | _native.GEMM_B_PI, m=M)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_pi_order_weights_give_the_same_mlp_step(gpu):
    """The _MLP step with the down, dhm and dx GEMMs on the pi_col-ordered weight copies (fused_mlp.B_PI, the
    default) and on the row-order ones: the same products summed in the same order, stored in other pieces, so y,
    dx and every LoRA gradient are bit-identical."""
    import fused_linear
    import fused_mlp
    import workloads
    model, inps = workloads.build_model(3, T=1500, device=gpu)
    mxfp8.enable_mxfp8(model)
    mod = model.layers[0].mlp
    assert "_mx_wp_tl" in mod.down_proj.base_layer.__dict__ and hasattr(mod.gate_proj.base_layer._mx_gu[0], "wtp_tl")
    out = []
    try:
        for pi in (False, True):
            fused_mlp.B_PI[0] = pi
            fused_linear.new_step()
            for p in mod.parameters():
                p.grad = None
            x = inps[0]["x"].to(gpu).requires_grad_(True)
            y = fused_mlp.mlp(mod, x)
            y.backward(inps[0]["dy"].to(gpu))
            torch.cuda.synchronize()
            grads = {n: p.grad.detach().clone() for n, p in mod.named_parameters() if p.requires_grad}
            out.append((y.detach().clone(), x.grad.detach().clone(), grads))
    finally:
        fused_mlp.B_PI[0] = True
    (y0, dx0, g0), (y1, dx1, g1) = out
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    assert torch.equal(dx0.view(torch.int16), dx1.view(torch.int16))
    assert g0.keys() == g1.keys() and len(g0) == 6
    for n in g0:
        assert torch.equal(g0[n], g1[n]), n
