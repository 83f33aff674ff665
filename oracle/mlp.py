"""CPU oracle for the MXFP8 fused SwiGLU-MLP forward/backward with LoRA.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker; the product path never imports it.

A PyTorch-CPU restatement of the reference path with every bf16 rounding point of the reference kept:
  - weight preparation   /root/reference/scripts/mxfp8.py:472-490 (W_gu along K and W_guᵀ along 2N;
                          W_down along N and W_downᵀ along K)
  - MX GEMM              torch._scaled_mm at fused_mlp.py:279, :283, :309, :329, restated as
                          dequantize -> fp32 matmul -> bf16 (RNE)
  - forward              fused_mlp.py:263-293 and the kernel math of :65-109 (_gu_tile, _fwd_kernel)
  - backward             fused_mlp.py:295-336 and the kernel math of :112-175 (_bwd_kernel)
  - LoRA bf16 products   cuBLAS bf16 GEMMs with fp32 accumulation (train.py:54 disables reduced-precision
                          reduction), restated as fp32 matmul -> bf16
fp32 summation order and transcendental ulps differ from the GPU; tests state their tolerances.

Pinned by tests/test_oracle_mlp.py without sharing this file's code: lossless MX inputs against an independent
float64 composition (stage by stage and end to end), torch.autograd and float64 central differences of the exact
MLP for every gradient, exact-zero reductions (LoRA scalings 0, LoRA B = 0), the bf16 rounding point of every
rounded backward tensor, and mutants of this file that those checks must reject.
"""
import torch

from . import mx

BF16 = torch.bfloat16


def bf(t):
    """Round to bf16 (RNE) and return as fp32, the way the kernels keep bf16-valued fp32 registers."""
    return t.to(BF16).float()


def mx_gemm(qa, sa, qb, sb, M, N, K):
    """bf16 C[M, N] = deq(A)[M, K] · deq(B)[N, K]ᵀ with fp32 accumulation (torch._scaled_mm contract)."""
    a = mx.dequant(qa, sa, M, K)
    b = mx.dequant(qb, sb, N, K)
    return (a @ b.t()).to(BF16)


def prepare_weights(Wg, Wu, Wd):
    """Frozen-weight MX preparation (mxfp8.py:472-490).  Wg, Wu: [N, K]; Wd: [K, N] (bf16)."""
    Wgu = torch.cat([Wg, Wu], 0).contiguous()  # [2N, K]
    w, ws = mx.quant(Wgu)
    wt, wts = mx.quant_t(Wgu)  # quant of W_guᵀ [K, 2N] along 2N
    dw, dws = mx.quant(Wd.contiguous())  # down forward operand, along N
    dwt, dwts = mx.quant_t(Wd)  # W_downᵀ [N, K] along K (dgrad operand)
    return dict(n=Wg.shape[0], K=Wg.shape[1], w=w, ws=ws, wt=wt, wts=wts, dw=dw, dws=dws, dwt=dwt, dwts=dwts)


def lora_cast(Ag, Bg, Au, Bu, Ad, Bd):
    """Per-step bf16 copies (fused_mlp.py:272-276)."""
    S = torch.cat([Ag.detach().to(BF16), Au.detach().to(BF16)])  # [2r, K]
    return S, Bg.detach().to(BF16), Bu.detach().to(BF16), Ad.detach().to(BF16), Bd.detach().to(BF16)


def gu_tile(gu, xs, bg, bu, s_g, s_u):
    """g, u = bf16(gu + s·(xa·Bᵀ)) with fp32 math (fused_mlp.py:65-71)."""
    N = gu.shape[1] // 2
    r = bg.shape[1]
    g = bf(gu[:, :N].float() + s_g * (xs[:, :r].float() @ bg.float().t()))
    u = bf(gu[:, N:].float() + s_u * (xs[:, r:].float() @ bu.float().t()))
    return g, u


def silu(g):
    """silu = g / (exp(-g) + 1) in fp32 (fused_mlp.py:104, :152)."""
    return g / (torch.exp(-g) + 1.0)


def forward(x2, W, S, bg, bu, ad, bd, s_g, s_u, s_d, need_out=True):
    """Forward of _MLP (fused_mlp.py:263-293).  Returns a dict with every intermediate the GPU path exposes."""
    T, K = x2.shape
    N = W["n"]
    r = ad.shape[0]
    out = {}
    xs = (x2.float() @ S.float().t()).to(BF16)  # :277
    q, sc = mx.quant(x2)  # :278
    gu = mx_gemm(q, sc, W["w"], W["ws"], T, 2 * N, K)  # :279
    out.update(xs=xs, qx=q, sx=sc, gu=gu)
    if need_out:
        g, u = gu_tile(gu, xs, bg, bu, s_g, s_u)
        h = (silu(g) * u).to(BF16)  # :104
        qh, sh = mx.quant(h)  # :106
        xsd = (h.float() @ ad.float().t()).to(BF16)  # :108-109, :214
        y0 = mx_gemm(qh, sh, W["dw"], W["dws"], T, K, N)  # :283
        y = (y0.float() + s_d * (xsd.float() @ bd.float().t())).to(BF16)  # :284 addmm_ (beta=1, alpha=s_d)
        out.update(g=g, u=u, h=h, qh=qh, sh=sh, xsd=xsd, y0=y0, y=y)
    return out


def backward(x2, xs, gu, W, S, bg, bu, ad, bd, s_g, s_u, s_d, dy2, need_x=True):
    """Backward of _MLP (fused_mlp.py:295-336) with the kernel math of _bwd_kernel (:112-175)."""
    T, K = x2.shape
    N = W["n"]
    r = ad.shape[0]
    dy2 = dy2.to(BF16)
    qd, sd = mx.quant(dy2)  # :307
    dhm = mx_gemm(qd, sd, W["dwt"], W["dwts"], T, N, K)  # :308-309
    dxd = (dy2.float() @ bd.float()).to(BF16)  # :311
    if s_d != 1:
        dxd = (dxd.float() * s_d).to(BF16)  # :312-313
    g, u = gu_tile(gu, xs, bg, bu, s_g, s_u)  # :151
    sl = silu(g)  # :152
    h = (sl * u).to(BF16)  # :153
    dh = bf(dhm.float() + dxd.float() @ ad.float())  # :155
    du = (dh * sl).to(BF16)  # :157
    sig = torch.sigmoid(g)  # :158
    dg = (((dh * u) * sig) * (g * (1.0 - sig) + 1.0)).to(BF16)  # :159
    out = dict(qd=qd, sd=sd, dhm=dhm, dxd=dxd, g=g, u=u, h=h, dh=dh, dg=dg, du=du)
    if need_x:  # :160-162 (dg into columns 0..N-1, du into N..2N-1 of one [T, 2N] buffer)
        qg, sg = mx.quant(torch.cat([dg, du], 1))
        out.update(qg=qg, sg=sg)
    dBg = dg.float().t() @ xs[:, :r].float()  # :163 [N, r]
    dBu = du.float().t() @ xs[:, r:].float()  # :164
    dAd = (h.float().t() @ dxd.float()).t().contiguous()  # :165, :175 -> [r, N]
    dxa_g = dg.float() @ bg.float()  # :166 [T, r]
    dxa_u = du.float() @ bu.float()  # :167
    xS = h.float() @ ad.float().t()  # :168 xS_down [T, r] fp32
    out.update(dxa_raw=torch.cat([dxa_g, dxa_u, xS], 1), dBg_raw=dBg.clone(), dBu_raw=dBu.clone(), dAd=dAd)
    dB_d = (dy2.float().t() @ bf(xS)).to(BF16)  # :316
    if s_d != 1:
        dB_d = (dB_d.float() * s_d).to(BF16)  # :317-318
    if s_g != 1:  # :320-322
        dxa_g = dxa_g * s_g
        dBg = dBg * s_g
    if s_u != 1:  # :323-325
        dxa_u = dxa_u * s_u
        dBu = dBu * s_u
    dxa = torch.cat([dxa_g, dxa_u], 1).to(BF16)  # :326
    dx = None
    if need_x:
        dx0 = mx_gemm(out["qg"], out["sg"], W["wt"], W["wts"], T, K, 2 * N)  # :329
        dx = (dx0.float() + dxa.float() @ S.float()).to(BF16)  # :331
        out.update(dx0=dx0)
    dA = (dxa.float().t() @ x2.float()).to(BF16)  # :333
    out.update(dxa=dxa, dx=dx, dA=dA, dA_g=dA[:r], dB_g=dBg, dA_u=dA[r:], dB_u=dBu, dA_d=dAd, dB_d=dB_d)
    return out
