"""The unfused MLP path (/root/reference/scripts/shared_prefix.py:172-197: group_linear(gate, up) -> _SWIGLU ->
group_linear(down)) on the library's kernels: the SwiGLU kernels against float64 math, and the whole unfused MLP
against the fused one as a second, independently composed implementation (fused_mlp.py:67-68 states that the two
agree on h).  Bars: one bf16 step per rounded output with >= 99% exact; MLP outputs and gradients within the 2e-2
tolerance (normwise <= 1e-2)."""
import pytest
import torch

import fused_mlp
import mxfp8
import shared_prefix
import workloads

pytestmark = pytest.mark.gpu


def _step_ok(got, ref64, frac_min=0.99):
    """Within one bf16 step of bf16(ref64), plus an absolute 2^-100: where sigmoid(g) falls below the fp32 normal
    range (g < -87.3) the hardware reciprocal flushes it to 0, and the true values there are below 1e-30."""
    got = got.detach().float().cpu().double()
    rounded = ref64.float().to(torch.bfloat16).double()
    mag = torch.maximum(rounded.abs(), got.abs()).clamp_min(2.0 ** -126)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)
    d = (got - rounded).abs()
    bad = d > ulp * 1.0001 + 2.0 ** -100
    assert not bool(bad.any()), (got[bad][:4], rounded[bad][:4])
    frac = (got == rounded).double().mean().item()
    assert frac >= frac_min, frac


@pytest.mark.parametrize("shape", [(300, 1024), (37, 200)])  # whole blocks; a partial last block in both kernels
def test_swiglu_kernels_match_float64(gpu, shape):
    g = torch.Generator().manual_seed(0)
    G = (torch.randn(*shape, generator=g) * 3).to(torch.bfloat16)
    G[0, :8] = torch.tensor([0.0, -0.0, 88.0, -88.0, 100.0, -100.0, 1e-3, -1e-3])  # exp overflow, tiny, zero
    U = torch.randn(*shape, generator=g).to(torch.bfloat16)
    DH = (torch.randn(*shape, generator=g) * 0.1).to(torch.bfloat16)
    Gd, Ud = G.to(gpu).requires_grad_(True), U.to(gpu).requires_grad_(True)
    h = shared_prefix._SWIGLU(Gd, Ud)
    h.backward(DH.to(gpu))
    g64, u64, d64 = G.double(), U.double(), DH.double()
    sig = torch.sigmoid(g64)
    _step_ok(h, g64 * sig * u64)
    _step_ok(Ud.grad, d64 * g64 * sig)
    _step_ok(Gd.grad, d64 * u64 * sig * (g64 * (1 - sig) + 1))


def _run(mlp, x, dy):
    params = [p for p in mlp.parameters() if p.requires_grad]
    for p in params:
        p.grad = None
    xg = x.clone().requires_grad_(True)
    y = shared_prefix._mlp(mlp, xg)
    y.backward(dy)
    return y.detach(), xg.grad, [p.grad.clone() for p in params]


def _close(got, want, what):
    got, want = got.double().cpu(), want.double().cpu()
    rms = want.pow(2).mean().sqrt().item()
    nrm = ((got - want).norm() / want.norm().clamp_min(1e-30)).item()
    assert nrm <= 1e-2, (what, nrm)
    bad = (got - want).abs() > 2e-2 * (want.abs() + rms)
    assert not bool(bad.any()), (what, int(bad.sum()))


def test_unfused_mlp_matches_fused(gpu):
    model, inps = workloads.build_model(2, T=600, layers=1, device=gpu)
    mxfp8.enable_mxfp8(model)
    mlp = model.layers[0].mlp
    x, dy = inps[0]["x"].to(gpu), inps[0]["dy"].to(gpu)
    before = fused_mlp.STATS.get("mlp gộp", 0)
    yf, dxf, gf = _run(mlp, x, dy)
    assert fused_mlp.STATS.get("mlp gộp", 0) == before + 1  # the fused path ran
    fused_mlp.ENABLED[0] = False
    try:
        yu, dxu, gu = _run(mlp, x, dy)
    finally:
        fused_mlp.ENABLED[0] = True
    assert fused_mlp.STATS.get("mlp gộp", 0) == before + 1  # ... and then the unfused one
    _close(yu, yf, "y")
    assert (yu == yf).double().mean().item() >= 0.9
    _close(dxu, dxf, "dx")
    for k, (a, b) in enumerate(zip(gu, gf)):
        _close(a, b, f"lora grad {k}")
