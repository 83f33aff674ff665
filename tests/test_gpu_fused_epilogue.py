"""GPU parity of the gate|up GEMM with the SwiGLU forward in its epilogue (mxfp8.swiglu_gemm ->
mxfp8_gemm_swiglu_fwd) against the separate path it replaces (the FT-output MX GEMM, then the fused forward
kernel mlp_fwd), which the oracle pins (tests/test_gpu_mlp.py): on identical operands gu, the MX codes of h and
their scales are bit-identical (same products, same epilogue arithmetic); xS_down is added over other partial
groupings (one partial per 128-column tile instead of per column group), so it is within one bf16 step."""
import pytest
import torch

import fused_linear
import fused_mlp
import mxfp8
import workloads
from oracle import mx

pytestmark = pytest.mark.gpu


def _ft_rows(t, T, C):
    return torch.from_numpy(mx.from_ft(t.view(torch.int16).cpu().reshape(-1).numpy(), T, C))


def _tiled_rows(q, T, C):
    return torch.from_numpy(mx.from_tiled(q.view(torch.uint8).cpu().reshape(-1).numpy(), T, C))


@pytest.mark.parametrize("cfg,T", [(3, 300), (2, 1000), (5, 1024), (61, 500), (62, 333), (3, None)])
def test_fused_forward_matches_separate_path(cfg, T, gpu, monkeypatch):
    extra = {61: dict(name="r32", T=1000, K=1024, N=3584, r=32, alpha=64, backward=True, layers=1),
             62: dict(name="odd128", T=700, K=384, N=640, r=16, alpha=32, backward=True, layers=1)}
    if cfg in extra:
        monkeypatch.setitem(workloads.CONFIGS, cfg, extra[cfg])
    model, inps = workloads.build_model(cfg, T=T, device=gpu)
    mxfp8.enable_mxfp8(model)
    fused_linear.new_step()
    inp, mod = inps[0], model.layers[0].mlp
    T, N, s = inp["T"], inp["N"], inp["s"]
    print(f"config {cfg} T={T} N={N} r={inp['r']}", flush=True)
    hold = mod.gate_proj.base_layer._mx_gu[0]
    g = lambda m: m.lora_A["default"].weight, lambda m: m.lora_B["default"].weight  # noqa: E731
    lw = fused_mlp._prep(g[0](mod.gate_proj), g[1](mod.gate_proj), g[0](mod.up_proj), g[1](mod.up_proj),
                         g[0](mod.down_proj), g[1](mod.down_proj), torch.bfloat16)
    x = inp["x"].to(gpu)
    if 2 * inp["r"] <= 32:
        q, sc, xs, _ = mxfp8.mx_quant_lora(x, lw.S, out_t=False)
    else:
        import _native
        xs = torch.empty((T, 2 * inp["r"]), dtype=torch.bfloat16, device=gpu)
        _native.lora_nt(x, lw.S, xs)
        q, sc = mxfp8.mx_quant_tiled(x)
    gu0 = mxfp8.mx_mm(q, sc, hold.w_tl, hold.ws, layout=fused_mlp._LAYOUT_FT, m=T)
    qh0, sh0, xsd0 = fused_mlp.mlp_fwd(gu0, xs, lw.bg, lw.bu, lw.ad, s, s, True, tiled=True, gu_ft=True)
    gu1, qh1, sh1, part = mxfp8.swiglu_gemm(q, sc, hold, xs, lw.bg, lw.bu, lw.ad, s, s, T)
    xsd1 = part.sum(0).to(torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(_ft_rows(gu1, T, 2 * N), _ft_rows(gu0, T, 2 * N)), "gu"
    assert torch.equal(_tiled_rows(qh1, T, N), _tiled_rows(qh0, T, N)), "codes of h"
    assert torch.equal(sh1.view(torch.uint8), sh0.view(torch.uint8)), "scales of h (padded rows 0)"
    a, b = xsd1.float().cpu(), xsd0.float().cpu()
    d = (a - b).abs()
    ulp = torch.exp2(torch.floor(torch.log2(torch.maximum(a.abs(), b.abs()).clamp_min(2.0 ** -126))) - 7)
    assert bool((d <= ulp).all()), d.max().item()
