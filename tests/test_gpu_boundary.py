"""GPU checks of the drop-in boundary around the fused MLP and the generic MX linear.

  - _MLP.backward returns the reference's values and shapes (/root/reference/scripts/fused_mlp.py:306-336: dx in
    x.dtype; dA_g / dA_u / dB_d bf16 values from bf16 GEMMs, held in the adapter parameter's dtype, which is what
    autograd casts the reference's bf16 returns to; dB_g / dB_u / dA_d fp32 partial sums);
  - the saved set is the reference's eight tensors; backward finds the transposed LoRA forms through the
    per-step cast cache and rebuilds them when the cache was cleared or the saved tensors come back as other
    objects (non-reentrant checkpointing): the gradients are bit-identical in every case;
  - enable_mxfp8 -> disable_mxfp8 restores the bf16 weights bit for bit and the class forward
    (/root/reference/scripts/mxfp8.py:452-509);
  - the generic MX linear that enable_mxfp8 installs (_forward -> _quant_act -> _MXLinear,
    /root/reference/scripts/mxfp8.py:296-341): forward against the oracle's dequantize -> matmul -> bf16,
    backward dx = MX(dy) · W against the same, and the activation-reuse rule of _quant_act.
Bars as in tests/test_gpu_gemm.py: one bf16 rounding step of the reference plus 1e-3 of max|ref| elementwise."""
import pytest
import torch
import torch.utils.checkpoint

import fused_linear
import fused_mlp
import mxfp8
import workloads
from oracle import mlp as omlp
from oracle import mx

pytestmark = pytest.mark.gpu


def _assert_gemm_close(got, ref):
    got, ref = got.float().cpu().double(), ref.double()
    err = (got - ref).abs()
    scale = ref.abs().max().item()
    bound = ref.abs() * 2.0 ** -8 + 1e-3 * scale
    assert (err <= bound).all(), (err.max().item(), scale)


def _mlp_run(gpu, T=256, clear_cache=False, checkpoint=False):
    model, inps = workloads.build_model(2, T=T, device=gpu)
    mxfp8.enable_mxfp8(model)
    fused_linear.new_step()
    mod = model.layers[0].mlp
    x = inps[0]["x"].to(gpu).requires_grad_(True)
    if checkpoint:
        y = torch.utils.checkpoint.checkpoint(fused_mlp.mlp, mod, x, use_reentrant=False)
    else:
        y = fused_mlp.mlp(mod, x)
    assert y is not None
    if clear_cache:
        fused_linear.new_step()  # backward must rebuild the transposed LoRA forms from the saved tensors
    y.backward(inps[0]["dy"].to(gpu))
    torch.cuda.synchronize()
    params = [mod.gate_proj.lora_A["default"].weight, mod.gate_proj.lora_B["default"].weight,
              mod.up_proj.lora_A["default"].weight, mod.up_proj.lora_B["default"].weight,
              mod.down_proj.lora_A["default"].weight, mod.down_proj.lora_B["default"].weight]
    return y.detach(), x.grad, [p.grad for p in params]


def test_backward_returns_reference_dtypes(gpu):
    model, inps = workloads.build_model(2, T=256, device=gpu)
    mxfp8.enable_mxfp8(model)
    fused_linear.new_step()
    mod = model.layers[0].mlp
    x = inps[0]["x"].to(gpu).requires_grad_(True)
    y = fused_mlp.mlp(mod, x)
    assert type(y.grad_fn).__name__ == "_MLPBackward"
    assert len(y.grad_fn.saved_tensors) == 8  # x2, xs, gu, S, bg, bu, ad, bd (fused_mlp.py:291)
    out = y.grad_fn.apply(inps[0]["dy"].to(gpu))  # the raw returns of _MLP.backward
    dx, m, n, dA_g, dB_g, dA_u, dB_u, dA_d, dB_d = out
    K, N, r = x.shape[-1], mod.gate_proj.base_layer.out_features, 16
    assert m is None and n is None
    # the PEFT-shaped adapters are fp32 parameters: dA_g, dA_u, dB_d come back as fp32 holding bf16 values
    want = dict(dx=(torch.bfloat16, (256, K)), dA_g=(torch.float32, (r, K)), dB_g=(torch.float32, (N, r)),
                dA_u=(torch.float32, (r, K)), dB_u=(torch.float32, (N, r)), dA_d=(torch.float32, (r, N)),
                dB_d=(torch.float32, (K, r)))
    got = dict(dx=dx, dA_g=dA_g, dB_g=dB_g, dA_u=dA_u, dB_u=dB_u, dA_d=dA_d, dB_d=dB_d)
    for k, (dt, shape) in want.items():
        assert got[k].dtype == dt and tuple(got[k].shape) == shape, (k, got[k].dtype, tuple(got[k].shape))
    for k in ("dA_g", "dA_u", "dB_d"):  # the values of the reference's bf16 GEMM outputs
        assert torch.equal(got[k], got[k].to(torch.bfloat16).float()), k
    # with bf16 adapter parameters the same returns are bf16
    for m in (mod.gate_proj, mod.up_proj, mod.down_proj):
        m.lora_A["default"].to(torch.bfloat16)
        m.lora_B["default"].to(torch.bfloat16)
    fused_linear.new_step()
    x.grad = None
    y = fused_mlp.mlp(mod, x)
    out16 = y.grad_fn.apply(inps[0]["dy"].to(gpu))
    for k, t in zip(("dA_g", "dA_u", "dB_d"), (out16[3], out16[5], out16[8])):
        assert t.dtype == torch.bfloat16 and torch.equal(t.float(), got[k]), k


def test_cleared_cache_and_checkpoint_give_identical_gradients(gpu):
    y0, dx0, g0 = _mlp_run(gpu)
    for kw in (dict(clear_cache=True), dict(checkpoint=True)):
        y1, dx1, g1 = _mlp_run(gpu, **kw)
        assert torch.equal(y0, y1) and torch.equal(dx0, dx1), kw
        for a, b in zip(g0, g1):
            assert torch.equal(a, b), kw


def _two_layer_grads(gpu, hooks):
    """x -> mlp(layer 0) -> mlp(layer 1) -> backward; LoRA gradients of both layers and dx.  hooks=True runs
    under a saved-tensor hook whose unpack returns a fresh clone at every access, so each layer's backward sees
    short-lived objects (whose addresses a later layer's clones may take) instead of the tensors forward saved."""
    model, inps = workloads.build_model(2, T=256, layers=2, device=gpu)
    mxfp8.enable_mxfp8(model)
    fused_linear.new_step()
    x = inps[0]["x"].to(gpu).requires_grad_(True)
    ctx = (torch.autograd.graph.saved_tensors_hooks(lambda t: t, lambda t: t.clone()) if hooks
           else torch.autograd.graph.saved_tensors_hooks(lambda t: t, lambda t: t))
    with ctx:
        h = fused_mlp.mlp(model.layers[0].mlp, x)
        y = fused_mlp.mlp(model.layers[1].mlp, h)
    y.backward(inps[0]["dy"].to(gpu))
    torch.cuda.synchronize()
    grads = [x.grad]
    for layer in model.layers:
        for name in ("gate_proj", "up_proj", "down_proj"):
            lin = getattr(layer.mlp, name)
            grads += [lin.lora_A["default"].weight.grad, lin.lora_B["default"].weight.grad]
    return grads


def test_cloning_unpack_hook_gives_identical_gradients(gpu):
    """Two layers with distinct adapters: backward under a cloning unpack hook must find each layer's own
    transposed LoRA forms (the per-step cache keeps its key tensors alive and checks object identity), so every
    gradient is bit-identical to the run without the hook."""
    g0 = _two_layer_grads(gpu, hooks=False)
    g1 = _two_layer_grads(gpu, hooks=True)
    for k, (a, b) in enumerate(zip(g0, g1)):
        assert a is not None and torch.equal(a, b), k
    # the two layers' adapters differ, so a lookup that returned the other layer's forms would change them
    assert not torch.equal(g0[1], g0[7])


def test_enable_disable_round_trip(gpu):
    model, inps = workloads.build_model(2, T=128, device=gpu)
    lins = [m for n, m in model.named_modules() if n.endswith("base_layer")]
    assert len(lins) == 3
    before = [lin.weight.detach().clone() for lin in lins]
    assert mxfp8.enable_mxfp8(model) == 3
    for lin in lins:
        assert lin.weight.numel() == 0 and "forward" in lin.__dict__ and mxfp8.is_mx(lin)
    mxfp8.disable_mxfp8(model)
    for lin, w in zip(lins, before):
        assert torch.equal(lin.weight, w) and lin.weight.device == w.device
        assert "forward" not in lin.__dict__ and not mxfp8.is_mx(lin)
        assert not [a for a in lin.__dict__ if a.startswith("_mx_") or a == "_bf16_cpu"]
    x = inps[0]["x"].to(gpu)
    assert torch.equal(lins[0](x), torch.nn.functional.linear(x, before[0]))  # the class forward again


def test_mx_linear_forward_backward_and_reuse(gpu):
    model, inps = workloads.build_model(2, T=384, device=gpu)
    inp = inps[0]
    mxfp8.enable_mxfp8(model)
    mlp = model.layers[0].mlp
    down = mlp.down_proj.base_layer  # a single MX linear: neither paired nor in a concatenated group
    K, N = inp["K"], inp["N"]
    g = torch.Generator().manual_seed(11)
    h = (torch.randn(384, N, generator=g) * 0.5).to(torch.bfloat16)
    x = h.to(gpu).requires_grad_(True)
    q0 = mxfp8.STATS["quant"]
    y = down(x)
    W = omlp.prepare_weights(inp["Wg"], inp["Wu"], inp["Wd"])
    qh, sh = mx.quant(h)
    _assert_gemm_close(y, mx.dequant(qh, sh, 384, N).double() @ mx.dequant(W["dw"], W["dws"], K, N).double().t())
    dy = (torch.randn(384, K, generator=g) * 1e-2).to(torch.bfloat16)
    y.backward(dy.to(gpu))
    qd, sd = mx.quant(dy)
    ref_dx = mx.dequant(qd, sd, 384, K).double() @ mx.dequant(W["dwt"], W["dwts"], N, K).double().t()
    _assert_gemm_close(x.grad, ref_dx)
    assert mxfp8.STATS["quant"] == q0 + 2  # x in forward, dy in backward
    # gate and up take the same live input: the second call reuses its codes; an in-place change does not
    xg = inp["x"].to(gpu)
    r0, q0 = mxfp8.STATS["reuse"], mxfp8.STATS["quant"]
    mlp.gate_proj.base_layer(xg)
    mlp.up_proj.base_layer(xg)
    assert (mxfp8.STATS["quant"], mxfp8.STATS["reuse"]) == (q0 + 1, r0 + 1)
    xg.mul_(1.0)
    mlp.up_proj.base_layer(xg)
    assert mxfp8.STATS["quant"] == q0 + 2
