"""Configuration 4 at full size: 24 Qwen3.5-2B-shaped MLP layers at 142,336 tokens per step (16 packed
conversations of 8,896 tokens), forward then backward through the stack, the training step of
/root/reference/scripts/shared_prefix.py:466-605 for the MLPs.  The layers sit on a residual stream as in the
reference decoder, x <- x + mlp(rms_norm(x)) (shared_prefix.py:239, :252; torch's RMSNorm with unit weight stands
in for post_attention_layernorm).  Without the norm the stream grows quadratically per layer until it overflows;
without the residual (y = mlp(y)) it shrinks quadratically and reaches exact zeros long before layer 24.

At this size gu holds 142,336 x 12,288 bf16 (3.5 GB, byte offsets past 2^31) and T * 2N is 81% of 2^31, so the
kernels' 64-bit byte offsets and 32-bit element indexing are both exercised.  The CPU oracle cannot run the whole
shape in test time, so the checks use properties that hold at any size:
  - two runs of the whole stack are bit-identical (the partial sums are added in a fixed order), and finite;
  - the MX codes and scales of x and dy are bit-exact against the oracle on sampled 128-row blocks (the first,
    two inner ones and the last), in both the row-major and the MX-tiled layouts;
  - forward rows are independent, so layers 0, 11 and 23 are checked against the oracle on the sampled rows of
    the GPU's own input to that layer (the boundary tensor), within the MLP tolerance;
  - the LoRA gradients are sums of per-token terms that vanish where dy is zero, so an inner layer (11) and the
    last one (23) are each run once more at full size on their own recorded input with dy zero outside the
    sampled rows; their gradients (and those rows of dx) must then match the oracle's on the sampled rows alone.
    The 22 inner layers share one code path, so layer 11 stands for them (its input has passed 11 fused MLPs and
    norms, not the seeded x)."""
import pytest
import torch

import fused_linear
import fused_mlp
import mxfp8
import workloads
from oracle import mlp as omlp
from oracle import mx

pytestmark = pytest.mark.gpu
TOL = 2e-2
BLOCKS = (0, 389, 777, 1111)  # 128-row blocks sampled from T = 142336 = 1112 * 128
INNER = 11  # the inner layer whose forward rows and LoRA gradients are checked against the oracle


def _rows():
    return torch.cat([torch.arange(128 * b, 128 * b + 128) for b in BLOCKS])


def _rel(got, ref):
    got, ref = got.float().cpu(), ref.float().cpu()
    return ((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def _lora_grads(m):
    return {"dA_g": m.gate_proj.lora_A["default"].weight.grad, "dB_g": m.gate_proj.lora_B["default"].weight.grad,
            "dA_u": m.up_proj.lora_A["default"].weight.grad, "dB_u": m.up_proj.lora_B["default"].weight.grad,
            "dA_d": m.down_proj.lora_A["default"].weight.grad, "dB_d": m.down_proj.lora_B["default"].weight.grad}


def _check_codes(x_gpu, x_cpu, name):
    """Row-major (mx_quant) and MX-tiled (mx_quant_lora) codes and the blocked scales on the sampled blocks."""
    K = x_cpu.shape[1]
    q, s = mxfp8.mx_quant(x_gpu)
    w = torch.zeros((16, K), dtype=torch.bfloat16, device=x_gpu.device)
    qt, st, _, _ = mxfp8.mx_quant_lora(x_gpu, w, out_t=False)
    tile_bytes = (K // 128) * 512  # scale bytes of one 128-row tile row
    for b in BLOCKS:
        rq, rs = mx.quant(x_cpu[128 * b:128 * b + 128])
        assert torch.equal(q[128 * b:128 * b + 128].view(torch.uint8).cpu(), rq), (name, b, "codes")
        got_t = mx.from_tiled(qt[128 * b:128 * b + 128].view(torch.uint8).cpu().reshape(-1).numpy(), 128, K)
        assert torch.equal(torch.from_numpy(got_t), rq), (name, b, "tiled codes")
        for sc in (s, st):
            assert torch.equal(sc.view(torch.uint8)[b * tile_bytes:(b + 1) * tile_bytes].cpu(), rs), (name, b)


def test_config4_full_size_stack(gpu):
    c = workloads.CONFIGS[4]
    T, L = c["T"], c["layers"]
    print(f"building {L} layers at T={T}", flush=True)
    model, inps = workloads.build_model(4, layers=L, device=gpu)
    mxfp8.enable_mxfp8(model)
    mods = [layer.mlp for layer in model.layers]
    inp0 = inps[0]
    x_cpu, dy_cpu = inp0["x"], inp0["dy"]
    x = x_cpu.to(gpu)
    dy = dy_cpu.to(gpu)
    _check_codes(x, x_cpu, "x")
    _check_codes(dy, dy_cpu, "dy")
    print("codes ok", flush=True)
    params = [p for p in model.parameters() if p.requires_grad]

    def run():
        fused_linear.new_step()
        for p in params:
            p.grad = None
        xin = x.clone().requires_grad_(True)
        acts, outs, y = [], [], xin
        for m in mods:
            xn = torch.nn.functional.rms_norm(y, (y.shape[-1],), eps=1e-6)
            acts.append(xn.detach())
            o = fused_mlp.mlp(m, xn)
            assert o is not None
            outs.append(o.detach())
            y = y + o
        y.backward(dy)
        torch.cuda.synchronize()
        return acts, outs, y.detach(), xin.grad, [g.clone() for m in mods for g in _lora_grads(m).values()]

    acts, outs, y1, dx1, g1 = run()
    print("run 1 done", flush=True)
    for t in [y1, dx1] + g1:
        assert bool(torch.isfinite(t).all())
    for li in (0, INNER, L - 1):  # every MLP computes on unit-scale inputs and gives non-vanishing outputs
        assert acts[li].float().std().item() > 0.5 and outs[li].float().std().item() > 0.05, li
    _, _, y2, dx2, g2 = run()
    print("run 2 done", flush=True)
    assert torch.equal(y1, y2) and torch.equal(dx1, dx2)
    assert all(torch.equal(a, b) for a, b in zip(g1, g2))

    rows = _rows()
    s = inp0["s"]
    checked = (INNER, L - 1)
    x_in = {li: acts[li] for li in checked}  # the GPU's input to those MLPs (the same bits in both runs)
    errs = {}
    for li in (0, INNER, L - 1):
        inp = inps[li]
        W = omlp.prepare_weights(inp["Wg"], inp["Wu"], inp["Wd"])
        S, bg, bu, ad, bd = omlp.lora_cast(inp["Ag"], inp["Bg"], inp["Au"], inp["Bu"], inp["Ad"], inp["Bd"])
        f = omlp.forward(acts[li][rows].cpu(), W, S, bg, bu, ad, bd, s, s, s)
        errs[f"y{li}"] = _rel(outs[li][rows], f["y"])
    del acts, outs, y1, y2, dx1, dx2, g1, g2
    print("forward rows ok", flush=True)

    # layers 11 and 23 again, each at full size on its recorded input, with dy zero outside the sampled rows
    for li in checked:
        m, inp = mods[li], inps[li]
        fused_linear.new_step()
        for p in params:
            p.grad = None
        xl = x_in[li].clone().requires_grad_(True)
        dy_sparse = torch.zeros_like(dy)
        dy_sparse[rows.to(gpu)] = dy[rows.to(gpu)]
        yl = fused_mlp.mlp(m, xl)
        yl.backward(dy_sparse)
        torch.cuda.synchronize()
        W = omlp.prepare_weights(inp["Wg"], inp["Wu"], inp["Wd"])
        S, bg, bu, ad, bd = omlp.lora_cast(inp["Ag"], inp["Bg"], inp["Au"], inp["Bu"], inp["Ad"], inp["Bd"])
        xr = x_in[li][rows].cpu()
        f = omlp.forward(xr, W, S, bg, bu, ad, bd, s, s, s)
        b = omlp.backward(xr, f["xs"], f["gu"], W, S, bg, bu, ad, bd, s, s, s, dy_cpu[rows])
        errs[f"dx{li}"] = _rel(xl.grad[rows.to(gpu)], b["dx"])
        for k, g in _lora_grads(m).items():
            assert bool(torch.isfinite(g).all()), (li, k)
            errs[f"{k}{li}"] = _rel(g, b[k])
        del xl, yl, dy_sparse
        print(f"layer {li} gradients checked", flush=True)
    print(" ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert all(v <= TOL for v in errs.values()), errs
