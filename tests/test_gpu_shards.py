"""Data parallelism over tokens, on one GPU: the fused MLP run on two token shards separately against the same
MLP run on the whole batch.  Sharding the tokens of a step over GPUs relies on three properties of the path,
checked here through the product kernels (configuration-3 shapes, T = 2048 split at row 1024, and at row 1000,
where the second shard's rows sit at other offsets inside their 32- and 128-row blocks):
  - forward rows are independent: quantization blocks run along a row, the GEMMs accumulate each output element
    over K in a fixed order whatever tile its row falls in, and the LoRA products and their partial sums are
    per row.  So every y row is bit-identical between the shard and the whole run;
  - dx rows are independent too, but the backward's grid (and so the grouping of the d(xa) partial sums) follows
    T, so a dx row may differ by fp32 summation order: within 2^-8 of max|dx| (measured: bit-identical at these
    splits);
  - the LoRA gradients are sums over tokens, so the whole run's gradient is the shards' sum (the one exchange of
    data parallelism, an all-reduce).  dB_g, dB_u and dA_d are fp32 sums: within 1e-5 of max|grad| (measured
    1.6e-7 to 2.4e-7).  dA_g, dA_u and dB_d are rounded to bf16 per product, as the reference rounds them, so
    each shard's rounding adds up to one bf16 step: within 2^-7 of max|grad| (measured 4.0e-3 to 4.1e-3)."""
import pytest
import torch

import fused_linear
import fused_mlp
import mxfp8
import workloads

pytestmark = pytest.mark.gpu

_FP32 = ("dB_g", "dB_u", "dA_d")  # fp32 sums over the tokens
_BF16 = ("dA_g", "dA_u", "dB_d")  # bf16-rounded products


def _grads(m):
    return {"dA_g": m.gate_proj.lora_A["default"].weight.grad, "dB_g": m.gate_proj.lora_B["default"].weight.grad,
            "dA_u": m.up_proj.lora_A["default"].weight.grad, "dB_u": m.up_proj.lora_B["default"].weight.grad,
            "dA_d": m.down_proj.lora_A["default"].weight.grad, "dB_d": m.down_proj.lora_B["default"].weight.grad}


def _run(model, mod, x, dy):
    fused_linear.new_step()
    for p in model.parameters():
        p.grad = None
    xi = x.clone().requires_grad_(True)
    y = fused_mlp.mlp(mod, xi)
    assert y is not None
    y.backward(dy)
    torch.cuda.synchronize()
    return y.detach(), xi.grad, {k: g.detach().clone() for k, g in _grads(mod).items()}


def _rel(got, ref):
    return ((got.float() - ref.float()).abs().max() / ref.float().abs().max().clamp_min(1e-30)).item()


@pytest.mark.parametrize("split", [1000, 1024])
def test_token_shards_match_the_whole_batch(split, gpu):
    T = 2048
    model, inps = workloads.build_model(3, T=T, device=gpu)
    mxfp8.enable_mxfp8(model)
    mod = model.layers[0].mlp
    x, dy = inps[0]["x"].to(gpu), inps[0]["dy"].to(gpu)
    y, dx, g = _run(model, mod, x, dy)
    parts = [_run(model, mod, x[a:b], dy[a:b]) for a, b in ((0, split), (split, T))]
    y_s = torch.cat([p[0] for p in parts])
    dx_s = torch.cat([p[1] for p in parts])
    assert torch.equal(y_s, y), (y_s != y).float().mean().item()
    errs = {"dx": _rel(dx_s, dx)}
    for k in _FP32 + _BF16:
        errs[k] = _rel(parts[0][2][k] + parts[1][2][k], g[k])
    print(f"split {split}: " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert errs["dx"] <= 2.0 ** -8, errs
    assert all(errs[k] <= 1e-5 for k in _FP32), errs
    assert all(errs[k] <= 2.0 ** -7 for k in _BF16), errs
