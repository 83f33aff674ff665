"""Host-side checks of the grouped linears (fused_linear._Group, group_linear, residual_add) on the CPU: with plain
(non-MX) layers the group runs the reference's bf16/fp32 torch path (fused_linear.py:79-196), so its outputs and
gradients must equal calling each module alone, up to fp32 summation order."""
import torch
from torch import nn

import fused_linear
import workloads


def _frozen(n_out, n_in, g):
    m = nn.Linear(n_in, n_out, bias=False)
    with torch.no_grad():
        m.weight.copy_(torch.randn(n_out, n_in, generator=g) * 0.05)
    m.weight.requires_grad_(False)
    return m


def _lora(n_out, n_in, r, g, alpha=32.0):
    A = torch.randn(r, n_in, generator=g) * 0.05
    B = torch.randn(n_out, r, generator=g) * 0.05
    return workloads.LoraLinear(_frozen(n_out, n_in, g), A, B, alpha)


def _params(mods):
    out = []
    for m in mods:
        if isinstance(m, workloads.LoraLinear):
            out += [m.lora_A["default"].weight, m.lora_B["default"].weight]
    return out


def test_part_protocol():
    g = torch.Generator().manual_seed(0)
    lin = _frozen(16, 64, g)
    assert fused_linear._part(lin) == (lin, None, None, 1.0)
    lo = _lora(128, 64, 8, g)
    base, A, B, s = fused_linear._part(lo)
    assert base is lo.base_layer and A is lo.lora_A["default"].weight and s == 4.0
    lin.weight.requires_grad_(True)  # a trainable base cannot be grouped
    assert fused_linear._part(lin) is None


def test_group_matches_modules_one_by_one():
    # q / k / v with LoRA plus a thin frozen linear (<= _THIN outputs), fp32 on the CPU
    g = torch.Generator().manual_seed(1)
    K, T = 96, 37
    mods = [_lora(128, K, 8, g), _lora(64, K, 16, g), _lora(64, K, 8, g), _frozen(16, K, g)]
    x = torch.randn(2, T, K, generator=g, requires_grad=True)
    dys = [torch.randn(2, T, m.base_layer.out_features if hasattr(m, "base_layer") else m.out_features, generator=g)
           for m in mods]
    before = fused_linear.STATS["gộp"]
    outs = fused_linear.group_linear(x, mods)
    assert fused_linear.STATS["gộp"] == before + 1
    torch.autograd.backward(outs, dys)
    got = [x.grad.clone()] + [p.grad.clone() for p in _params(mods)]
    x.grad = None
    for p in _params(mods):
        p.grad = None
    ref_outs = [m(x) for m in mods]
    torch.autograd.backward(ref_outs, dys)
    want = [x.grad] + [p.grad for p in _params(mods)]
    for a, b in zip(outs, ref_outs):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6)
    for a, b in zip(got, want):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


def test_unused_output_gets_no_gradient_and_need_out_false():
    g = torch.Generator().manual_seed(2)
    K = 64
    mods = [_lora(128, K, 8, g), _lora(128, K, 8, g)]
    x = torch.randn(5, K, generator=g, requires_grad=True)
    a, b = fused_linear.group_linear(x, mods)
    b.sum().backward()  # a unused: its B gets no gradient
    assert mods[0].lora_B["default"].weight.grad is None
    assert mods[1].lora_B["default"].weight.grad is not None
    outs = fused_linear.group_linear(x.detach(), mods, need_out=False)
    assert [o.shape for o in outs] == [(5, 128), (5, 128)]


def test_ungroupable_layer_calls_modules_directly():
    g = torch.Generator().manual_seed(3)
    K = 64
    lo = _lora(128, K, 8, g)
    lo.lora_dropout["default"] = nn.Dropout(0.1)
    before = fused_linear.STATS["gọi thẳng"]
    lo.eval()
    x = torch.randn(3, K, generator=g)
    (y,) = fused_linear.group_linear(x, [lo])
    assert fused_linear.STATS["gọi thẳng"] == before + 1
    torch.testing.assert_close(y, lo(x))


def test_residual_add_plain_and_fallback():
    g = torch.Generator().manual_seed(4)
    x, y = torch.randn(4, 128, generator=g), torch.randn(4, 128, generator=g)
    torch.testing.assert_close(fused_linear.residual_add(x, y), x + y)
    # a Deferred in fp32 (not the bf16 kernel's case) takes the addmm path
    xa, B = torch.randn(4, 8, generator=g), torch.randn(128, 8, generator=g)
    d = fused_linear.Deferred((y, xa, B, 0.5))
    torch.testing.assert_close(fused_linear.residual_add(x, d), x + y + 0.5 * xa @ B.t())
