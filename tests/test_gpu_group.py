"""Grouped MX linears (fused_linear._Group with mxfp8.lora_bwd and the concatenated Wᵀ GEMM, after
/root/reference/scripts/fused_linear.py:79-330 and mxfp8.py:360-439) against the CPU oracle: the MX operands are the
oracle quantizer's codes, dequantized exactly, and every product is taken in float64.  Bar: normwise relative error
<= 1e-2 and elementwise within 2e-2 of (|value| + the tensor's rms), under the 2e-2 output/gradient tolerance."""
import pytest
import torch
from torch import nn

import fused_linear
import workloads

pytestmark = pytest.mark.gpu

T, K, NQ, NKV, R, ALPHA, NTHIN = 300, 1024, 1024, 256, 16, 32.0, 16


class _Attn(nn.Module):
    def __init__(self, g):
        super().__init__()

        def lin(n_out, n_in):
            m = nn.Linear(n_in, n_out, bias=False)
            with torch.no_grad():
                m.weight.copy_(torch.randn(n_out, n_in, generator=g) * 0.03)
            m.weight.requires_grad_(False)
            return m

        def lora(n_out, n_in):
            return workloads.LoraLinear(lin(n_out, n_in), torch.randn(R, n_in, generator=g) * 0.03,
                                        torch.randn(n_out, R, generator=g) * 0.03, ALPHA)

        self.q_proj, self.k_proj, self.v_proj = lora(NQ, K), lora(NKV, K), lora(NKV, K)
        self.o_proj = lora(K, NQ)
        self.thin = lin(NTHIN, K)  # not an MX name: a thin plain linear that joins the S GEMM


class _Model(nn.Module):
    def __init__(self, g):
        super().__init__()
        self.model = nn.Module()
        layer = nn.Module()
        layer.self_attn = _Attn(g)
        self.model.layers = nn.ModuleList([layer])

    @property
    def attn(self):
        return self.model.layers[0].self_attn


def _build(gpu, seed=0):
    import mxfp8
    g = torch.Generator().manual_seed(seed)
    m = _Model(g)
    for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
        getattr(m.attn, name).base_layer.to(dtype=torch.bfloat16)
    m.attn.thin.to(dtype=torch.bfloat16)
    m = m.to(gpu)
    w_cpu = {n: getattr(m.attn, n).base_layer.weight.detach().cpu().clone() for n in ("q_proj", "k_proj", "v_proj",
                                                                                      "o_proj")}
    mxfp8.enable_mxfp8(m)
    fused_linear.new_step()
    return m, w_cpu


def _close(got, want, what):
    got, want = got.detach().double().cpu(), want.double()
    rms = want.pow(2).mean().sqrt().item()
    nrm = ((got - want).norm() / want.norm().clamp_min(1e-30)).item()
    assert nrm <= 1e-2, (what, nrm)
    bad = (got - want).abs() > 2e-2 * (want.abs() + rms)
    assert not bool(bad.any()), (what, int(bad.sum()), (got - want).abs().max().item())


def _deq(x2d):
    from oracle import mx
    q, s = mx.quant(x2d)
    return mx.dequant(q, s, x2d.shape[0], x2d.shape[1]).double()


def _deq_t(w):
    """Wᵀ quantized along N (the dx operand), dequantized, as [K, N]."""
    return _deq(w.t().contiguous())


def _bf(t):
    return t.to(torch.bfloat16).double()


def _oracle(m, w_cpu, x, dys, names):
    """Outputs, dx, dB, dA of the group in float64 from the oracle's MX codes (bf16 rounding of xa = x·Aᵀ and of
    d(xa) kept, as the path stores them in bf16)."""
    xd = x.double()
    xq = _deq(x)
    outs, dx, grads = [], 0.0, {}
    dS, Srows = [], []
    for n, dy in zip(names, dys):
        mod = getattr(m.attn, n)
        if n == "thin":
            W = mod.weight.detach().cpu().double()
            outs.append(_bf(xd @ W.t()))
            dS.append(dy.double())
            Srows.append(W)
            continue
        A = mod.lora_A["default"].weight.detach().cpu().to(torch.bfloat16).double()
        B = mod.lora_B["default"].weight.detach().cpu().to(torch.bfloat16).double()
        s = mod.scaling["default"]
        xa = _bf(xd @ A.t())
        y0 = _bf(xq @ _deq(w_cpu[n]).t())
        outs.append(y0 + s * xa @ B.t())
        dyd = dy.double()
        dx = dx + _deq(dy) @ _deq_t(w_cpu[n]).t()
        dxa = _bf(s * dyd @ B)
        grads[n] = (s * dyd.t() @ xa, dxa.t() @ xd)  # dB, dA
        dS.append(dxa)
        Srows.append(A)
    dx = dx + torch.cat(dS, 1) @ torch.cat(Srows, 0)
    return outs, dx, grads


@pytest.mark.parametrize("fused", [True, False])
def test_group_qkv_thin_matches_oracle(fused, gpu):
    import mxfp8
    m, w_cpu = _build(gpu)
    a = m.attn
    names = ["q_proj", "k_proj", "v_proj", "thin"]
    assert a.q_proj.base_layer.__dict__.get("_mx_cat") is not None and a.q_proj.base_layer._mx_fbwd
    if not fused:
        for n in names[:3]:
            getattr(a, n).base_layer._mx_fbwd = False  # the plain path: one MX GEMM per layer, bf16 adds
    g = torch.Generator().manual_seed(11)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16)
    dys = [(torch.randn(T, n, generator=g) * 0.1).to(torch.bfloat16) for n in (NQ, NKV, NKV, NTHIN)]
    xg = x.to(gpu).requires_grad_(True)
    before = fused_linear.STATS.get("lan ngược gộp", 0)
    outs = fused_linear.group_linear(xg, [getattr(a, n) for n in names])
    torch.autograd.backward(outs, [d.to(gpu) for d in dys])
    assert fused_linear.STATS.get("lan ngược gộp", 0) == before + (1 if fused else 0)
    w_outs, w_dx, w_grads = _oracle(m, w_cpu, x, dys, names)
    for n, o, w in zip(names, outs, w_outs):
        _close(o, w, n)
    _close(xg.grad, w_dx, "dx")
    for n in names[:3]:
        mod = getattr(a, n)
        dB, dA = w_grads[n]
        assert mod.lora_B["default"].weight.grad.dtype == torch.float32
        _close(mod.lora_B["default"].weight.grad, dB, n + ".dB")
        _close(mod.lora_A["default"].weight.grad, dA, n + ".dA")
    assert mxfp8.group_wt([a.q_proj.base_layer, a.k_proj.base_layer]) is not None
    assert mxfp8.group_wt([a.k_proj.base_layer, a.q_proj.base_layer]) is None


def test_group_odd_multiples_of_128(gpu, monkeypatch):
    # d_model 384 and a q width of 640 (odd multiples of 128): the thin products (lora_nt / lora_tn), the grouped
    # GEMMs and their segment boundaries away from multiples of 256
    import sys
    here = sys.modules[__name__]
    monkeypatch.setattr(here, "K", 384)
    monkeypatch.setattr(here, "NQ", 640)
    test_group_qkv_thin_matches_oracle(True, gpu)


def test_cat_ranges_are_the_layers_own_quantization(gpu):
    # a column range of the concatenated Wᵀ (codes and cut-out scales) equals quantizing that layer's Wᵀ alone
    import mxfp8
    from oracle import mx
    m, w_cpu = _build(gpu, seed=3)
    for k, n in enumerate(("q_proj", "k_proj", "v_proj")):
        base = getattr(m.attn, n).base_layer
        mat2, sc = mxfp8.wt_of(base)
        qr, sr = mx.quant_t(w_cpu[n])
        assert torch.equal(mat2.t().contiguous().view(torch.uint8).cpu(), qr)
        assert torch.equal(sc.view(torch.uint8).cpu(), sr)
        qf, sf = mx.quant(w_cpu[n])  # forward codes: rows of the concatenated quantization
        assert torch.equal(base._mx_w.view(torch.uint8).cpu(), qf) and torch.equal(base._mx_ws.view(torch.uint8).cpu(),
                                                                                  sf)


def test_residual_add_deferred_matches_plain(gpu):
    # o_proj's output with LoRA added in the residual kernel == the grouped output added to the residual
    m, _ = _build(gpu, seed=5)
    o = m.attn.o_proj
    g = torch.Generator().manual_seed(12)
    h = torch.randn(T, NQ, generator=g).to(torch.bfloat16).to(gpu)
    resid = torch.randn(T, K, generator=g).to(torch.bfloat16).to(gpu)
    (d,) = fused_linear.group_linear(h, [o], defer=True)
    assert isinstance(d, fused_linear.Deferred)
    before = fused_linear.STATS.get("residual LoRA", 0)
    got = fused_linear.residual_add(resid, d)
    assert fused_linear.STATS.get("residual LoRA", 0) == before + 1
    (y,) = fused_linear.group_linear(h, [o])
    want = resid + y
    # both round y + s·xa·Bᵀ to bf16, then x + that; the r products are summed in another order, so an element may
    # differ by one step of the intermediate
    d_ = (got.float() - want.float()).abs()
    t = torch.maximum(y.float().abs(), got.float().abs())
    assert bool((d_ <= torch.exp2(torch.floor(torch.log2(t.clamp_min(1e-30)))) * 2 ** -7 * 1.0001 + 1e-30).all())
    assert (got == want).double().mean().item() >= 0.99


@pytest.mark.parametrize("r", [32, 8])
def test_group_other_ranks_match_plain_path(r, gpu):
    # r = 32 takes the fused kernels with a 64-wide padded S (3 layers x 32 = 96 rows: the torch thin GEMMs);
    # r = 8 is outside the fused kernels' ranks (codes from lora_bwd, products as plain GEMMs): the grouped
    # backward must match the plain backward of the same layers within tolerance either way
    import mxfp8
    g = torch.Generator().manual_seed(20 + r)
    m = _Model.__new__(_Model)
    nn.Module.__init__(m)
    m.model = nn.Module()
    layer = nn.Module()
    attn = nn.Module()

    def lin(n_out, n_in):
        x = nn.Linear(n_in, n_out, bias=False)
        with torch.no_grad():
            x.weight.copy_(torch.randn(n_out, n_in, generator=g) * 0.03)
        x.weight.requires_grad_(False)
        return x

    for name, n in (("q_proj", NQ), ("k_proj", NKV), ("v_proj", NKV)):
        setattr(attn, name, workloads.LoraLinear(lin(n, K), torch.randn(r, K, generator=g) * 0.03,
                                                 torch.randn(n, r, generator=g) * 0.03, ALPHA))
        getattr(attn, name).base_layer.to(dtype=torch.bfloat16)
    layer.self_attn = attn
    m.model.layers = nn.ModuleList([layer])
    m = m.to(gpu)
    mxfp8.enable_mxfp8(m)
    mods = [attn.q_proj, attn.k_proj, attn.v_proj]
    x = (torch.randn(T, K, generator=g)).to(torch.bfloat16).to(gpu)
    dys = [(torch.randn(T, n, generator=g) * 0.1).to(torch.bfloat16).to(gpu) for n in (NQ, NKV, NKV)]

    def run():
        fused_linear.new_step()
        for p in m.parameters():
            p.grad = None
        xg = x.clone().requires_grad_(True)
        outs = fused_linear.group_linear(xg, mods)
        torch.autograd.backward(outs, dys)
        return [o.detach() for o in outs], xg.grad, [p.grad.clone() for p in m.parameters() if p.requires_grad]

    before = fused_linear.STATS.get("lan ngược gộp", 0)
    of, dxf, gf = run()
    assert fused_linear.STATS.get("lan ngược gộp", 0) == before + 1
    for mod in mods:
        mod.base_layer._mx_fbwd = False
    op, dxp, gp = run()
    for a, b in zip(of, op):
        assert torch.equal(a, b)  # same forward path
    _close(dxf, dxp.double().cpu(), "dx")
    for k, (a, b) in enumerate(zip(gf, gp)):
        _close(a, b.double().cpu(), f"grad {k}")


def test_need_out_false_keeps_gradients(gpu):
    # the recompute mode builds the same graph without the base GEMM outputs: identical gradients
    m, _ = _build(gpu, seed=9)
    a = m.attn
    mods = [a.q_proj, a.k_proj, a.v_proj]
    g = torch.Generator().manual_seed(13)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16).to(gpu)
    dys = [(torch.randn(T, n, generator=g) * 0.1).to(torch.bfloat16).to(gpu) for n in (NQ, NKV, NKV)]
    res = []
    for need_out in (True, False):
        fused_linear.new_step()
        for p in m.parameters():
            p.grad = None
        xg = x.clone().requires_grad_(True)
        outs = fused_linear.group_linear(xg, mods, need_out=need_out)
        torch.autograd.backward(outs, dys)
        res.append([xg.grad.clone()] + [p.grad.clone() for p in m.parameters() if p.grad is not None])
    for u, v in zip(*res):
        assert torch.equal(u, v)


def test_merged_forward_gemm_matches_one_gemm_per_layer(gpu):
    # q|k|v as ONE GEMM over the concatenated forward weight with the block-diagonal LoRA epilogue: the same bits
    # as one GEMM per layer (the zero blocks add nothing), each output contiguous
    import mxfp8
    m, _ = _build(gpu, seed=21)
    a = m.attn
    mods = [a.q_proj, a.k_proj, a.v_proj]
    g = torch.Generator().manual_seed(22)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16).to(gpu)
    fused_linear.new_step()
    merged = fused_linear.group_linear(x, mods)
    assert all(o.is_contiguous() for o in merged)
    saved = mxfp8.group_fwd_operand
    mxfp8.group_fwd_operand = lambda lins: None  # one GEMM per layer
    try:
        fused_linear.new_step()
        single = fused_linear.group_linear(x, mods)
    finally:
        mxfp8.group_fwd_operand = saved
    for u, v in zip(merged, single):
        assert torch.equal(u, v)
    # two consecutive layers of the group (k|v) merge too; a non-consecutive pair (q, v) does not
    assert mxfp8.group_fwd_operand([a.k_proj.base_layer, a.v_proj.base_layer]) is not None
    assert mxfp8.group_fwd_operand([a.q_proj.base_layer, a.v_proj.base_layer]) is None


def test_weight_forms_follow_in_place_updates_and_new_parameters(gpu):
    # the per-step weight forms come from a buffer and job table kept across steps (fused_linear._PLANS): an
    # optimizer's in-place update and a parameter replaced by a new tensor must both reach the next step, with
    # the same bits as a plan built from scratch
    m, _ = _build(gpu, seed=31)
    a = m.attn
    mods = [a.q_proj, a.k_proj, a.v_proj]
    g = torch.Generator().manual_seed(32)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16).to(gpu)
    dys = [(torch.randn(T, n, generator=g) * 0.1).to(torch.bfloat16).to(gpu) for n in (NQ, NKV, NKV)]

    def step(fresh):
        if fresh:
            fused_linear._PLANS.clear()
        fused_linear.new_step()
        for p in m.parameters():
            p.grad = None
        xg = x.clone().requires_grad_(True)
        outs = fused_linear.group_linear(xg, mods)
        torch.autograd.backward(outs, dys)
        return [o.detach().clone() for o in outs] + [xg.grad.clone()] + [
            p.grad.clone() for p in m.parameters() if p.grad is not None]

    def same(u, v):
        assert len(u) == len(v) and all(torch.equal(s, t) for s, t in zip(u, v))

    first = step(fresh=True)
    same(step(fresh=False), first)  # the kept plan, unchanged weights
    with torch.no_grad():  # an optimizer step: in place, same addresses
        a.q_proj.lora_A["default"].weight.mul_(1.5)
        a.v_proj.lora_B["default"].weight.add_(0.01)
    updated = step(fresh=False)
    assert not torch.equal(updated[0], first[0]) and not torch.equal(updated[2], first[2])
    same(updated, step(fresh=True))
    old = a.k_proj.lora_A["default"].weight
    a.k_proj.lora_A["default"].weight = nn.Parameter(old.detach() * -1.0)  # a new tensor at a new address
    replaced = step(fresh=False)
    assert not torch.equal(replaced[1], updated[1])
    same(replaced, step(fresh=True))


def test_group_mixed_ranks(gpu):
    # q and v at rank 16, k at rank 32 (S 64 rows): the merged forward GEMM cannot take one rank window per
    # layer and runs its block-diagonal epilogue over all 64 columns, bit-identical to one GEMM per layer; the
    # grouped backward matches the plain per-layer backward within tolerance
    import mxfp8
    g = torch.Generator().manual_seed(40)
    m = _Model.__new__(_Model)
    nn.Module.__init__(m)
    m.model = nn.Module()
    layer = nn.Module()
    attn = nn.Module()

    def lin(n_out, n_in):
        x = nn.Linear(n_in, n_out, bias=False)
        with torch.no_grad():
            x.weight.copy_(torch.randn(n_out, n_in, generator=g) * 0.03)
        x.weight.requires_grad_(False)
        return x

    for name, n, r in (("q_proj", NQ, 16), ("k_proj", NKV, 32), ("v_proj", NKV, 16)):
        setattr(attn, name, workloads.LoraLinear(lin(n, K), torch.randn(r, K, generator=g) * 0.03,
                                                 torch.randn(n, r, generator=g) * 0.03, ALPHA))
        getattr(attn, name).base_layer.to(dtype=torch.bfloat16)
    layer.self_attn = attn
    m.model.layers = nn.ModuleList([layer])
    m = m.to(gpu)
    mxfp8.enable_mxfp8(m)
    mods = [attn.q_proj, attn.k_proj, attn.v_proj]
    x = (torch.randn(T, K, generator=g)).to(torch.bfloat16).to(gpu)
    dys = [(torch.randn(T, n, generator=g) * 0.1).to(torch.bfloat16).to(gpu) for n in (NQ, NKV, NKV)]

    fused_linear.new_step()
    merged = [o.clone() for o in fused_linear.group_linear(x, mods)]
    saved = mxfp8.group_fwd_operand
    mxfp8.group_fwd_operand = lambda lins: None  # one GEMM per layer
    try:
        fused_linear.new_step()
        single = fused_linear.group_linear(x, mods)
    finally:
        mxfp8.group_fwd_operand = saved
    for u, v in zip(merged, single):
        assert torch.equal(u, v)

    def run():
        fused_linear.new_step()
        for p in m.parameters():
            p.grad = None
        xg = x.clone().requires_grad_(True)
        torch.autograd.backward(fused_linear.group_linear(xg, mods), dys)
        return xg.grad, [p.grad.clone() for p in m.parameters() if p.requires_grad]

    dxf, gf = run()
    for mod in mods:
        mod.base_layer._mx_fbwd = False
    dxp, gp = run()
    _close(dxf, dxp.double().cpu(), "dx")
    for k, (a, b) in enumerate(zip(gf, gp)):
        _close(a, b.double().cpu(), f"grad {k}")


def _qkv_grads(m, x, dys):
    return [x.grad] + [getattr(m.attn, n).lora_A["default"].weight.grad for n in ("q_proj", "k_proj", "v_proj")] + \
        [getattr(m.attn, n).lora_B["default"].weight.grad for n in ("q_proj", "k_proj", "v_proj")]


def test_backward_after_next_step_keeps_its_own_weights(gpu):
    """A graph whose backward runs after the next step's new_step(), in-place parameter update and forward (a
    retained graph, a deferred prefix backward) must use the weights of its own step, as the reference's per-step
    bf16 copies do, although the group's weight forms live in a buffer that each step repacks (fused_linear._PLANS:
    a pending reader makes the next step pack into a fresh buffer).  Reference: the same step 1 with its backward
    run at once.  Bit-identical gradients."""
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(T, K, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    dys = [(torch.randn(T, n, generator=g) * 1e-2).to(torch.bfloat16).to(gpu) for n in (NQ, NKV, NKV)]
    names = ("q_proj", "k_proj", "v_proj")

    def forward(m):
        xx = x.clone().requires_grad_(True)
        return xx, fused_linear.group_linear(xx, [getattr(m.attn, n) for n in names])

    def bump(m):  # an optimizer step: every adapter parameter changes in place, at the same address
        with torch.no_grad():
            for n in names:
                for p in (getattr(m.attn, n).lora_A["default"].weight, getattr(m.attn, n).lora_B["default"].weight):
                    p.mul_(1.5).add_(0.01)

    m, _ = _build(gpu, seed=3)
    xx, outs = forward(m)
    torch.autograd.backward(list(outs), dys)
    torch.cuda.synchronize()
    want = [t.clone() for t in _qkv_grads(m, xx, dys)]

    m, _ = _build(gpu, seed=3)
    xx, outs = forward(m)       # step 1
    fused_linear.new_step()
    bump(m)
    xx2, outs2 = forward(m)     # step 2 packs its forms while step 1's backward is pending
    for n in names:
        for p in (getattr(m.attn, n).lora_A["default"].weight, getattr(m.attn, n).lora_B["default"].weight):
            p.grad = None
    torch.autograd.backward(list(outs), dys)  # step 1's backward
    torch.cuda.synchronize()
    got = _qkv_grads(m, xx, dys)
    for k, (a, b) in enumerate(zip(got, want)):
        assert a is not None and torch.equal(a, b), k
    del outs2, xx2


@pytest.mark.parametrize("names", [("q_proj", "k_proj", "v_proj"), ("o_proj",)])
def test_group_backward_with_and_without_the_dx_fold(names, gpu, monkeypatch):
    """The grouped backward's dA = dSᵀ·x2 in its dx GEMM's launch (fused_linear.FOLD_TN: mxfp8_gemm_nt_tn with the
    rank-48 epilogue and a rank-64 reduction at q|k|v, rank 16 and 16 at o_proj) against its own launch after the
    GEMM: bit-identical dx and LoRA gradients, and the folded entry point called once per backward."""
    import mxfp8
    m, _ = _build(gpu, seed=5)
    mods = [getattr(m.attn, n) for n in names]
    g = torch.Generator().manual_seed(17)
    x = (torch.randn(T, mods[0].base_layer.in_features, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    dys = [(torch.randn(T, mod.base_layer.out_features, generator=g) * 1e-2).to(torch.bfloat16).to(gpu)
           for mod in mods]
    calls = []
    real = mxfp8.mx_mm_tn
    monkeypatch.setattr(mxfp8, "mx_mm_tn", lambda *a, **k: calls.append(1) or real(*a, **k))

    def run(fold):
        monkeypatch.setattr(fused_linear, "FOLD_TN", [fold])
        fused_linear.new_step()
        for p in m.parameters():
            p.grad = None
        xg = x.clone().requires_grad_(True)
        outs = fused_linear.group_linear(xg, mods)
        torch.autograd.backward(list(outs), dys)
        torch.cuda.synchronize()
        return [xg.grad] + [p.grad.clone() for mod in mods
                            for p in (mod.lora_A["default"].weight, mod.lora_B["default"].weight)]

    off = run(False)
    assert not calls
    on = run(True)
    assert len(calls) == 1
    for k, (a, b) in enumerate(zip(on, off)):
        assert a is not None and torch.equal(a, b), k
