"""GPU checks that whole training steps can be captured into a HIP graph and replayed.  The fused MLP: the forward and
backward of fused_mlp.mlp (the reference's _MLP autograd function, /root/reference/scripts/fused_mlp.py:262-366),
with the per-step LoRA casts, the quantizers, the four MX GEMMs (the down GEMM records its summing path as two
launches under capture), the backward kernel and the token reductions.  Each replay runs on new inputs copied into
the captured buffers, with eager steps of the same inputs between the replays; the replay's output, dx and every
LoRA gradient must be bit-identical to the eager step's.  The same for the grouped attention projections (q|k|v
as one group, o_proj deferred into residual_add)."""
import pytest
import torch

import fused_linear
import fused_mlp
import mxfp8
import workloads

pytestmark = pytest.mark.gpu


def _lora(mod):
    return [mod.gate_proj.lora_A["default"].weight, mod.gate_proj.lora_B["default"].weight,
            mod.up_proj.lora_A["default"].weight, mod.up_proj.lora_B["default"].weight,
            mod.down_proj.lora_A["default"].weight, mod.down_proj.lora_B["default"].weight]


def _eager(mod, x, dy):
    fused_linear.new_step()
    for p in _lora(mod):
        p.grad = None
    xi = x.clone().requires_grad_(True)
    y = fused_mlp.mlp(mod, xi)
    y.backward(dy)
    torch.cuda.synchronize()
    return [y.detach().clone(), xi.grad.clone()] + [p.grad.clone() for p in _lora(mod)]


@pytest.mark.parametrize("T", [1000, 2048])
def test_mlp_step_replayed_from_a_hip_graph(T, gpu):
    model, inps = workloads.build_model(3, T=T, device=gpu)
    mxfp8.enable_mxfp8(model)
    mod = model.layers[0].mlp
    x0, dy0 = inps[0]["x"].to(gpu), inps[0]["dy"].to(gpu)
    sx = x0.clone().requires_grad_(True)
    sdy = dy0.clone()

    def step():
        fused_linear.new_step()
        for p in _lora(mod):
            p.grad = None
        sx.grad = None
        y = fused_mlp.mlp(mod, sx)
        y.backward(sdy)
        return y

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    for p in _lora(mod):
        p.grad = None
    sx.grad = None
    with torch.cuda.graph(graph):
        sy = step()
    static = [sy, sx.grad] + [p.grad for p in _lora(mod)]
    assert all(t is not None for t in static)

    g = torch.Generator(device=gpu).manual_seed(T)
    for it in range(3):
        x = (torch.randn(x0.shape, device=gpu, generator=g) * (1 + it)).to(x0.dtype)
        dy = (torch.randn(dy0.shape, device=gpu, generator=g) * 1e-2).to(dy0.dtype)
        with torch.no_grad():
            sx.copy_(x)
        sdy.copy_(dy)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [t.detach().clone() for t in static]
        ref = _eager(mod, x, dy)  # eager work between the replays
        for k, (a, b) in enumerate(zip(got, ref)):
            assert torch.equal(a, b), (it, k)
    del graph


def _attn_params(a):
    return [getattr(a, n).lora_A["default"].weight for n in ("q_proj", "k_proj", "v_proj", "o_proj")] + \
        [getattr(a, n).lora_B["default"].weight for n in ("q_proj", "k_proj", "v_proj", "o_proj")]


@pytest.mark.parametrize("T", [1000, 2048])
def test_attention_projection_step_replayed_from_a_hip_graph(T, gpu):
    """The grouped linears (fused_linear.group_linear, /root/reference/scripts/fused_linear.py:79-330): q|k|v as
    one group, o_proj deferred into residual_add, forward and backward, captured into a HIP graph (the per-step
    weight forms' pack, the quantizers, the merged and per-layer MX GEMMs, lora_bwd, the dx GEMMs with dA in their
    launches, the residual epilogue) and replayed three times on new inputs, with eager steps between the replays:
    outputs, dx and every LoRA gradient bit-identical to the eager step's."""
    K, nq, nkv = 1024, 1024, 256
    m = workloads.build_attn(K, nq, nkv, 16, 32.0, device=gpu, seed=23)
    mxfp8.enable_mxfp8(m)
    a = m.model.layers[0].self_attn
    params = _attn_params(a)
    g = torch.Generator(device=gpu).manual_seed(T + 1)
    sx = torch.randn(T, K, device=gpu, generator=g).to(torch.bfloat16).requires_grad_(True)
    sres = torch.randn(T, K, device=gpu, generator=g).to(torch.bfloat16)
    sdy = [(torch.randn(T, n, device=gpu, generator=g) * 1e-2).to(torch.bfloat16) for n in (K, nkv, nkv)]

    def step(x, res, dys):
        fused_linear.new_step()
        for p in params:
            p.grad = None
        x.grad = None
        q, k, v = fused_linear.group_linear(x, [a.q_proj, a.k_proj, a.v_proj])
        (o,) = fused_linear.group_linear(q, [a.o_proj], defer=True)
        out = fused_linear.residual_add(res, o)
        torch.autograd.backward([out, k, v], dys)
        return [out, k, v]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step(sx, sres, sdy)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    for p in params:
        p.grad = None
    sx.grad = None
    with torch.cuda.graph(graph):
        souts = step(sx, sres, sdy)
    static = [t.detach() for t in souts] + [sx.grad] + [p.grad for p in params]
    assert all(t is not None for t in static)

    for it in range(3):
        x = (torch.randn(T, K, device=gpu, generator=g) * (1 + it)).to(torch.bfloat16)
        res = torch.randn(T, K, device=gpu, generator=g).to(torch.bfloat16)
        dys = [(torch.randn(T, n, device=gpu, generator=g) * 1e-2).to(torch.bfloat16) for n in (K, nkv, nkv)]
        with torch.no_grad():
            sx.copy_(x)
        sres.copy_(res)
        for s, d in zip(sdy, dys):
            s.copy_(d)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [t.detach().clone() for t in static]
        xe = x.clone().requires_grad_(True)  # eager work between the replays
        outs = step(xe, res, dys)
        torch.cuda.synchronize()
        ref = [t.detach() for t in outs] + [xe.grad] + [p.grad for p in params]
        for k, (u, w) in enumerate(zip(got, ref)):
            assert torch.equal(u, w), (it, k)
    del graph
