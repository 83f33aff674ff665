"""GPU check that a whole fused MLP training step can be captured into a HIP graph and replayed: the forward and
backward of fused_mlp.mlp (the reference's _MLP autograd function, /root/reference/scripts/fused_mlp.py:262-366),
with the per-step LoRA casts, the quantizers, the four MX GEMMs (the down GEMM records its summing path as two
launches under capture), the backward kernel and the token reductions.  Each replay runs on new inputs copied into
the captured buffers, with eager steps of the same inputs between the replays; the replay's output, dx and every
LoRA gradient must be bit-identical to the eager step's."""
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
