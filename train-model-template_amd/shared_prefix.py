"""The MLP step of the training script's decoder layer (/root/reference/scripts/shared_prefix.py:172-197): the fused
MXFP8 MLP when gate/up are paired (fused_mlp.mlp), otherwise the unfused path group_linear(gate, up) -> SwiGLU ->
group_linear(down).  The unfused path is also the cross-check of the fused one: its h = bf16(silu(g)·u) is computed
with the same sigmoid and rounding, so the codes of MX(h) agree (fused_mlp.py:67-68).  Only this function of the
script is part of the library; attention, DeltaNet and the training loop are not.
"""
import torch
import torch.nn.functional as F

from fused_linear import STATS, group_linear


def _swiglu_eager(g, u):
    return F.silu(g) * u


class _SwiGLU(torch.autograd.Function):
    """h = bf16(silu(g)·u) and its backward on the library's elementwise kernels (mxfp8_swiglu / _bwd): one rounding
    per output, as the reference's compiled _SWIGLU (shared_prefix.py:194-197)."""

    @staticmethod
    def forward(ctx, g, u):
        import _native
        g, u = g.contiguous(), u.contiguous()
        h = torch.empty_like(g)
        _native.swiglu(g, u, h)
        ctx.save_for_backward(g, u)
        return h

    @staticmethod
    def backward(ctx, dh):
        import _native
        g, u = ctx.saved_tensors
        dg, du = torch.empty_like(g), torch.empty_like(u)
        _native.swiglu_bwd(g, u, dh.contiguous(), dg, du)
        return dg, du


def _SWIGLU(g, u):
    """silu(g) * u: the HIP kernels for bf16 GPU tensors whose size the kernels take; other dtypes or devices follow
    the reference's eager definition (the same as the non-MX torch path of group_linear)."""
    if g.is_cuda and g.dtype == u.dtype == torch.bfloat16 and g.shape == u.shape and g.numel() % 8 == 0:
        return _SwiGLU.apply(g, u)
    return _swiglu_eager(g, u)


def _mlp(mlp, x, need_out=True):
    """down(silu(gate(x)) * up(x)) as a Qwen3.5 MLP (shared_prefix.py:179-197): the fused MXFP8 MLP when gate/up
    are paired by mxfp8.enable_mxfp8 and fused_mlp.mlp takes the shapes, else gate/up as one group_linear, SwiGLU,
    and down as a group_linear.  need_out=False: the down GEMM's output is not computed (see group_linear)."""
    if type(mlp.act_fn).__name__ not in ("SiLU", "SiLUActivation"):
        STATS["mlp gọi thẳng"] = STATS.get("mlp gọi thẳng", 0) + 1
        return mlp(x)
    if getattr(getattr(mlp.gate_proj, "base_layer", mlp.gate_proj), "_mx_gu", None) is not None:
        import fused_mlp
        y = fused_mlp.mlp(mlp, x, need_out)
        if y is not None:
            return y
    g, u = group_linear(x, (mlp.gate_proj, mlp.up_proj))
    return group_linear(_SWIGLU(g, u), (mlp.down_proj,), need_out)[0]
