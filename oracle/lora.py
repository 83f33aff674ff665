"""CPU oracle of the LoRA epilogues next to the MLP path (test infrastructure only; see oracle/__init__.py).

  res_lora   -- out = bf16(x + bf16(y + scale * xa @ Bᵀ))       (/root/reference/scripts/mxfp8.py:265-293)
  lora_bwd   -- d(xa) = bf16(scale * dy @ B), dB = scale * dyᵀ @ xa (fp32), codes of dy via mx.quant_into
                                                                  (/root/reference/scripts/mxfp8.py:89-262)

Pinned by tests/test_oracle_lora.py against closed forms (B = 0, scale = 0, exactly representable integer products,
the transpose relation between the two products) and known-answer cases where rounding at another point (once
instead of twice; before instead of after the scale) gives a different result.
"""
import torch


def res_lora(x, y, xa, B, scale):
    """mxfp8.py:271-282: acc = xa @ Bᵀ in fp32; t = bf16(y + scale * acc); out = bf16(x + t).  x, y [T, N] bf16,
    xa [T, r] bf16, B [N, r] bf16 (CPU tensors).  The product is taken in float64 and rounded to fp32 once, which
    bounds the difference from any fp32 summation order by the fp32 rounding of the sum."""
    acc = (xa.double() @ B.double().t()).float()
    t = (y.float() + scale * acc).to(torch.bfloat16)
    return (x.float() + t.float()).to(torch.bfloat16)


def lora_bwd(dy, xa, B, scale):
    """mxfp8.py:146-176 (_lora_bwd_kernel) with _sum_rows (:180-190): d = dy @ B in fp32, d(xa) = bf16(d * scale)
    ([T, r] bf16); dB = (dyᵀ @ xa in fp32) * scale ([N, r] fp32).  dy [T, N], xa [T, r], B [N, r] bf16 on the CPU.
    Products in float64 rounded to fp32 once (the reference adds fp32 partials in a fixed order; any fp32 order
    differs from this by the fp32 rounding of the sum).  The MX codes of dy are mx.quant_into's."""
    d = (dy.double() @ B.double()).float()
    dxa = (d * scale).to(torch.bfloat16)
    dB = (dy.double().t() @ xa.double()).float() * scale
    return dxa, dB
