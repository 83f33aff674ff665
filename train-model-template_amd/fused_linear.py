"""The part of /root/reference/scripts/fused_linear.py that the fused MLP path depends on (fused_linear.py:26-69):
the PEFT LoRA-part extraction `_part`, the per-step bf16 cast cache `_cast` / `new_step`, and `STATS`.

The grouped LoRA linears of the attention / DeltaNet projections (fused_linear.py:72-330) are not part of
this library.
"""
import torch
from torch import nn

STATS = {"gộp": 0, "gọi thẳng": 0}  # path counters, same keys as the reference (fused / called directly)


def _part(m):
    """(base Linear, A, B, scaling) of a PEFT LoRA Linear; (m, None, None, 1.0) for a plain frozen Linear;
    None if the layer cannot take the fused path (fused_linear.py:30-48)."""
    base = getattr(m, "base_layer", None)
    if base is None:
        if type(m) is nn.Linear and m.bias is None and not m.weight.requires_grad:
            return m, None, None, 1.0
        return None
    if base.bias is not None or base.weight.requires_grad or m.merged or m.disable_adapters:
        return None
    ads = [a for a in m.active_adapters if a in m.lora_A]
    if len(ads) != 1:
        return None
    a = ads[0]
    drop = m.lora_dropout[a]
    if (a in getattr(m, "lora_variant", {}) or m.use_dora.get(a, False) or m.lora_B[a].bias is not None
            or not (isinstance(drop, nn.Identity) or getattr(drop, "p", 1) == 0)):
        return None
    return base, m.lora_A[a].weight, m.lora_B[a].weight, m.scaling[a]


# bf16 copies of the LoRA A/B parameters (fp32) and the concatenated S matrix, made once per training step
# instead of at every call.  The optimizer may update parameters in place without bumping _version, so the
# step driver calls new_step() at the start of each step (fused_linear.py:55-62).
_CAST = {}


def new_step():
    _CAST.clear()


def _cast(key, make):
    t = _CAST.get(key)
    if t is None:
        t = _CAST[key] = make()
    return t
