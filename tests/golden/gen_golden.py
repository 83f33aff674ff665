"""Writes tests/golden/c1_golden.npz and c1_golden.json from the CPU oracle (oracle/), for configuration 1
(T=256, d_model 1024, d_ffn 3584, LoRA r16 alpha 32) and a table of known-answer blocks.

The reference ships no vectors for this path and cannot run here (Triton + torchao + NVIDIA PTX), so these
fixtures are the oracle's outputs, which tests/test_oracle_quant.py pins against exact arithmetic and an
independent encoder; they serve as a regression pin for the oracle and as committed data the GPU tests
compare with.  Run from the repo root:  python tests/golden/gen_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "train-model-template_amd"))

import workloads  # noqa: E402
from oracle import mlp as omlp  # noqa: E402
from oracle import mx  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def sha(t):
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def kat_blocks():
    vals = [[448.0 * 2.0 ** k] + [0.5 * 2.0 ** k] * 31 for k in range(-20, 21)]
    vals += [[0.0] * 32, [-0.0] * 32, [448.0, 17.0, 19.0, 2.0 ** -10, 3 * 2.0 ** -10, -17.0] + [0.0] * 26,
             [float("inf"), 2.0 ** 127] + [0.0] * 30, [1.0, float("nan")] + [1.0] * 30, [450.0] + [1.0] * 31,
             [2.0 ** -120] + [0.0] * 31, [3.0e38] + [1.0] * 31]
    x = torch.zeros(len(vals), 128)
    for i, v in enumerate(vals):
        x[i, :32] = torch.tensor(v)
        x[i, 32:] = torch.linspace(-3, 3, 96)
    return x.to(torch.bfloat16)


def main():
    out, meta = {}, {}
    kx = kat_blocks()
    kq, ks = mx.quant(kx)
    out.update(kat_x=kx.view(torch.int16).numpy(), kat_q=kq.numpy(), kat_s=ks.numpy())
    inp = workloads.make_inputs(1)
    q, s = mx.quant(inp["x"])
    out.update(c1_xq_head=q[:16].numpy(), c1_xs=s.numpy())
    meta["c1_xq_sha256"] = sha(q)
    W = omlp.prepare_weights(inp["Wg"], inp["Wu"], inp["Wd"])
    for k in ("w", "ws", "wt", "wts", "dw", "dws", "dwt", "dwts"):
        meta[f"c1_W_{k}_sha256"] = sha(W[k])
    S, bg, bu, ad, bd = omlp.lora_cast(inp["Ag"], inp["Bg"], inp["Au"], inp["Bu"], inp["Ad"], inp["Bd"])
    f = omlp.forward(inp["x"], W, S, bg, bu, ad, bd, inp["s"], inp["s"], inp["s"])
    out.update(c1_y_head=f["y"][:16].view(torch.int16).numpy(), c1_xsd_head=f["xsd"][:16].view(torch.int16).numpy())
    meta["c1_hq_sha256"] = sha(f["qh"])
    meta["c1_hs_sha256"] = sha(f["sh"])
    meta["note"] = "oracle outputs for configuration 1; y / xsd compared within tolerance, codes bit-exact"
    np.savez_compressed(os.path.join(HERE, "c1_golden.npz"), **out)
    with open(os.path.join(HERE, "c1_golden.json"), "w") as fh:
        json.dump(meta, fh, indent=1, sort_keys=True)
    print("wrote", sorted(out), sorted(meta))


if __name__ == "__main__":
    main()
