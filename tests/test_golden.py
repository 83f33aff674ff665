"""The committed golden fixtures (tests/golden/, written by gen_golden.py from the oracle): the oracle must keep
reproducing them (CPU), and the HIP path must match them (GPU): codes/scales bit-exact, y within the stated
tolerance."""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

import workloads

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
G = np.load(os.path.join(HERE, "c1_golden.npz"))
META = json.load(open(os.path.join(HERE, "c1_golden.json")))
TOL = 2e-2


def sha(t):
    return hashlib.sha256(t.contiguous().view(torch.uint8).cpu().numpy().tobytes()).hexdigest()


def _bf16(a):
    return torch.from_numpy(a).view(torch.bfloat16)


def test_oracle_reproduces_golden():
    from oracle import mlp as omlp
    from oracle import mx
    kq, ks = mx.quant(_bf16(G["kat_x"]))
    assert np.array_equal(kq.numpy(), G["kat_q"]) and np.array_equal(ks.numpy(), G["kat_s"])
    inp = workloads.make_inputs(1)
    q, s = mx.quant(inp["x"])
    assert sha(q) == META["c1_xq_sha256"] and np.array_equal(s.numpy(), G["c1_xs"])
    W = omlp.prepare_weights(inp["Wg"], inp["Wu"], inp["Wd"])
    for k in ("w", "ws", "wt", "wts", "dw", "dws", "dwt", "dwts"):
        assert sha(W[k]) == META[f"c1_W_{k}_sha256"], k
    S, bg, bu, ad, bd = omlp.lora_cast(inp["Ag"], inp["Bg"], inp["Au"], inp["Bu"], inp["Ad"], inp["Bd"])
    f = omlp.forward(inp["x"], W, S, bg, bu, ad, bd, inp["s"], inp["s"], inp["s"])
    ref = _bf16(G["c1_y_head"]).float()
    assert ((f["y"][:16].float() - ref).abs() <= ref.abs() * 2.0 ** -7 + 1e-6).all()


@pytest.mark.gpu
def test_gpu_matches_golden(gpu):
    import fused_linear
    import fused_mlp
    import mxfp8
    kq, ks = mxfp8.mx_quant(_bf16(G["kat_x"]).to(gpu))
    assert np.array_equal(kq.view(torch.uint8).cpu().numpy(), G["kat_q"])
    assert np.array_equal(ks.view(torch.uint8).cpu().numpy(), G["kat_s"])
    inp = workloads.make_inputs(1)
    q, s = mxfp8.mx_quant(inp["x"].to(gpu))
    assert sha(q) == META["c1_xq_sha256"] and np.array_equal(s.view(torch.uint8).cpu().numpy(), G["c1_xs"])
    Wgu = torch.cat([inp["Wg"], inp["Wu"]]).to(gpu)
    w, ws, wt, wts = mxfp8.quant_both(Wgu)
    dw, dws, dwt, dwts = mxfp8.quant_both(inp["Wd"].to(gpu))
    for k, t in dict(w=w, ws=ws, wt=wt, wts=wts, dw=dw, dws=dws, dwt=dwt, dwts=dwts).items():
        assert sha(t) == META[f"c1_W_{k}_sha256"], k
    model, inps = workloads.build_model(1, device=gpu)
    mxfp8.enable_mxfp8(model)
    fused_linear.new_step()
    y = fused_mlp.mlp(model.layers[0].mlp, inps[0]["x"].to(gpu))
    ref = _bf16(G["c1_y_head"]).float()
    err = (y[:16].float().cpu() - ref).abs().max() / ref.abs().max()
    assert err <= TOL, err
