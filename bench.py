"""Benchmark of the MXFP8 fused SwiGLU-MLP hot path on one MI355X.

One step = forward + backward of one Qwen3.5-2B-shaped LoRA MLP layer (configuration 3: 10,752 tokens,
d_model 2048, d_ffn 6144, LoRA r16 alpha 32) through the drop-in API the training script uses
(mxfp8.enable_mxfp8 once, then fused_mlp.mlp + backward), on synthetic seeded inputs already resident in HBM.

Prints one JSON line:
  value        MX GEMM work of the step (12·T·K·N flops; LoRA bf16 flops not counted) / step time, TFLOP/s
  roofline     the dominant kernel, the MX GEMM: its algorithmic flops / its launch time measured with HIP
               events on the launch stream over the timed steps, against the 5.0 PFLOP/s dense MXFP8 peak
  quantizer    mx_quant on the [T, K] activation and on a [T, 2N] buffer (back-to-back launches), GB/s of
               algorithmic bytes (read bf16, write codes + blocked scales) against 8 TB/s
  cpu_baseline the CPU oracle of the same path on a bounded token sample, on this host's cores
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "train-model-template_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

PEAK_MXFP8_TFLOPS = 5000.0  # MI355X dense MXFP8 (f8f6f4 MFMA) peak, public figure
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E peak
CFG = 3


def _traffic_from_profiles():
    """HBM bytes per GEMM launch from the committed rocprofv3 PMC summary (profiles/), or None."""
    p = os.path.join(ROOT, "profiles", "mx_gemm_c3_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("bytes_per_launch")


def _cpu_baseline(T_sample):
    """Oracle fwd+bwd of the same layer on T_sample tokens (1 warmup, median of 3), TFLOP/s."""
    import torch

    import workloads
    from oracle import mlp as omlp

    cores = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(cores)
    inp = workloads.make_inputs(CFG, T=T_sample)
    W = omlp.prepare_weights(inp["Wg"], inp["Wu"], inp["Wd"])
    S, bg, bu, ad, bd = omlp.lora_cast(inp["Ag"], inp["Bg"], inp["Au"], inp["Bu"], inp["Ad"], inp["Bd"])
    s = inp["s"]

    def step():
        f = omlp.forward(inp["x"], W, S, bg, bu, ad, bd, s, s, s)
        omlp.backward(inp["x"], f["xs"], f["gu"], W, S, bg, bu, ad, bd, s, s, s, inp["dy"])

    step()
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        step()
        ts.append(time.perf_counter() - t0)
    t = sorted(ts)[1]
    fl = workloads.flops(T_sample, inp["K"], inp["N"])
    return {"value": round(fl / t / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"oracle fwd+bwd of the config-3 layer on {T_sample} of its 10752 tokens (median of 3 after "
                      f"1 warmup, {t:.2f} s per step; weight preparation excluded as on the GPU)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-tokens", type=int, default=1024)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the MLP shards by tokens with "
              "one LoRA-gradient all-reduce per layer; see DESIGN.md).", file=sys.stderr)
        sys.exit(2)

    import torch

    import fused_linear
    import fused_mlp
    import mxfp8
    import workloads

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    c = workloads.CONFIGS[CFG]
    model, inps = workloads.build_model(CFG, device=dev)
    mxfp8.enable_mxfp8(model)
    mod = model.layers[0].mlp
    inp = inps[0]
    T, K, N = inp["T"], inp["K"], inp["N"]
    x = inp["x"].to(dev).requires_grad_(True)
    dy = inp["dy"].to(dev)
    params = [p for p in mod.parameters() if p.requires_grad]

    def step():
        fused_linear.new_step()
        for p in params:
            p.grad = None
        x.grad = None
        y = fused_mlp.mlp(mod, x)
        y.backward(dy)

    assert fused_mlp.mlp(mod, x) is not None, "fused path not taken"
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    mxfp8.GEMM_EVENTS = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev = mxfp8.GEMM_EVENTS
    mxfp8.GEMM_EVENTS = None
    # untimed instrumented-event overhead is inside the wall time; report it anyway as measured
    gemm_ms = sum(a.elapsed_time(b) for a, b, _ in ev)
    gemm_fl = sum(f for _, _, f in ev)
    ms = wall * 1e3 / args.steps
    fl = workloads.flops(T, K, N)
    value = fl / (ms * 1e-3) / 1e12
    gemm_tf = gemm_fl / (gemm_ms * 1e-3) / 1e12
    traffic = _traffic_from_profiles()

    # quantizer: back-to-back launches over >= 1 ms
    quant = {}
    for name, shape in (("x[T,K]", (T, K)), ("dgu[T,2N]", (T, 2 * N))):
        src = torch.randn(shape, device=dev).to(torch.bfloat16)
        n = 200 if shape[1] == K else 40
        for _ in range(5):
            mxfp8.mx_quant(src)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(n):
            mxfp8.mx_quant(src)
        e1.record()
        torch.cuda.synchronize()
        qms = e0.elapsed_time(e1) / n
        by = workloads.quant_bytes(*shape)
        quant[name] = {"GB/s": round(by / (qms * 1e-3) / 1e9, 1), "us": round(qms * 1e3, 2), "bytes": by,
                       "frac": round(by / (qms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
        del src

    line = {
        "metric": "MXFP8 MLP fwd+bwd TFLOP/s (% MXFP8 peak); quantizer GB/s (% of HBM)",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp8",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights and LoRA A/B, N(0,1e-2) upstream grad)",
        "config": {"workload": workloads.DESCRIPTIONS[CFG], "tokens": T, "d_model": K, "d_ffn": N,
                   "lora_r": c["r"], "lora_alpha": c["alpha"], "frac_of_mxfp8_peak": round(value / PEAK_MXFP8_TFLOPS, 4)},
        "roofline": {"bound": "mfma", "achieved": round(gemm_tf, 2), "peak": PEAK_MXFP8_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(gemm_tf / PEAK_MXFP8_TFLOPS, 4), "traffic": traffic,
                     "kernel": "mx_gemm (4 launches per step: gate|up, down, dh, dx)",
                     "launches": len(ev), "kernel_ms_per_step": round(gemm_ms / args.steps, 4)},
        "quantizer": quant,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = _cpu_baseline(args.cpu_tokens)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
