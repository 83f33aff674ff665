"""Benchmark of the MXFP8 fused SwiGLU-MLP hot path on one MI355X.

One step = forward + backward through the drop-in API the training script uses (mxfp8.enable_mxfp8 once, then
fused_mlp.mlp per layer + backward), on synthetic seeded inputs already resident in HBM:
  --config 3 (default, the headline): one Qwen3.5-2B-shaped LoRA MLP layer, 10,752 tokens, d_model 2048,
             d_ffn 6144, LoRA r16 alpha 32;
  --config 4: a stack of 24 such layers at 142,336 tokens on a residual stream, x <- x + mlp(rms_norm(x)), as
             the reference decoder runs each MLP (shared_prefix.py:239, :252; torch's RMSNorm with unit weight
             for post_attention_layernorm).  The norms and adds are torch kernels inside the step; without them
             the stream vanishes (y = mlp(y)) or overflows (y = y + mlp(y));
  --config 5: configuration 3's shape on the outlier inputs (Student-t activations with edge blocks).

Prints one JSON line:
  value        MX GEMM work of the step (12·T·K·N flops per layer; LoRA bf16 flops not counted) / step time
  roofline     the dominant kernel, the MX GEMM: its algorithmic flops / its launch time measured with HIP
               events on the launch stream over K more steps run right after the timed ones (an event record
               idles the GPU for a few microseconds beside the kernel it brackets, so the K steps of `value`
               carry no events), against the 5.0 PFLOP/s dense MXFP8 peak; traffic = HBM bytes per GEMM launch
               from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
  quantizer    mx_quant on the [T, K] activation and on a [T, 2N] buffer, the quantizer the MLP step runs
               (quant_lora: MX codes + the rank-r product of x with S and of dy with B_d), and the dual-axis
               preparation of the frozen weights (quant_both on W_gate|up and W_down): a HIP graph of
               back-to-back launches covering >= 1 ms, GB/s of algorithmic bytes (read bf16, write codes +
               blocked scales, plus the rank-r operands and products) against 8 TB/s
  with_requant the step plus the dual-axis weight preparation of every layer
  cpu_baseline the CPU oracle of the same layer on a bounded token sample, on this host's cores

Profiling helpers (same file, so every profile names committed code only):
  --copy-calib           also run a plain 1 GiB bf16 copy kernel (torch.neg, read 1 GiB + write 1 GiB) three
                         times, so a rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE run can scale its counters
  --traffic-summary F W  read two rocprofv3 --pmc output directories (FETCH_SIZE run, WRITE_SIZE run) and write
                         profiles/mx_gemm_c<cfg>_traffic.json + .md (no GPU needed)
"""
import argparse
import csv
import glob
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "train-model-template_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

PEAK_MXFP8_TFLOPS = 5000.0  # MI355X dense MXFP8 (f8f6f4 MFMA) peak, public figure
WARMUP_FLOOR_S = 0.3  # least wall time of untimed warmup steps before the timed ones
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E peak
COPY_CALIB_BYTES = 1 << 30  # bytes read (and written) by one --copy-calib launch
N_XCD = 8                   # accelerator complex dies of an MI355X (GRBM_GUI_ACTIVE counts on each)


def _traffic_path(cfg, ext):
    return os.path.join(ROOT, "profiles", f"mx_gemm_c{cfg}_traffic.{ext}")


def _traffic_from_profiles(cfg):
    """HBM bytes per GEMM launch from the committed rocprofv3 PMC summary (profiles/), or None."""
    p = _traffic_path(cfg, "json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("bytes_per_launch")


def _cpu_baseline(cfg, T_sample):
    """Oracle fwd+bwd of one layer of the configuration on T_sample tokens (1 warmup, median of 3), TFLOP/s."""
    import torch

    import workloads
    from oracle import mlp as omlp

    cores = len(os.sched_getaffinity(0))  # every core this process may run on
    torch.set_num_threads(cores)
    inp = workloads.make_inputs(cfg, T=T_sample)
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
    c = workloads.CONFIGS[cfg]
    what = f"one layer of configuration {cfg} on {T_sample} of its {c['T']} tokens"
    if c["layers"] > 1:
        what += f" (the stack is {c['layers']} such layers; the per-token rate is the same)"
    return {"value": round(fl / t / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"oracle fwd+bwd of {what}, median of 3 after 1 warmup, {t:.2f} s per step; weight "
                      f"preparation excluded as on the GPU"}


def _time_launches(fn, n):
    import torch
    for _ in range(3):
        fn()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(n):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n


def _time_graph(fn, min_ms=1.0, reps=5):
    """Mean time of one fn() in ms, fn launching GPU work only (outputs preallocated): n back-to-back calls are
    captured in one HIP graph, with n chosen from a first timing so that a replay covers >= min_ms, and the
    median of `reps` replays is divided by n.  A replay has no host gaps between the launches, so a kernel
    shorter than its Python call is timed by itself.  fn must not record memsets (none of the timed entry
    points does)."""
    import torch
    fn()
    torch.cuda.synchronize()
    one = _time_launches(fn, 20)
    n = max(10, int(min_ms / max(one, 1e-3)) + 1)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(g):
        for _ in range(n):
            fn()
    # untimed replays first (>= 10 ms), so the first entry timed in a process does not pay for the clock ramp
    # from idle (measured: the first of several quantizer timings ran 2% slower than the same kernel later)
    for _ in range(max(1, int(10.0 / max(one * n, 1e-3)) + 1)):
        g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    del g
    return sorted(ts)[reps // 2] / n, n


def _rate(by, ms, n):
    gbs = by / (ms * 1e-3) / 1e9
    return {"GB/s": round(gbs, 1), "us": round(ms * 1e3, 2), "bytes": by, "frac": round(gbs / PEAK_HBM_GBS, 4),
            "launches": n}


def _quantizer(T, K, N, dev):
    import torch

    import _native
    import mxfp8
    import workloads
    out = {}
    for name, shape in (("x[T,K]", (T, K)), ("dgu[T,2N]", (T, 2 * N))):
        src = torch.randn(shape, device=dev).to(torch.bfloat16)
        q = torch.empty(shape, dtype=torch.uint8, device=dev)
        sc = torch.empty(mxfp8.scale_numel(*shape), dtype=torch.uint8, device=dev)
        ms, n = _time_graph(lambda: _native.quant_rows(src, q, sc))
        out[name] = _rate(workloads.quant_bytes(*shape), ms, n)
        del src, q, sc
    # the quantizer the MLP step runs: MX codes (tiled) + xs = x·Sᵀ (2r = 32 rows) in the forward, MX codes +
    # dxd = bf16(bf16(dy·B_d)·s_d) (r = 16) with its zero-padded transpose in the backward
    x = torch.randn((T, K), device=dev).to(torch.bfloat16)
    q = torch.empty((mxfp8.tiled_rows(T), K), dtype=torch.uint8, device=dev)
    sc = torch.empty(mxfp8.scale_numel(T, K), dtype=torch.uint8, device=dev)
    for name, rp, with_t in (("quant_lora x[T,K] rp32", 32, False), ("quant_lora dy[T,K] rp16 +T", 16, True)):
        w = (torch.randn((rp, K), device=dev) * 0.02).to(torch.bfloat16)
        o = torch.empty((T, rp), dtype=torch.bfloat16, device=dev)
        oT = torch.empty((rp, -(-T // 128) * 128), dtype=torch.bfloat16, device=dev) if with_t else None
        ms, n = _time_graph(lambda: _native.quant_lora(x, q, sc, w, o, scale=2.0, outT=oT))
        by = workloads.quant_lora_bytes(T, K, rp, with_t)
        out[name] = _rate(by, ms, n)
        del w, o, oT
    del x, q, sc
    wq_ms = 0.0
    for name, shape in (("W_gate|up dual[2N,K]", (2 * N, K)), ("W_down dual[K,N]", (K, N))):
        w = (torch.randn(shape, device=dev) * 0.02).to(torch.bfloat16)
        R, C = shape
        q, qt = torch.empty((R, C), dtype=torch.uint8, device=dev), torch.empty((C, R), dtype=torch.uint8, device=dev)
        sq = torch.empty(mxfp8.scale_numel(R, C), dtype=torch.uint8, device=dev)
        st = torch.empty(mxfp8.scale_numel(C, R), dtype=torch.uint8, device=dev)
        ms, n = _time_graph(lambda: _native.quant_dual(w, q, sq, qt, st))
        out[name] = _rate(workloads.quant_bytes(*shape, dual=True), ms, n)
        wq_ms += ms
        del w, q, qt, sq, st
    return out, wq_ms


def _time_calls_gpu(fn, n):
    """Mean GPU time of fn() in ms: an event pair around each call, so host-side gaps between calls (the Python
    wrapper of a ~20 us kernel pair takes about as long) are not counted."""
    import torch
    for _ in range(3):
        fn()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    torch.cuda.synchronize()
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in ev) / n


def _lora_epilogues(T, K, N, r, dev):
    """The LoRA epilogues beside the MLP (mxfp8.lora_bwd, mxfp8.res_lora) at the workload's token count: GPU time
    per call (events around each call), algorithmic bytes over it."""
    import torch

    import mxfp8
    import workloads
    g = torch.Generator(device=dev).manual_seed(7)
    out = {}

    def rec(name, ms, by):
        out[name] = {"GB/s": round(by / (ms * 1e-3) / 1e9, 1), "us": round(ms * 1e3, 2), "bytes": by,
                     "frac": round(by / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}

    for cols in (K, N):
        dy = torch.randn(T, cols, device=dev, generator=g).to(torch.bfloat16)
        xS = torch.randn(T, 2 * r, device=dev, generator=g).to(torch.bfloat16)
        B = (torch.randn(cols, r, device=dev, generator=g) * 0.02).to(torch.bfloat16)
        q = torch.empty(T, cols, dtype=mxfp8.F8, device=dev)
        s = torch.empty(mxfp8.scale_numel(T, cols), dtype=torch.uint8, device=dev)
        dS = torch.empty(T, 2 * r, dtype=torch.bfloat16, device=dev)
        ms = _time_calls_gpu(lambda: mxfp8.lora_bwd(dy, xS[:, :r], B, 2.0, q, s, 0, dS[:, :r]), 50)
        rec(f"lora_bwd+q dy[T,{cols}] r{r}", ms, workloads.lora_bwd_bytes(T, cols, r))
        del dy, q, s
    x = torch.randn(T, K, device=dev, generator=g).to(torch.bfloat16)
    y = torch.randn(T, K, device=dev, generator=g).to(torch.bfloat16)
    B = (torch.randn(K, r, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    ms = _time_calls_gpu(lambda: mxfp8.res_lora(x, y, xS[:, :r], B, 2.0), 50)
    rec(f"res_lora [T,{K}] r{r}", ms, workloads.res_lora_bytes(T, K, r))
    return out


def _grouped_linears(T, K, r, alpha, dev, steps=10):
    """Attention projections through fused_linear (q|k|v grouped with the concatenated Wᵀ, o_proj deferred into the
    residual add), forward + backward per step.  q 2048 and k, v 512 outputs for d_model 2048 (GQA shape).  FLOPs
    counted: the MX GEMMs only (forward x·Wᵀ and backward dx, 2·T·K·N each).  Timed eagerly (steps enqueued by
    Python and autograd, the figure a training loop without graphs sees) and as replays of the step captured into
    a HIP graph."""
    import torch

    import fused_linear
    import mxfp8
    import workloads
    nq, nkv = K, K // 4
    m = workloads.build_attn(K, nq, nkv, r, alpha, device=dev, seed=17)
    mxfp8.enable_mxfp8(m)
    a = m.model.layers[0].self_attn
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(T, K, device=dev, generator=g).to(torch.bfloat16).requires_grad_(True)
    # the residual stream takes no gradient here: its gradient is dy itself (residual_add passes it through), and
    # a leaf that required it would add a [T, K] copy into .grad per step (autograd copies a gradient that the
    # other branch still holds), which a decoder's residual stream, whose gradient flows on, never makes
    resid = torch.randn(T, K, device=dev, generator=g).to(torch.bfloat16)
    dy = (torch.randn(T, K, device=dev, generator=g) * 1e-2).to(torch.bfloat16)
    params = [p for p in m.parameters() if p.requires_grad]

    dk = (torch.randn(T, nkv, device=dev, generator=g) * 1e-2).to(torch.bfloat16)
    dv = (torch.randn(T, nkv, device=dev, generator=g) * 1e-2).to(torch.bfloat16)

    def step():
        fused_linear.new_step()
        q, k, v = fused_linear.group_linear(x, [a.q_proj, a.k_proj, a.v_proj])
        (o,) = fused_linear.group_linear(q, [a.o_proj], defer=True)  # q stands in for the attention output
        out = fused_linear.residual_add(resid, o)
        torch.autograd.backward([out, k, v], [dy, dk, dv])
        for p in params:
            p.grad = None
        x.grad = None

    for _ in range(3):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    before = fused_linear.STATS.get("lan ngược gộp", 0)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    assert fused_linear.STATS.get("lan ngược gộp", 0) - before == 2 * steps  # both groups took the fused backward
    fl = 2 * 2 * T * K * (nq + 2 * nkv) + 2 * 2 * T * nq * K
    # the same step captured into a HIP graph (warmed up on a side stream, as capture needs) and replayed: the
    # kernels' own pace, without the Python and autograd work that the eager step enqueues them with
    # (tests/test_gpu_graph.py checks replays bit for bit against eager steps)
    out = {"ms_per_step": round(ms, 4), "MX_GEMM_TFLOP/s": round(fl / (ms * 1e-3) / 1e12, 1)}
    try:  # a side figure: a failed capture is reported in the entry, never at the cost of the bench line
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        gms = e0.elapsed_time(e1) / steps
        out.update({"graph_ms_per_step": round(gms, 4), "graph_MX_GEMM_TFLOP/s": round(fl / (gms * 1e-3) / 1e12, 1)})
        del graph
    except RuntimeError as e:
        torch.cuda.synchronize()
        out["graph_error"] = str(e)[:200]
    del m, x, resid, dy
    return {**out,
            "shape": f"T={T} d_model={K} q={nq} k=v={nkv} o={nq}->{K} r={r}",
            "note": "fwd+bwd of q|k|v (one group) and o_proj (deferred, residual_add) on q; seeded upstream grads"}


def _unfused_mlp(T, K, N, r, dev, steps=10):
    """The unfused MLP path (shared_prefix._mlp with fused_mlp off: gate|up as one group_linear, the SwiGLU
    kernels, down as a group_linear), forward + backward per step on one configuration-3 layer, and the SwiGLU
    kernels alone on [T, N] (graph timing; algorithmic bytes: g, u read and h written forward, g, u, dh read and
    dg, du written backward).  FLOPs counted: the MX GEMMs only, 12·T·K·N as for the fused step."""
    import torch

    import _native
    import fused_mlp
    import mxfp8
    import shared_prefix
    import workloads
    g = torch.Generator(device=dev).manual_seed(11)
    G = torch.randn(T, N, device=dev, generator=g).to(torch.bfloat16)
    U = torch.randn(T, N, device=dev, generator=g).to(torch.bfloat16)
    D = (torch.randn(T, N, device=dev, generator=g) * 1e-2).to(torch.bfloat16)
    H, DG, DU = torch.empty_like(G), torch.empty_like(G), torch.empty_like(G)
    out = {}
    for name, fn, by in (("swiglu fwd [T,N]", lambda: _native.swiglu(G, U, H), 6 * T * N),
                         ("swiglu bwd [T,N]", lambda: _native.swiglu_bwd(G, U, D, DG, DU), 10 * T * N)):
        ms, n = _time_graph(fn)
        out[name] = _rate(by, ms, n)
    del G, U, D, H, DG, DU
    model, inps = workloads.build_model(3, T=T, layers=1, device=dev)
    mxfp8.enable_mxfp8(model)
    mlp = model.layers[0].mlp
    x = inps[0]["x"].to(dev).requires_grad_(True)
    dy = inps[0]["dy"].to(dev)
    params = [p for p in mlp.parameters() if p.requires_grad]

    def step():
        y = shared_prefix._mlp(mlp, x)
        y.backward(dy)
        for p in params:
            p.grad = None
        x.grad = None

    fused_mlp.ENABLED[0] = False
    try:
        before = fused_mlp.STATS.get("mlp gộp", 0)
        for _ in range(3):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        assert fused_mlp.STATS.get("mlp gộp", 0) == before  # the unfused path ran
    finally:
        fused_mlp.ENABLED[0] = True
    ms = e0.elapsed_time(e1) / steps
    del model, x, dy, params
    out["unfused step"] = {"ms_per_step": round(ms, 4), "MX_GEMM_TFLOP/s": round(12 * T * K * N / (ms * 1e-3) / 1e12, 1),
                           "note": "one configuration-3 layer through shared_prefix._mlp with the fused MLP off"}
    return out


def _copy_calib(dev):
    import torch
    src = torch.ones(COPY_CALIB_BYTES // 2, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def _pmc_rows(d):
    files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {d}")
    rows = []
    for f in files:
        with open(f) as fh:
            rows += list(csv.DictReader(fh))
    return rows


def _traffic_summary(cfg, fetch_dir, write_dir, cmd_fetch, cmd_write):
    """Per-dispatch FETCH_SIZE / WRITE_SIZE (KiB) of the MX GEMM launches, scaled by what the same counters read
    for the 1 GiB copy kernel; writes profiles/mx_gemm_c<cfg>_traffic.{json,md}."""
    import workloads
    c = workloads.CONFIGS[cfg]
    T, K, N, r = c["T"], c["K"], c["N"], c["r"]

    def per_dispatch(d, counter):
        vals = {}
        for row in _pmc_rows(d):
            if row["Counter_Name"] != counter:
                continue
            key = (row["Dispatch_Id"], row["Kernel_Name"], row.get("Grid_Size", ""))
            vals[key] = vals.get(key, 0.0) + float(row["Counter_Value"])
        return vals

    fetch, write = per_dispatch(fetch_dir, "FETCH_SIZE"), per_dispatch(write_dir, "WRITE_SIZE")

    def copy_kib(vals):
        v = [x for (_, name, _), x in vals.items() if "neg" in name]
        if not v:
            raise SystemExit("no copy-calibration dispatch (run bench.py with --copy-calib)")
        return sorted(v)[len(v) // 2]

    f_scale = (COPY_CALIB_BYTES / 1024) / copy_kib(fetch)
    w_scale = (COPY_CALIB_BYTES / 1024) / copy_kib(write)

    # the four GEMM shapes of one layer, told apart by kernel template (epilogue rank) and grid size
    shapes = {"gate|up": (T, 2 * N, K, 0), "down": (T, K, N, r), "dh": (T, N, K, 0), "dx": (T, K, 2 * N, 2 * r)}

    def gemm_groups(vals):
        g = {}
        for (_, name, grid), v in vals.items():
            if "gemm_kernel" not in name:
                continue
            m = re.search(r"(\w*gemm_kernel<[^>]*>)", name)
            g.setdefault((m.group(1) if m else name[:60], grid), []).append(v)
        return {k: (sum(v) / len(v), len(v)) for k, v in g.items()}

    gf, gw = gemm_groups(fetch), gemm_groups(write)
    rows = []
    for (name, grid), (kib, n) in sorted(gf.items()):
        fb = kib * 1024 * f_scale
        wb = gw.get((name, grid), (0.0, 0))[0] * 1024 * w_scale
        rows.append({"kernel": name, "grid": grid, "dispatches": n, "fetch_bytes": round(fb), "write_bytes": round(wb)})
    if not rows:
        raise SystemExit("no gemm_kernel dispatches in the PMC output")
    # algorithmic bytes of each shape: read both MX operands and their scales once, write the bf16 output,
    # read the rank-r LoRA operands of the epilogue; the gate|up launch, with the SwiGLU forward in its epilogue,
    # also reads xs and the LoRA-B / A_down rows and writes MX(h) (codes and scales) and the bf16 xS_down
    alg = {}
    for nm, (M, Nn, Kk, rr) in shapes.items():
        sc = lambda R, C: -(-R // 128) * (C // 128) * 512 // 4  # noqa: E731  (one scale per 32 along K)
        alg[nm] = M * Kk + Nn * Kk + sc(M, Kk) + sc(Nn, Kk) + M * Nn * 2 + (M + Nn) * rr * 2
    alg["gate|up"] += T * 2 * r * 2 + 3 * N * r * 2 + T * N + sc(T, N) + T * r * 2
    # weighted by dispatches: the few launches of the bench's fold-off roofline steps count as few
    per_launch = (sum((x["fetch_bytes"] + x["write_bytes"]) * x["dispatches"] for x in rows)
                  / sum(x["dispatches"] for x in rows))
    alg_mean = sum(alg.values()) / len(alg)
    summary = {"config": cfg, "kernel": "mx_gemm (gate|up, down, dh, dx)",
               "bytes_per_launch": round(per_launch),
               "algorithmic_bytes_per_launch": round(alg_mean),
               "copy_calibration": {"bytes": COPY_CALIB_BYTES, "fetch_scale": round(f_scale, 4),
                                    "write_scale": round(w_scale, 4)},
               "launches": rows, "algorithmic_bytes": alg,
               "commands": [cmd_fetch, cmd_write]}
    with open(_traffic_path(cfg, "json"), "w") as f:
        json.dump(summary, f, indent=1)
    with open(_traffic_path(cfg, "md"), "w") as f:
        f.write(f"# Memory traffic beyond L2 of the MX GEMM launches, configuration {cfg} (rocprofv3 FETCH_SIZE / "
                "WRITE_SIZE)\n\n")
        f.write("Commands (GPU box; one counter per run):\n\n```\ncd /tmp && export TMPDIR=/tmp\n"
                f"{cmd_fetch}\n{cmd_write}\n```\n\n")
        f.write(f"Scaled by the same counters on a plain copy kernel (torch.neg of 1 GiB bf16: reads 1 GiB, writes "
                f"1 GiB): FETCH x{f_scale:.4f}, WRITE x{w_scale:.4f}.  FETCH_SIZE counts what the L2 fetches from "
                "beyond itself, so reads served by the 256 MB last-level cache count as well as HBM reads: the "
                "columns are an upper bound on HBM bytes.\n\n")
        f.write("| kernel | shape | grid (threads) | dispatches | beyond-L2 read MB | beyond-L2 write MB |\n"
                "|---|---|---|---|---|---|\n")
        for x in rows:
            f.write(f"| {x['kernel']} | {_md(_kernel_key(x['kernel'], x['grid']).split('> ', 1)[-1])} | {x['grid']} | "
                    f"{x['dispatches']} | {x['fetch_bytes'] / 1e6:.1f} | {x['write_bytes'] / 1e6:.1f} |\n")
        f.write("\n| shape | algorithmic MB (operands + scales once, bf16 output, LoRA operands) |\n|---|---|\n")
        for nm, b in alg.items():
            f.write(f"| {_md(nm)} | {b / 1e6:.1f} |\n")
        f.write(f"\nMean per launch, weighted by dispatches: measured {per_launch / 1e6:.1f} MB, algorithmic "
                f"{alg_mean / 1e6:.1f} MB (the GEMMs' own bytes; the default dx and down launches also carry the "
                "token reductions, about 95 MB, and the xS_down sum, 66 MB).  The rows with few dispatches are the "
                "bench's fold-off roofline steps.\n")
    print(json.dumps({"bytes_per_launch": summary["bytes_per_launch"],
                      "algorithmic_bytes_per_launch": summary["algorithmic_bytes_per_launch"]}))


_TABLE_CAPTIONS = {
    "lora_epilogues_c3_kernel_trace":
        "T = 10752 tokens, r = 16. The run times `lora_bwd` at dy [T, 2048] (grid y = 16) and [T, 6144] (y = 48) and "
        "`res_lora` at [T, 2048] (50 calls each), then 13 steps (3 warmup + 10) of the attention-projection step "
        "(q|k|v 2048/512/512 grouped, o_proj 2048 -> 2048 deferred into `residual_add`, forward + backward; the dx "
        "GEMMs, `gemm_kernel<48, 1, 0>` and `<16, 1, 0>` with 928 workgroups, run the dA reductions in their launch), "
        "3 more on a side stream and 13 replays of the step captured into a HIP graph, then the "
        "SwiGLU kernels alone on [T, 6144] and 13 steps of the unfused MLP (`shared_prefix._mlp` with the fused MLP "
        "off: gate and up as one `group_linear`, the SwiGLU kernels, down as a `group_linear`; gate/up/down are not "
        "in `mxfp8.FUSED_BWD`, as in the reference, so their backward is the per-layer one, whose bf16 LoRA products "
        "run on hipBLASLt).  The two steps' kernels share some names and grids, so those rows mix both.  The bench "
        "line's `lora_epilogues`, `grouped_linears` and `unfused_mlp` entries give the rates.",
}


def _kernel_table(name, d, cmd, min_calls=6):
    """rocprofv3 --kernel-trace in `d` -> profiles/<name>.md: per (kernel, grid in workgroups) the calls and the
    mean duration, kernels launched fewer than `min_calls` times (input generation, weight preparation) left out."""
    files = glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no *kernel_trace.csv under {d}")
    agg = {}
    for f in files:
        with open(f) as fh:
            for r in csv.DictReader(fh):
                kname = r["Kernel_Name"]
                if "at::native" in kname:
                    m = re.search(r"at::native::(?:\(anonymous namespace\)::)?([A-Za-z_0-9]+)", kname)
                    key = "torch " + (m.group(1) if m else kname[:30])
                elif kname.startswith("Cijk_"):  # a hipBLASLt kernel: its macro tile
                    m = re.search(r"_MT(\d+x\d+x\d+)_", kname)
                    key = f"hipBLASLt GEMM (MT{m.group(1) if m else '?'})"
                else:
                    key = re.sub(r"\(anonymous namespace\)::", "", kname).split("(")[0].replace("void ", "")
                wg = max(int(r.get("Workgroup_Size_X") or 1), 1)
                grid = f"{int(r['Grid_Size_X']) // wg} x {r['Grid_Size_Y']}"
                agg.setdefault((key, grid), []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    rows = sorted(((k, g, v) for (k, g), v in agg.items() if len(v) >= min_calls), key=lambda x: -sum(x[2]))
    with open(os.path.join(ROOT, "profiles", name + ".md"), "w") as f:
        f.write(f"# Kernel trace: {name}\n\nCommand (GPU box, repo root as `$GRAFT_REPO_ROOT`):\n\n```\ncd /tmp && "
                f"export TMPDIR=/tmp\n{cmd}\npython3 bench.py --kernel-table {name} <trace dir>\n```\n\n")
        if name in _TABLE_CAPTIONS:
            f.write(_TABLE_CAPTIONS[name] + "\n\n")
        f.write(f"Kernels launched fewer than {min_calls} times are left out.\n\n| kernel | grid (workgroups) | calls | "
                "mean us |\n|---|---|---|---|\n")
        for k, g, v in rows:
            f.write(f"| {_md(k)} | {g} | {len(v)} | {sum(v) / len(v):.1f} |\n")


def _md(text):
    """A markdown table cell: the label's '|' (gate|up) escaped."""
    return text.replace("|", "\\|")


def _kernel_key(name, grid):
    """A short kernel name: the template head of the demangled name, and for the MX GEMM the MLP shape its grid
    and epilogue rank identify at configuration 3 (4032 / 2016 / 672 workgroups of 256 threads; the dx GEMM with
    the backward's token reductions folded into its launch has 672 + 512, the down GEMM with the xS_down sum
    168 + 672)."""
    m = re.search(r"(\w+_kernel)(<[^>]*>)?", name)
    k = (m.group(1) + (m.group(2) or "")) if m else name[:48]
    if m and m.group(1) == "gemm_kernel":
        wg = int(grid) // 256 if grid else 0
        shape = {(4032, "0"): "gate|up", (2016, "0"): "dh", (672, "16"): "down", (672, "32"): "dx",
                 (1184, "32"): "dx + token reductions", (840, "16"): "down + xS_down sum"}
        targs = [a.strip() for a in (m.group(2) or "<0").strip("<>").split(",")]
        r = targs[0]
        if len(targs) > 2 and targs[2] == "1":
            k += " gate|up + SwiGLU epilogue"
        elif len(targs) > 2 and targs[2] == "2":
            k += " dh + SwiGLU backward epilogue"
        else:
            # other grids (configuration 4): at LoRA rank 16 the epilogue rank alone tells the shapes apart
            k += " " + shape.get((wg, r), {"0": "dh", "16": "down", "32": "dx"}.get(r, f"{wg} WGs"))
    return k


def _counters_summary(name, dirs, cmds):
    """Per-kernel medians over the dispatches of the rocprofv3 --pmc passes in `dirs` (one counter set per pass; each dispatch row
    carries its start and end timestamps), with the derived figures: sustained shader clock = GRBM_GUI_ACTIVE / kernel duration; MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES
    / (GRBM_GUI_ACTIVE x 256 CUs x 4 SIMDs); FP8 MFMA flops = 512 x SQ_INSTS_VALU_MFMA_MOPS_F8; L2 hit rate =
    TCC_HIT / (TCC_HIT + TCC_MISS); TA / TD busy = TA_TA_BUSY_sum / TD_TD_BUSY_sum / (GRBM_GUI_ACTIVE x 256); beyond-L2 read / write = FETCH_SIZE
    / WRITE_SIZE scaled by their reading on a 1 GiB copy kernel in the same pass (--copy-calib): bytes the L2
    moves to and from the last-level cache and HBM, an upper bound on HBM bytes.
    Writes profiles/<name>.md and .json."""
    per = {}  # kernel key -> counter -> [per-dispatch values]
    for d in dirs:
        dur, vals = {}, {}
        for row in _pmc_rows(d):
            k = (row["Dispatch_Id"], row["Kernel_Name"], row.get("Grid_Size", ""))
            vals.setdefault(k, {})
            c = row["Counter_Name"]
            vals[k][c] = vals[k].get(c, 0.0) + float(row["Counter_Value"])
            dur[row["Dispatch_Id"]] = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
        # FETCH_SIZE / WRITE_SIZE (KiB per dispatch) scaled to bytes by what they read on the 1 GiB copy kernel
        for c in ("FETCH_SIZE", "WRITE_SIZE"):
            calib = sorted(cs[c] for (_, kname, _), cs in vals.items() if "neg" in kname and c in cs)
            for cs in vals.values():
                if c in cs:
                    cs[c] = cs[c] * COPY_CALIB_BYTES / calib[len(calib) // 2] if calib else float("nan")
        for (did, kname, grid), cs in vals.items():
            if "at::native" in kname:  # torch's own kernels (input generation, the copy calibration)
                continue
            key = _kernel_key(kname, grid)
            ent = per.setdefault(key, {})
            for c, v in cs.items():
                ent.setdefault(c, []).append(v)
            if did in dur and "GRBM_GUI_ACTIVE" in cs:
                ent.setdefault("_clock_mhz", []).append(cs["GRBM_GUI_ACTIVE"] / dur[did] * 1e3)
            if did in dur:
                ent.setdefault("_us_" + os.path.basename(d.rstrip("/")), []).append(dur[did] / 1e3)
    med = lambda v: sorted(v)[len(v) // 2] if v else float("nan")  # noqa: E731  (robust to a warm-up dispatch)
    table = {}
    for key, ent in per.items():
        m = {c: med(v) for c, v in ent.items()}
        if "GRBM_GUI_ACTIVE" in m:  # summed over the 8 XCDs' graphics register bus managers
            m["GRBM_GUI_ACTIVE"] /= N_XCD
            m["_clock_mhz"] /= N_XCD
        gui = m.get("GRBM_GUI_ACTIVE")
        row = {"dispatches": max(len(v) for v in ent.values())}
        us = [v for c, v in m.items() if c.startswith("_us_")]
        if "_clock_mhz" in m and us and min(us) >= 50:  # short dispatches: profiling overhead dominates GUI_ACTIVE
            row["clock_MHz"] = round(m["_clock_mhz"])
        if gui and "SQ_VALU_MFMA_BUSY_CYCLES" in m:
            row["mfma_busy"] = round(m["SQ_VALU_MFMA_BUSY_CYCLES"] / (gui * 256 * 4), 4)
        if "SQ_INSTS_VALU_MFMA_MOPS_F8" in m:
            row["fp8_mfma_GFLOP"] = round(512 * m["SQ_INSTS_VALU_MFMA_MOPS_F8"] / 1e9, 1)
        if "TCC_HIT_sum" in m and "TCC_MISS_sum" in m and m["TCC_HIT_sum"] + m["TCC_MISS_sum"] > 0:
            row["l2_hit"] = round(m["TCC_HIT_sum"] / (m["TCC_HIT_sum"] + m["TCC_MISS_sum"]), 4)
        for c, out_name in (("FETCH_SIZE", "beyond_l2_read_MB"), ("WRITE_SIZE", "beyond_l2_write_MB")):
            if c in m:
                row[out_name] = round(m[c] / 1e6, 1)
        for c, out_name in (("TA_TA_BUSY_sum", "ta_busy"), ("TD_TD_BUSY_sum", "td_busy")):
            if c in m and gui:
                row[out_name] = round(m[c] / (gui * 256), 4)
        for c, v in m.items():
            if c.startswith("_us_"):
                row["us[" + c[4:] + "]"] = round(v, 1)
        table[key] = row
    os.makedirs(os.path.join(ROOT, "profiles"), exist_ok=True)
    with open(os.path.join(ROOT, "profiles", name + ".json"), "w") as f:
        json.dump({"commands": cmds, "kernels": table}, f, indent=1)
    cols = sorted({c for r in table.values() for c in r})
    with open(os.path.join(ROOT, "profiles", name + ".md"), "w") as f:
        f.write(f"# rocprofv3 counters per kernel: {name}\n\n")
        f.write("Commands (GPU box, one pass each; repo root as `$GRAFT_REPO_ROOT`):\n\n```\ncd /tmp && export "
                "TMPDIR=/tmp\n" + "\n".join(cmds) + "\n```\n\n")
        f.write(_counters_summary.__doc__.split("derived figures:")[1].split("Writes")[0].strip()
                .replace("\n    ", " ") + "\n\n")
        f.write("Durations (`us[...]`) are each pass's own dispatch timestamps (counter collection serializes and "
                "instruments every dispatch, so they run a little longer than in the timed bench).\n\n")
        f.write("| kernel | " + " | ".join(cols) + " |\n|" + "---|" * (len(cols) + 1) + "\n")
        for key in sorted(table):
            f.write(f"| {_md(key)} | " + " | ".join(str(table[key].get(c, "")) for c in cols) + " |\n")
    print(json.dumps(table))


def _trace_summary(name, d, steps, cmd, layers=1):
    """rocprofv3 --kernel-trace of a bench run in `d` -> profiles/<name>.md: per kernel (the MX GEMM split into
    its MLP shapes by _kernel_key) the launches from the first MX GEMM on, the median duration, and the share of a
    step = median x round(launches / steps), where `steps` counts every step the profiled process ran (warmup,
    timed and instrumented); steps = 0 takes it from the trace: the backward kernel runs once per layer and step
    (the gating forward has no backward), so steps = its launches / layers."""
    files = glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no *kernel_trace.csv under {d}")
    rows_all = []
    for f in files:
        with open(f) as fh:
            rows_all += list(csv.DictReader(fh))
    # the steps' window: from the first MX GEMM launch (the gating forward) on; input generation, the model's
    # host-to-device copies and the weight preparation before it are one-off work
    gemm_starts = [int(r["Start_Timestamp"]) for r in rows_all if "gemm_kernel" in r["Kernel_Name"]]
    t0 = min(gemm_starts) if gemm_starts else 0
    given = steps
    if steps <= 0:
        steps = sum(1 for r in rows_all if re.search(r"\bbwd_kernel<", r["Kernel_Name"])) / max(layers, 1)
        if steps <= 0:
            raise SystemExit("no backward-kernel launches to count steps by")
    durs = {}
    for row in rows_all:
        if int(row["Start_Timestamp"]) < t0:
            continue
        kname = row["Kernel_Name"]
        if "at::native" in kname:
            m = re.search(r"at::native::(?:\(anonymous namespace\)::)?([A-Za-z_0-9]+)", kname)
            key = "torch " + (m.group(1) if m else kname[:30])
        else:
            grid = int(row["Grid_Size_X"]) * int(row["Grid_Size_Y"]) * int(row["Grid_Size_Z"])
            key = _kernel_key(kname, str(grid))
        durs.setdefault(key, []).append((int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3)
    rows = []
    for key, v in durs.items():
        med = sorted(v)[len(v) // 2]
        rows.append((key, len(v), med, med * round(len(v) / steps)))
    rows.sort(key=lambda r: -r[3])
    tot = sum(r[3] for r in rows)
    with open(os.path.join(ROOT, "profiles", name + ".md"), "w") as f:
        f.write(f"# Kernel trace: {name}\n\nCommand (GPU box, repo root as `$GRAFT_REPO_ROOT`):\n\n```\ncd /tmp && "
                f"export TMPDIR=/tmp\n{cmd}\npython3 bench.py --trace-summary {name} <trace dir> {given:g}"
                f"{f' --trace-layers {layers}' if layers != 1 else ''}\n```\n\n")
        f.write(f"The profiled process runs {steps:g} steps (warmup, timed and instrumented"
                f"{'; counted from the backward-kernel launches' if given <= 0 else ''}) after one forward for the "
                "gating check; "
                "dispatches before that forward's first MX GEMM (input generation, host-to-device copies, weight "
                "preparation) are left out. 'per step' = median duration x round(launches / steps); kernels of the "
                "gating forward alone, and the separate launches of the bench's fold-off roofline steps (a few "
                "steps with the token reductions and the xS_down sum outside the GEMM launches), show 0.\n\n"
                "| kernel | launches | median us | us per step | % |\n"
                "|---|---|---|---|---|\n")
        for key, n, med, ps in rows:
            f.write(f"| {_md(key)} | {n} | {med:.1f} | {ps:.1f} | {100 * ps / tot if tot else 0:.1f} |\n")
        f.write(f"\nSum of kernel time per step: {tot:.1f} us.\n")
        stats = glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True)
        if stats:  # rocprofv3 --stats of the same run: every dispatch of the process, warmup and gating forward too
            with open(stats[0]) as fh:
                srows = list(csv.DictReader(fh))
            f.write("\nrocprofv3 --stats of the same run (every dispatch of the process by kernel name, the gating "
                    "forward and the warmup steps included; in the MLP step each MX GEMM shape has its own template "
                    "arguments: <16, 1, 1> gate|up with the SwiGLU epilogue, <16, 1, 0> down (with the xS_down "
                    "sum in its launch by default), <0, 1, 0> dh, <32, 1, 0> dx (with the token reductions in its "
                    "launch by default)):\n\n| kernel | calls | average us | min us | max us | % |\n"
                    "|---|---|---|---|---|---|\n")
            for r in srows[:16]:
                m = re.search(r"(\w+_kernel)(<[^>]*>)?", r["Name"])
                kn = (m.group(1) + (m.group(2) or "")) if m else r["Name"][:48]
                f.write(f"| {kn} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                        f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | "
                        f"{float(r['Percentage']):.1f} |\n")
    print(json.dumps({k: round(ps, 1) for k, _, _, ps in rows}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=3, choices=(3, 4, 5))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-quant", action="store_true", help="skip the standalone quantizer timings")
    ap.add_argument("--graph", action="store_true", help="also time the step as replays of a HIP graph (hip_graph)")
    ap.add_argument("--no-gemm-alone", action="store_true",
                    help="skip roofline.gemm_alone (the fold-off GEMM steps), e.g. for a kernel trace of a run with "
                         "few steps, whose per-step accounting would count their launches")
    ap.add_argument("--cpu-tokens", type=int, default=1024)
    ap.add_argument("--copy-calib", action="store_true")
    ap.add_argument("--only", choices=("epilogues",), help="time only the LoRA epilogues and the grouped linears "
                    "(one JSON line of those figures, not the MLP metric line): the profiling command of that section")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"))
    ap.add_argument("--traffic-commands", nargs=2, default=("", ""), metavar=("CMD_FETCH", "CMD_WRITE"))
    ap.add_argument("--counters-summary", nargs="+", metavar=("NAME", "DIR"),
                    help="summarize rocprofv3 --pmc passes (each with --kernel-trace) into profiles/NAME.{md,json}")
    ap.add_argument("--counters-commands", nargs="*", default=[], help="the profiling commands, for the summary")
    ap.add_argument("--trace-summary", nargs=3, metavar=("NAME", "DIR", "STEPS"),
                    help="summarize a rocprofv3 --kernel-trace run of STEPS steps into profiles/NAME.md")
    ap.add_argument("--trace-command", default="", help="the profiling command, for the summary")
    ap.add_argument("--trace-layers", type=int, default=1, help="MLP layers per step of the traced run (steps = 0)")
    ap.add_argument("--kernel-table", nargs=2, metavar=("NAME", "DIR"),
                    help="rocprofv3 --kernel-trace output -> profiles/NAME.md: calls and mean duration per kernel and "
                         "grid (with --trace-command)")
    args = ap.parse_args()
    if args.trace_summary:
        _trace_summary(args.trace_summary[0], args.trace_summary[1], float(args.trace_summary[2]), args.trace_command,
                       args.trace_layers)
        return
    if args.counters_summary:
        _counters_summary(args.counters_summary[0], args.counters_summary[1:], args.counters_commands)
        return
    if args.kernel_table:
        _kernel_table(args.kernel_table[0], args.kernel_table[1], args.trace_command)
        return
    if args.traffic_summary:
        _traffic_summary(args.config, *args.traffic_summary, *args.traffic_commands)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the MLP shards by tokens with "
              "one LoRA-gradient all-reduce per layer).", file=sys.stderr)
        sys.exit(2)

    import torch

    import fused_linear
    import fused_mlp
    import mxfp8
    import workloads

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = args.config
    c = workloads.CONFIGS[cfg]
    if args.only == "epilogues":
        T, K, N = c["T"], c["K"], c["N"]
        print(json.dumps({"config": workloads.DESCRIPTIONS[cfg],
                          "lora_epilogues": _lora_epilogues(T, K, N, c["r"], dev),
                          "grouped_linears": _grouped_linears(T, K, c["r"], c["alpha"], dev),
                          "unfused_mlp": _unfused_mlp(T, K, N, c["r"], dev)}), flush=True)
        return
    model, inps = workloads.build_model(cfg, layers=c["layers"], device=dev)
    mxfp8.enable_mxfp8(model)
    mods = [layer.mlp for layer in model.layers]
    inp = inps[0]
    T, K, N = inp["T"], inp["K"], inp["N"]
    x = inp["x"].to(dev).requires_grad_(True)
    dy = inp["dy"].to(dev)
    del inps
    params = [p for p in model.parameters() if p.requires_grad]

    stacked = len(mods) > 1  # a stack: x <- x + mlp(rms_norm(x)) (shared_prefix.py:239)

    def step():
        fused_linear.new_step()
        for p in params:
            p.grad = None
        x.grad = None
        y = x
        for m in mods:
            if stacked:
                y = y + fused_mlp.mlp(m, torch.nn.functional.rms_norm(y, (K,), eps=1e-6))
            else:
                y = fused_mlp.mlp(m, y)
        y.backward(dy)

    assert fused_mlp.mlp(mods[0], x) is not None, "fused path not taken"
    # W untimed warmup steps, continued until at least WARMUP_FLOOR_S of steps have run: the first ~20 steps
    # after a cold start run ~7% slower (clock and cache state), which a 5-step warmup at 1 ms per step leaves
    # inside the timed steps; the steps actually run are reported as warmup_steps_run
    warm = 0
    tw = time.perf_counter()
    while warm < args.warmup or time.perf_counter() - tw < WARMUP_FLOOR_S:
        step()
        warm += 1
        if warm >= args.warmup:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # The roofline: the same K steps again, each MX GEMM launch bracketed by two timing events on its stream.
    # An event record costs a few microseconds of idle GPU on each side of the kernel it brackets, so these
    # steps are timed apart from the K steps above (their own time is reported as instrumented_ms_per_step).
    mxfp8.GEMM_EVENTS = []
    t1 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall_ev = time.perf_counter() - t1
    ev = mxfp8.GEMM_EVENTS
    mxfp8.GEMM_EVENTS = None
    gemm_ms = sum(a.elapsed_time(b) for a, b, _ in ev)
    gemm_fl = sum(f for _, _, f in ev)
    # The same instrumented steps with the folds off, so that each GEMM launch runs the GEMM alone: the dx and down
    # launches otherwise also run the token reductions and the xS_down sum, and their events time that work as GEMM
    # time.  Reported beside the main figures as roofline.gemm_alone; the timed steps above keep the folds.
    folds = (fused_mlp.FOLD_TN[0], fused_mlp.FOLD_SUM[0])
    gemm_alone = None
    if any(folds) and not args.no_gemm_alone:
        fused_mlp.FOLD_TN[0] = fused_mlp.FOLD_SUM[0] = False
        mxfp8.GEMM_EVENTS = []
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        ev2 = mxfp8.GEMM_EVENTS
        mxfp8.GEMM_EVENTS = None
        fused_mlp.FOLD_TN[0], fused_mlp.FOLD_SUM[0] = folds
        ms2 = sum(a.elapsed_time(b) for a, b, _ in ev2)
        tf2 = sum(f for _, _, f in ev2) / (ms2 * 1e-3) / 1e12
        gemm_alone = {"achieved": round(tf2, 2), "frac": round(tf2 / PEAK_MXFP8_TFLOPS, 4),
                      "kernel_ms_per_step": round(ms2 / args.steps, 4),
                      "note": "the same steps with the token reductions and the xS_down sum in launches of their "
                              "own (MXFP8_FOLD_TN=0, MXFP8_FOLD_SUM=0), so the four GEMM launches run only GEMMs"}
    ms = wall * 1e3 / args.steps
    fl = workloads.flops(T, K, N) * len(mods)
    value = fl / (ms * 1e-3) / 1e12
    gemm_tf = gemm_fl / (gemm_ms * 1e-3) / 1e12
    # With --graph, a side figure, not `value`: the same step captured into a HIP graph and replayed K times (a
    # training loop that captures its step replays every kernel without the Python and autograd enqueue work
    # between them; tests/test_gpu_graph.py checks replays bit for bit against eager steps).  The eager steps
    # already run back to back, and the replays measured slower, so it is off by default.  A failed capture is
    # reported here and leaves the line intact.
    hip_graph = None
    if args.graph:
        try:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(3):
                    step()
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                step()
            for _ in range(3):
                graph.replay()
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            for _ in range(args.steps):
                graph.replay()
            torch.cuda.synchronize()
            gms = (time.perf_counter() - t2) * 1e3 / args.steps
            hip_graph = {"ms_per_step": round(gms, 4), "TFLOP/s": round(fl / (gms * 1e-3) / 1e12, 2),
                         "frac_of_mxfp8_peak": round(fl / (gms * 1e-3) / 1e12 / PEAK_MXFP8_TFLOPS, 4)}
            del graph
        except RuntimeError as e:
            torch.cuda.synchronize()
            hip_graph = {"error": str(e)[:200]}

    line = {
        "metric": "MXFP8 MLP fwd+bwd TFLOP/s (% MXFP8 peak); quantizer GB/s (% of HBM)",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": warm,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp8",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights and LoRA A/B, N(0,1e-2) upstream grad)"
                if cfg != 5 else "synthetic (seeded Student-t(3) activations with x100 channels, all-zero, -0 and "
                                 "448*2^k blocks; N(0,0.02) weights and LoRA A/B)",
        "config": {"workload": workloads.DESCRIPTIONS[cfg], "layers": len(mods), "tokens": T, "d_model": K,
                   "d_ffn": N, "lora_r": c["r"], "lora_alpha": c["alpha"],
                   "frac_of_mxfp8_peak": round(value / PEAK_MXFP8_TFLOPS, 4)},
        "roofline": {"bound": "mfma", "achieved": round(gemm_tf, 2), "peak": PEAK_MXFP8_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(gemm_tf / PEAK_MXFP8_TFLOPS, 4), "traffic": _traffic_from_profiles(cfg),
                     "kernel": "mx_gemm (4 launches per layer: gate|up, down, dh, dx)" +
                               ("; the dx launch also runs the backward's token reductions (mxfp8_gemm_nt_tn)"
                                if fused_mlp.FOLD_TN[0] else "") +
                               ("; the down launch also sums xS_down (mxfp8_gemm_nt_sum)"
                                if fused_mlp.FOLD_SUM[0] else "") +
                               ("; timed as GEMM time" if fused_mlp.FOLD_TN[0] or fused_mlp.FOLD_SUM[0] else ""),
                     "launches": len(ev), "kernel_ms_per_step": round(gemm_ms / args.steps, 4),
                     "instrumented_ms_per_step": round(wall_ev * 1e3 / args.steps, 4),
                     "gemm_alone": gemm_alone},
    }
    if hip_graph is not None:
        line["hip_graph"] = hip_graph
    del model, mods, params, x, dy
    torch.cuda.empty_cache()
    if not args.no_quant:
        quant, wq_ms = _quantizer(T, K, N, dev)
        line["quantizer"] = quant
        line["lora_epilogues"] = _lora_epilogues(T, K, N, c["r"], dev)
        line["grouped_linears"] = _grouped_linears(T, K, c["r"], c["alpha"], dev)
        line["unfused_mlp"] = _unfused_mlp(T, K, N, c["r"], dev)
        tot = ms + wq_ms * c["layers"]
        line["with_requant"] = {"ms_per_step": round(tot, 4), "TFLOP/s": round(fl / (tot * 1e-3) / 1e12, 2),
                                "weight_prep_ms_per_layer": round(wq_ms, 4)}
    if args.copy_calib:
        _copy_calib(dev)
    if not args.no_cpu:
        line["cpu_baseline"] = _cpu_baseline(cfg, args.cpu_tokens)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
