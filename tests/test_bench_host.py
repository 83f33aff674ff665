"""Host-side checks of bench.py's profile summaries (no GPU): the kernel-trace summary on a synthetic rocprofv3
trace (step count taken from the backward-kernel launches, per-step shares, the --stats table), the MX GEMM shape
names, and the JSON-line contract of the --gpus guard."""
import csv
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402

_FIELDS = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id", "Kernel_Id", "Kernel_Name",
           "Correlation_Id", "Start_Timestamp", "End_Timestamp", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
           "Accum_VGPR_Count", "SGPR_Count", "Workgroup_Size_X", "Workgroup_Size_Y", "Workgroup_Size_Z",
           "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"]


def _row(i, name, t0, us, grid):
    r = dict.fromkeys(_FIELDS, "0")
    r.update(Kind="KERNEL_DISPATCH", Dispatch_Id=str(i), Kernel_Name=name, Start_Timestamp=str(t0),
             End_Timestamp=str(t0 + int(us * 1000)), Grid_Size_X=str(grid), Grid_Size_Y="1", Grid_Size_Z="1")
    return r


def _write_trace(d, steps):
    """One gating forward (gate|up, down) and `steps` fwd+bwd steps of the configuration-3 launch sequence."""
    seq_fwd = [("void (anonymous namespace)::gemm_kernel<16, 1, 1>(...)", 270.0, 4032 * 256),
               ("void (anonymous namespace)::gemm_kernel<16, 1, 0>(...)", 121.0, 672 * 256)]
    seq_bwd = [("void (anonymous namespace)::gemm_kernel<0, 1, 0>(...)", 118.0, 2016 * 256),
               ("void (anonymous namespace)::bwd_kernel<16, true, false, 2>(...)", 150.0, 504 * 512),
               ("void (anonymous namespace)::gemm_kernel<32, 1, 0>(...)", 237.0, 672 * 256)]
    rows, t, i = [], 1_000_000, 0
    rows.append(_row(i, "void at::native::fill_kernel(...)", 10, 5.0, 256))  # before the first GEMM: left out
    for k in range(steps + 1):
        for name, us, grid in seq_fwd + (seq_bwd if k else []):
            rows.append(_row(i, name, t, us, grid))
            t += int(us * 1000) + 100
            i += 1
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "run_kernel_trace.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=_FIELDS, quoting=csv.QUOTE_ALL)
        w.writeheader()
        w.writerows(rows)
    with open(os.path.join(d, "run_kernel_stats.csv"), "w", newline="") as f:
        w = csv.writer(f, quoting=csv.QUOTE_ALL)
        w.writerow(["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"])
        w.writerow(["void (anonymous namespace)::gemm_kernel<16, 1, 1>(...)", steps + 1, 1, 270000.0, 30.0, 1, 2, 0])


def test_trace_summary_counts_steps_from_the_backward_kernel(tmp_path, monkeypatch):
    d = tmp_path / "kt"
    _write_trace(str(d), steps=7)
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    os.makedirs(tmp_path / "profiles")
    bench._trace_summary("t", str(d), 0, "cmd")
    md = (tmp_path / "profiles" / "t.md").read_text()
    assert "runs 7 steps" in md and "counted from the backward-kernel launches" in md
    # 8 gate|up launches over 7 steps round to one per step; the fill before the first GEMM is left out
    assert "| gemm_kernel<16, 1, 1> gate\\|up + SwiGLU epilogue | 8 | 270.0 | 270.0 |" in md
    assert "| bwd_kernel<16, true, false, 2> | 7 | 150.0 | 150.0 |" in md
    assert "| gemm_kernel<32, 1, 0> dx | 7 | 237.0 | 237.0 |" in md
    assert "fill_kernel" not in md
    assert "Sum of kernel time per step: 896.0 us." in md  # 270 + 121 + 118 + 150 + 237
    assert "| gemm_kernel<16, 1, 1> | 8 | 270.0 |" in md  # the --stats table of the same run


def test_trace_summary_with_layers(tmp_path, monkeypatch):
    d = tmp_path / "kt"
    _write_trace(str(d), steps=6)
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    os.makedirs(tmp_path / "profiles")
    bench._trace_summary("t", str(d), 0, "cmd", layers=3)  # 6 backward launches = 2 steps of 3 layers
    assert "runs 2 steps" in (tmp_path / "profiles" / "t.md").read_text()


@pytest.mark.parametrize("name,grid,want", [
    ("gemm_kernel<16, 1, 1>(x)", str(4032 * 256), "gate|up + SwiGLU epilogue"),
    ("gemm_kernel<0, 1, 0>(x)", str(2016 * 256), "dh"), ("gemm_kernel<16, 1, 0>(x)", str(672 * 256), "down"),
    ("gemm_kernel<32, 1, 0>(x)", str(672 * 256), "dx"),
    ("gemm_kernel<32, 1, 0>(x)", str(8896 * 256), "dx"),   # configuration 4's grid: named by the epilogue rank
    ("gemm_kernel<0, 1, 0>(x)", str(26688 * 256), "dh"),
    ("gemm_kernel<16, 1, 2>(x)", str(2016 * 256), "dh + SwiGLU backward epilogue")])
def test_gemm_shape_names(name, grid, want):
    assert bench._kernel_key(name, grid).endswith(want)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_kernel_table_groups_by_kernel_and_grid(tmp_path, monkeypatch):
    """--kernel-table: one row per (kernel, grid in workgroups) with calls and mean duration, hipBLASLt names cut to
    their macro tile, torch kernels by their functor name, kernels launched fewer than six times left out."""
    rows, t, i = [], 1000, 0
    spec = [("void (anonymous namespace)::lora_bwd_kernel<16, true, true>(...)", 20.0, 31 * 256, 8),
            ("void (anonymous namespace)::lora_bwd_kernel<16, true, true>(...)", 50.0, 11 * 256, 6),
            ("Cijk_Ailk_Bjlk_BBS_BH_Bias_HA_S_SAV_UserArgs_MT16x64x256_MI16x16x1_SN_LDSB1", 60.0, 96 * 256, 7),
            ("void at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<float>>(...)", 3.0, 48 * 256, 6),
            ("void (anonymous namespace)::pack_kernel(...)", 6.0, 496 * 256, 5)]
    for name, us, grid, n in spec:
        for _ in range(n):
            r = _row(i, name, t, us, grid)
            r["Workgroup_Size_X"] = "256"
            rows.append(r)
            t += int(us * 1000) + 100
            i += 1
    d = tmp_path / "epi"
    os.makedirs(d)
    with open(d / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=_FIELDS, quoting=csv.QUOTE_ALL)
        w.writeheader()
        w.writerows(rows)
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    os.makedirs(tmp_path / "profiles")
    bench._kernel_table("lora_epilogues_c3_kernel_trace", str(d), "cmd")
    md = (tmp_path / "profiles" / "lora_epilogues_c3_kernel_trace.md").read_text()
    assert "| lora_bwd_kernel<16, true, true> | 31 x 1 | 8 | 20.0 |" in md
    assert "| lora_bwd_kernel<16, true, true> | 11 x 1 | 6 | 50.0 |" in md
    assert "| hipBLASLt GEMM (MT16x64x256) | 96 x 1 | 7 | 60.0 |" in md
    assert "| torch vectorized_elementwise_kernel | 48 x 1 | 6 | 3.0 |" in md
    assert "pack_kernel" not in md and "attention-projection step" in md
