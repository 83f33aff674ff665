"""CPU checks of the boundary and the host logic: the C-ABI library loads, exports every function that
include/mxfp8_mlp.h declares, reports the ABI version the Python side expects, and rejects bad arguments
before launching anything; the launch-grid choices and the workload generators behave as documented.
No GPU compute is called."""
import ctypes
import os
import re

import pytest
import torch

import _native
import fused_mlp
import workloads

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mxfp8_mlp.h")


def _declared():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(mxfp8_\w+)\s*\(", txt, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("libmxfp8_mlp.so not built")
    return _native.load()


def test_header_declares_the_abi():
    names = _declared()
    assert "mxfp8_quant_rows" in names and "mxfp8_gemm_nt" in names and "mxfp8_mlp_bwd" in names
    assert len(names) == 37, names


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name
    assert set(_declared()) == set(_native.SIGNATURES)


def _arg_counts():
    txt = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for name, args in re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(mxfp8_\w+)\s*\(([^)]*)\)", txt, flags=re.M):
        args = args.strip()
        out[name] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_signatures_match_the_header_argument_counts():
    # every pointer-sized argument, the trailing stream included, must be typed: an untyped Python int is
    # passed as a C int
    counts = _arg_counts()
    for name, args in _native.SIGNATURES.items():
        assert len(args) == counts[name], (name, len(args), counts[name])


def test_abi_version(lib):
    assert lib.mxfp8_abi_version() == _native.ABI_VERSION
    txt = open(HEADER).read()
    assert f"#define MXFP8_MLP_ABI_VERSION {_native.ABI_VERSION}" in txt


def test_argument_checks_reject_before_launch(lib):
    p = ctypes.c_void_p(16)  # never dereferenced: the checks fail first
    # cols not a multiple of 128
    assert lib.mxfp8_quant_rows(p, 4, 100, 100, p, 112, p, 1, 0, None) == -1
    assert b"cols" in lib.mxfp8_last_error()
    # null pointer
    assert lib.mxfp8_quant_rows(None, 4, 128, 128, p, 128, p, 1, 0, None) == -1
    # transpose: C outside {16, 32, 64}, padded length below T
    assert lib.mxfp8_transpose_pad(p, 8, 24, 24, p, 128, None) == -1
    assert lib.mxfp8_transpose_pad(p, 200, 32, 32, p, 128, None) == -1
    # allocation-free token reduction: rp * K * 4 bytes beyond its 16 MiB static scratch (checked first, no GPU call)
    assert lib.mxfp8_lora_tn_noalloc(p, 64, 65536 + 128, 65536 + 128, p, 64, 1.0, 0, 0, p, None) == -1
    assert b"static scratch" in lib.mxfp8_last_error()
    # GEMM with folded token reductions: only the rank-16, 32 or 48 epilogue of the 4-wave shape, and the batch's own
    # checks (ranks 16, 32 and 64)
    job = _native.LoraTnJob(16, 2048, 16, 32, 1.0, 0, 0, 16)
    jobs = (_native.LoraTnJob * 1)(job)
    gemm = lambda r, layout, jb: lib.mxfp8_gemm_nt_tn(p, p, 2048, p, p, 2048, 256, 2048, 2048, p, 2048, p, 32, p, 32,  # noqa: E731
                                                      r, 1.0, layout, jb, 1, 256, 2048, 8, p, None)
    assert gemm(64, 0, jobs) == -1 and b"rank-16, 32 or 48" in lib.mxfp8_last_error()
    assert gemm(32, _native.GEMM_WIDE, jobs) == -1 and b"4-wave" in lib.mxfp8_last_error()
    bad = (_native.LoraTnJob * 1)(_native.LoraTnJob(16, 2048, 16, 48, 1.0, 0, 0, 16))
    assert gemm(32, 0, bad) == -1 and b"mxfp8_gemm_nt_tn: job 0" in lib.mxfp8_last_error()
    # GEMM with its epilogue operand summed in the launch: rank 16 and the 4-wave shape only, aligned buffers
    gsum = lambda r, layout, part: lib.mxfp8_gemm_nt_sum(p, p, 2048, p, p, 2048, 256, 2048, 2048, p, 2048, part, 96,  # noqa: E731
                                                         1.0, p, p, 16, r, 1.0, layout, -1, None)
    assert gsum(32, 0, p) == -1 and b"r == 16" in lib.mxfp8_last_error()
    assert gsum(16, _native.GEMM_WIDE, p) == -1 and b"4-wave" in lib.mxfp8_last_error()
    assert gsum(16, 0, ctypes.c_void_p(8)) == -1 and b"misaligned" in lib.mxfp8_last_error()
    assert lib.mxfp8_lora_tn_noalloc_chunks(10752, 2048, 32) == lib.mxfp8_lora_tn_chunks(10752, 2048)
    assert lib.mxfp8_lora_tn_noalloc_chunks(10752, 2048, 32) * 32 * 2048 * 4 <= 16 << 20
    # GEMM K not a multiple of 128
    assert lib.mxfp8_gemm_nt(p, p, 96, p, p, 96, 4, 128, 96, p, 128, None, 0, None, 0, 0, 1.0, 0, None, 0, None) == -1
    # GEMM epilogue rank not supported
    assert lib.mxfp8_gemm_nt(p, p, 128, p, p, 128, 4, 128, 128, p, 128, p, 8, p, 8, 8, 1.0, 0, None, 0, None) == -1
    # unknown operand layout
    assert lib.mxfp8_gemm_nt(p, p, 128, p, p, 128, 4, 128, 128, p, 128, None, 0, None, 0, 0, 1.0, 32, None, 0, None) == -1
    assert b"layout" in lib.mxfp8_last_error()
    # B in the pi_col order stores 16-byte pieces: a row-major C with ldc % 8 != 0 is refused
    assert lib.mxfp8_gemm_nt(p, p, 128, p, p, 128, 4, 128, 128, p, 132, None, 0, None, 0, 0, 1.0, 16, None, 0, None) == -1
    assert b"B_PI" in lib.mxfp8_last_error()
    # workspace given but misaligned
    assert lib.mxfp8_gemm_nt(p, p, 128, p, p, 128, 4, 128, 128, p, 128, None, 0, None, 0, 0, 1.0, 0,
                             ctypes.c_void_p(16), 1 << 20, None) == -1
    assert b"workspace" in lib.mxfp8_last_error()
    # GEMMs with the SwiGLU epilogues: the backward takes r = 16 only; null pointers are refused
    fp = ctypes.cast(p, ctypes.POINTER(ctypes.c_float))
    bwd = [p] * 4 + [256, 512, 256] + [p] * 11 + [32, 1.0, 1.0, p, p] + [fp] * 4 + [None]
    assert lib.mxfp8_gemm_swiglu_bwd(*bwd) == -1
    assert b"r == 16" in lib.mxfp8_last_error()
    bwd[18] = 16
    bwd[8] = None
    assert lib.mxfp8_gemm_swiglu_bwd(*bwd) == -1
    assert b"null" in lib.mxfp8_last_error()
    fwd = [p] * 4 + [256, 512, 256] + [p] * 4 + [64, 1.0, 1.0, p, p, p, fp, None]
    assert lib.mxfp8_gemm_swiglu_fwd(*fwd) == -1
    assert b"r in {16, 32}" in lib.mxfp8_last_error()
    # backward column group must divide N and be a multiple of 128
    args = [p] * 12 + [256, 512, 16, 1.0, 1.0, 128, 384] + [p] * 2 + [ctypes.cast(p, ctypes.POINTER(ctypes.c_float))] * 4 + [None, 0, None]
    assert lib.mxfp8_mlp_bwd(*args) == -1
    # LoRA products: K must be a multiple of 64 (x · Wᵀ) / 128 (token reduction), rp in {16, 32, 64}
    assert lib.mxfp8_lora_nt(p, 4, 200, 200, p, 16, 1.0, p, None, 0, None) == -1
    assert lib.mxfp8_lora_nt(p, 4, 256, 256, p, 8, 1.0, p, None, 0, None) == -1
    # fused quantizer + rank-r product: K % 128, rp in {16, 32}, Tpad = ceil(T/128)*128
    assert lib.mxfp8_quant_lora(p, 4, 200, 200, p, p, p, 16, 1.0, p, None, 128, None) == -1
    assert lib.mxfp8_quant_lora(p, 4, 256, 256, p, p, p, 48, 1.0, p, None, 128, None) == -1
    assert lib.mxfp8_quant_lora(p, 4, 256, 256, p, p, p, 16, 1.0, p, None, 256, None) == -1
    assert b"Tpad" in lib.mxfp8_last_error()
    assert lib.mxfp8_lora_tn(p, 4, 96, 96, p, 16, 1, ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), 1.0, 0, 0, p,
                             None) == -1
    assert lib.mxfp8_lora_tn_chunks(10752, 2048) > 0 and lib.mxfp8_lora_tn_chunks(10752, 100) == 0
    # segmented GEMM output: boundaries at multiples of 128 from 0, 4-wave row-major only
    cols = (ctypes.c_int64 * 2)(0, 100)
    ptrs = (ctypes.c_void_p * 2)(16, 16)
    lds = (ctypes.c_int64 * 2)(128, 128)
    assert lib.mxfp8_gemm_nt_seg(p, p, 128, p, p, 128, 4, 256, 128, 2, cols, ptrs, lds, None, 0, None, 0, 0, None,
                                 1.0, 0, None) == -1
    cols = (ctypes.c_int64 * 2)(0, 128)
    assert lib.mxfp8_gemm_nt_seg(p, p, 128, p, p, 128, 4, 256, 128, 2, cols, ptrs, lds, None, 0, None, 0, 0, None,
                                 1.0, 4, None) == -1
    assert lib.mxfp8_gemm_nt_seg(p, p, 128, p, p, 128, 4, 256, 128, 5, cols, ptrs, lds, None, 0, None, 0, 0, None,
                                 1.0, 0, None) == -1
    # per-segment rank columns: a multiple of 8, inside ld_p and ld_q
    for bad in ((0, 20), (0, 24)):
        rc = (ctypes.c_int64 * 2)(*bad)
        assert lib.mxfp8_gemm_nt_seg(p, p, 128, p, p, 128, 4, 256, 128, 2, cols, ptrs, lds, p, 32, p, 32, 16, rc,
                                     1.0, 0, None) == -1
        assert b"rank columns" in lib.mxfp8_last_error()
    # SwiGLU: n % 8, aligned
    assert lib.mxfp8_swiglu(p, p, 12, p, None) == -1
    assert lib.mxfp8_swiglu_bwd(p, p, p, 16, p, ctypes.c_void_p(18), None) == -1
    # residual LoRA epilogue: N % 128, r in {16, 32}
    assert lib.mxfp8_res_lora(p, p, p, 16, p, 4, 100, 16, 1.0, p, None) == -1
    assert lib.mxfp8_res_lora(p, p, p, 16, p, 4, 128, 8, 1.0, p, None) == -1
    # LoRA backward: N % 128, something to do, rank, code columns inside q and its scale tiles
    lb = lambda T, N, q, ld_q, s_tiles, off, xa, r: lib.mxfp8_lora_bwd(  # noqa: E731
        p, T, N, N, q, ld_q, p if q else None, s_tiles, off, xa, 48, p, r, 1.0, p, 48, p, p, p, None)
    assert lb(4, 100, p, 128, 1, 0, None, 16) == -1
    assert lb(4, 128, None, 0, 0, 0, None, 16) == -1
    assert lb(4, 128, None, 0, 0, 0, p, 8) == -1
    assert lb(4, 256, p, 384, 3, 2, None, 16) == -1   # columns 256..511 past ld_q = 384
    assert lb(4, 256, p, 512, 3, 2, None, 16) == -1   # scale tiles 2..3 past s_col_tiles = 3
    assert b"destination" in lib.mxfp8_last_error()
    assert lib.mxfp8_lora_bwd_chunks(10752, 4096) > 0 and lib.mxfp8_lora_bwd_chunks(10752, 100) == 0
    # tiled quantizer / tile_codes shape checks
    assert lib.mxfp8_quant_tiled(p, 4, 100, 100, p, p, None) == -1
    assert lib.mxfp8_tile_codes(p, 4, 96, 96, p, None) == -1
    assert lib.mxfp8_sum_parts(None, 1, 4, 1.0, p, 0, None) == -1
    # bf16 pack: job count, a destination row shorter than the job's columns
    jobs = (_native.PackJob * 2)(_native.PackJob(None, 0, 0, 4, 64, p, 64, 0),
                                 _native.PackJob(p, 64, 1, 4, 64, p, 32, 0))
    assert lib.mxfp8_pack_bf16(ctypes.cast(jobs, ctypes.c_void_p), 0, None) == -1
    assert lib.mxfp8_pack_bf16(ctypes.cast(jobs, ctypes.c_void_p), 33, None) == -1
    assert lib.mxfp8_pack_bf16(ctypes.cast(jobs, ctypes.c_void_p), 2, None) == -1
    assert b"bad job 1" in lib.mxfp8_last_error()


def test_gemm_workspace_plan(lib):
    # the 8-wave shape's plan (the default 4-wave shape never splits); without a GPU the library plans for 256
    # CUs (MI355X): tail waves that fill at most half of the CUs are split along K into up to 4 pieces of an
    # even number of 64-wide K steps; 4 KB of counters come first
    ws = lib.mxfp8_gemm_workspace_size
    part = 256 * 256 * 4
    assert ws(10752, 12288, 2048) == 0  # 2016 tiles: last wave 224 of 256 CUs
    assert ws(10752, 6144, 2048) == 0   # 1008 tiles: last wave 240
    assert ws(10752, 2048, 12288) == 4096 + 80 * 3 * part  # 336 tiles: 80 split in 3 (64 steps each)
    assert ws(10752, 2048, 6144) == 4096 + 80 * 3 * part
    assert ws(256, 7168, 1024) == 4096 + 28 * 4 * part  # 28 tiles: 4 pieces of 4 steps
    assert ws(256, 1024, 128) == 0  # 2 K steps cannot be split into pieces of at least 4
    assert ws(0, 128, 128) == 0 and ws(4, 100, 128) == 0


def test_native_refuses_cpu_tensors(lib):
    x = torch.zeros(4, 128, dtype=torch.bfloat16)
    q = torch.empty(4, 128, dtype=torch.uint8)
    s = torch.empty(512, dtype=torch.uint8)
    with pytest.raises(_native.NativeError):
        _native.quant_rows(x, q, s)


def test_bwd_grid_choice():
    fused_mlp._CUS[0] = 256
    for T, N in [(10752, 6144), (4096, 3584), (256, 3584), (142336, 6144), (8896, 6144)]:
        sb, cg = fused_mlp._bwd_grid(T, N, 16)
        tpad = -(-T // 128) * 128
        assert sb % 128 == 0 and cg % 128 == 0 and N % cg == 0 and sb <= tpad
        nsb, ncg = -(-tpad // sb), N // cg
        # work per CU slot (rounds of 512 workgroups x row blocks x column quads) within 15% of the balanced
        # lower bound (SB is at least 4 row blocks)
        work = -(-(nsb * ncg) // 512) * (sb // 32) * (cg // 128)
        lower = max(4, -(-(tpad // 32) * (N // 128) // 512))
        assert work <= 1.15 * lower, (T, N, sb, cg, work, lower)


def test_fwd_groups_choice(lib):
    # one wave per (32-row block, column group); without a GPU the library assumes 256 CUs, and the kernel is
    # built for 2 waves per SIMD (two tiles in flight per wave): 2048 waves per round
    cap = 256 * 4 * 2
    for T, N in [(10752, 6144), (256, 3584), (4096, 3584), (8896, 6144)]:
        ng = fused_mlp._fwd_groups(T, N)
        nt = N // 32
        assert ng > 0 and nt % ng == 0
        nrb = -(-T // 128) * 4
        cost = -(-nrb * ng // cap) * (nt // ng + 1)
        for g in [d for d in range(1, nt + 1) if nt % d == 0]:
            assert cost <= -(-nrb * g // cap) * (nt // g + 1), (T, N, ng, g)
    assert lib.mxfp8_mlp_fwd_groups(10752, 100, 16) == 0 and lib.mxfp8_mlp_fwd_groups(10752, 6144, 8) == 0


def test_mlp_gating_on_cpu_returns_none():
    model, inps = workloads.build_model(1, T=8, device="cpu")
    assert fused_mlp.mlp(model.layers[0].mlp, inps[0]["x"]) is None


def test_workloads_shapes_and_seeds():
    a = workloads.make_inputs(1, T=64)
    b = workloads.make_inputs(1, T=64)
    assert torch.equal(a["x"], b["x"]) and a["x"].dtype == torch.bfloat16 and a["x"].shape == (64, 1024)
    assert a["Wg"].shape == (3584, 1024) and a["Wd"].shape == (1024, 3584)
    assert a["Ag"].shape == (16, 1024) and a["Bg"].shape == (3584, 16) and a["Ad"].shape == (16, 3584)
    assert a["Ag"].dtype == torch.float32 and a["s"] == 2.0
    assert workloads.flops(10752, 2048, 6144) == 1623497637888
    assert workloads.quant_bytes(10752, 2048) == 10752 * 2048 * 3 + 84 * 16 * 512


def test_outlier_config_contains_edge_blocks():
    x = workloads.make_inputs(5, T=512, dy=False)["x"].float()
    blocks = x.view(512, -1, 32)
    amax = blocks.abs().amax(-1)
    assert bool((amax == 0).any())  # all-zero blocks
    k = torch.log2(amax[amax > 0] / 448.0)
    assert bool((k == torch.round(k)).any())  # blocks whose amax is exactly 448 * 2^k
    assert bool(torch.signbit(blocks[(amax == 0)]).any())  # a -0.0 block


def test_job_structs_match_the_c_layout(tmp_path):
    """The ctypes job tables (_native.LoraBwdJob, PackJob, LoraTnJob) against the header's structs as gcc lays them
    out: every field's offset and the struct size, and the MAX_JOBS constants."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no gcc")
    structs = {"mxfp8_lora_bwd_job": _native.LoraBwdJob, "mxfp8_pack_job": _native.PackJob,
               "mxfp8_lora_tn_job": _native.LoraTnJob}
    lines = ['#include <stddef.h>', '#include <stdio.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, ct in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in ct._fields_:
            lines.append(f'  printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    for k in ("MXFP8_LORA_BWD_MAX_JOBS", "MXFP8_PACK_MAX_JOBS", "MXFP8_LORA_TN_MAX_JOBS"):
        lines.append(f'  printf("const {k} %d\\n", {k});')
    lines.append("  return 0;\n}\n")
    src, exe = tmp_path / "layout.c", tmp_path / "layout"
    src.write_text("\n".join(lines))
    subprocess.run([gcc, "-std=c11", "-o", str(exe), str(src)], check=True)
    got = {}
    for ln in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        a, b, v = ln.split()
        got[(a, b)] = int(v)
    for cname, ct in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(ct), cname
        for f, _ in ct._fields_:
            assert got[(cname, f)] == getattr(ct, f).offset, (cname, f)
    assert got[("const", "MXFP8_LORA_BWD_MAX_JOBS")] == _native.LORA_BWD_MAX_JOBS
    assert got[("const", "MXFP8_PACK_MAX_JOBS")] == _native.PACK_MAX_JOBS
    assert got[("const", "MXFP8_LORA_TN_MAX_JOBS")] == _native.LORA_TN_MAX_JOBS
