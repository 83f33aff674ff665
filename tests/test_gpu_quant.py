"""GPU parity of the MX quantizer kernels (libmxfp8_mlp.so via mxfp8.py) against the CPU oracle: codes and
scales must be bit-exact (north star), on the benchmark configurations' activations, the outlier config, the
frozen-weight dual-axis path, column-slice destinations and edge shapes."""
import numpy as np
import pytest
import torch

import mxfp8
import workloads
from oracle import mx

pytestmark = pytest.mark.gpu


def _bytes(t):
    return t.view(torch.uint8).cpu()


def _check_quant(x_cpu, gpu):
    q, s = mxfp8.mx_quant(x_cpu.to(gpu))
    qr, sr = mx.quant(x_cpu)
    assert torch.equal(_bytes(s), sr), "scales differ"
    qd = _bytes(q)
    if not torch.equal(qd, qr):
        bad = (qd != qr).nonzero()[:5].tolist()
        raise AssertionError(f"codes differ at {bad}")


@pytest.mark.parametrize("cfg", [1, 3, 5])
def test_quant_x_configs(cfg, gpu):
    inp = workloads.make_inputs(cfg, dy=(cfg != 1))
    print(f"config {cfg}: x {tuple(inp['x'].shape)}", flush=True)
    _check_quant(inp["x"], gpu)
    if cfg != 1:
        _check_quant(inp["dy"], gpu)


@pytest.mark.parametrize("T", [1, 2, 127, 129, 300, 8896])
def test_quant_ragged_rows(T, gpu):
    g = torch.Generator().manual_seed(T)
    x = (torch.randn(T, 384, generator=g) * torch.exp2(torch.randint(-20, 20, (T, 1), generator=g).float()))
    _check_quant(x.to(torch.bfloat16), gpu)


def test_quant_empty(gpu):
    q, s = mxfp8.mx_quant(torch.empty(0, 256, dtype=torch.bfloat16, device=gpu))
    assert q.shape == (0, 256) and s.numel() == 0


def test_quant_all_bf16_patterns(gpu):
    # every bf16 bit pattern (incl. subnormals, +-0, inf, NaN) in 32-element blocks with random partners
    allv = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    g = torch.Generator().manual_seed(0)
    perm = torch.randperm(65536, generator=g)
    x = allv[perm].view(512, 128)
    _check_quant(x, gpu)
    # and the same values as block maxima over small partners (scale selection on every exponent)
    fin = allv.float()
    fin = fin[torch.isfinite(fin) & (fin != 0)]
    n = fin.numel() // 32 * 32
    base = (torch.rand(n, generator=g) * 0.5 + 0.25)
    blk = (fin[:n].abs().view(-1, 32).amax(1, keepdim=True) * base.view(-1, 32))
    blk[:, 0] = fin[:n].view(-1, 32)[:, 0]
    rows = blk.numel() // 128 * 128
    _check_quant(blk.reshape(-1)[:rows].view(-1, 128).to(torch.bfloat16), gpu)


def test_quant_kat_blocks(gpu):
    vals = [[448.0 * 2.0 ** k] + [0.5 * 2.0 ** k] * 31 for k in range(-20, 21)]
    vals += [[0.0] * 32, [-0.0] * 32, [448.0, 17.0, 19.0, 2.0 ** -10, 3 * 2.0 ** -10, -17.0] + [0.0] * 26,
             [float("inf"), 2.0 ** 127] + [0.0] * 30, [1.0, float("nan")] + [1.0] * 30, [450.0] + [1.0] * 31]
    x = torch.zeros(len(vals), 128)
    for i, v in enumerate(vals):
        x[i, :32] = torch.tensor(v)
        x[i, 32:] = torch.linspace(-3, 3, 96)
    _check_quant(x.to(torch.bfloat16), gpu)


def test_quant_column_slice_destination(gpu):
    # dg into columns [0, N) and du into [N, 2N) of one [T, 2N] buffer (fused_mlp.py:160-162)
    g = torch.Generator().manual_seed(11)
    T, N = 300, 384
    dg = torch.randn(T, N, generator=g).to(torch.bfloat16)
    du = (torch.randn(T, N, generator=g) * 1e-3).to(torch.bfloat16)
    import _native
    q = torch.zeros(T, 2 * N, dtype=torch.uint8, device=gpu)
    s = torch.full((mxfp8.scale_numel(T, 2 * N),), 0xAA, dtype=torch.uint8, device=gpu)
    _native.quant_rows(dg.to(gpu), q, s, s_col_tiles=2 * N // 128, s_tile0=0)
    _native.quant_rows(du.to(gpu), q[:, N:], s, ld_q=2 * N, s_col_tiles=2 * N // 128, s_tile0=N // 128)
    qr, sr = mx.quant(torch.cat([dg, du], 1))
    assert torch.equal(q.cpu(), qr) and torch.equal(s.cpu(), sr)


@pytest.mark.parametrize("shape", [(12288, 2048), (2048, 6144), (7168, 1024), (128, 128), (384, 256)])
def test_quant_both_axes(shape, gpu):
    R, C = shape
    g = torch.Generator().manual_seed(R + C)
    w = (torch.randn(R, C, generator=g) * 0.02).to(torch.bfloat16)
    q, s, qt, st = mxfp8.quant_both(w.to(gpu))
    qr, sr = mx.quant(w)
    qtr, str_ = mx.quant_t(w)
    assert torch.equal(_bytes(q), qr) and torch.equal(_bytes(s), sr)
    assert torch.equal(_bytes(qt), qtr) and torch.equal(_bytes(st), str_)


def test_dequant_matches_oracle(gpu):
    inp = workloads.make_inputs(5, T=512)
    q, s = mxfp8.mx_quant(inp["x"].to(gpu))
    d = mxfp8.dequant(q, s, (512, inp["K"])).cpu()
    qr, sr = mx.quant(inp["x"])
    ref = mx.dequant(qr, sr, 512, inp["K"])
    assert torch.equal(torch.isnan(d), torch.isnan(ref))
    assert torch.equal(d.nan_to_num(), ref.nan_to_num())


@pytest.mark.parametrize("T,K", [(1, 128), (45, 384), (300, 1024), (8896, 2048)])
def test_quant_tiled_layout(T, K, gpu):
    # the GEMM operand layout: the same codes and scales as the oracle, bytes in the MX-tiled order
    g = torch.Generator().manual_seed(T + K)
    x = (torch.randn(T, K, generator=g) * torch.exp2(torch.randint(-10, 10, (T, 1), generator=g).float()))
    x = x.to(torch.bfloat16)
    q, s = mxfp8.mx_quant_tiled(x.to(gpu))
    qr, sr = mx.quant(x)
    assert torch.equal(_bytes(s), sr)
    assert q.shape == (mxfp8.tiled_rows(T), K)
    qt = _bytes(q).numpy().reshape(-1)
    ref = mx.to_tiled(qr.numpy())
    live = mx.from_tiled(qt, T, K)  # padding rows are not written by the quantizer
    assert np.array_equal(live, qr.numpy())
    assert np.array_equal(qt.reshape(-1, K)[:T // 16 * 16], ref.reshape(-1, K)[:T // 16 * 16])


@pytest.mark.parametrize("R,K", [(128, 128), (6144, 2048), (37, 640)])
def test_tile_codes(R, K, gpu):
    g = torch.Generator().manual_seed(R * K)
    q = torch.randint(0, 256, (R, K), generator=g, dtype=torch.uint8)
    out = mxfp8.tile_codes(q.to(gpu).view(torch.float8_e4m3fn))
    assert np.array_equal(_bytes(out).numpy().reshape(-1), mx.to_tiled(q.numpy()))
