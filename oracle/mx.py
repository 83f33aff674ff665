"""CPU oracle for the MXFP8 quantizer and its blocked scale layout.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker; the product path never imports it.

Follows /root/reference/scripts/mxfp8.py:40-86 (quant_ref, _quant_kernel, mx_quant) and
/root/reference/scripts/fused_mlp.py:40-62 (_mx_store).  The element arithmetic lives in mx_oracle.c
(compiled to liboracle_mx.so by oracle/Makefile); this module adds the tensor plumbing, a second restatement of
the blocked layout written the way torchao's ``to_blocked`` builds it (reshape/permute of padded tiles, torchao
0.18.0 ``prototype/mx_formats/utils.py``), its inverse, and dequantization.
"""
import ctypes
import os
import subprocess

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_mx.so")
_lib = None


def build():
    """Compile liboracle_mx.so with the host C compiler (oracle/Makefile)."""
    subprocess.run(["make", "-C", _HERE, "-s", "liboracle_mx.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        i64, p = ctypes.c_int64, ctypes.c_void_p
        L.oracle_e8m0_ieee.argtypes = [ctypes.c_float]
        L.oracle_e8m0_ieee.restype = ctypes.c_int
        L.oracle_e8m0_closed.argtypes = [ctypes.c_uint32]
        L.oracle_e8m0_closed.restype = ctypes.c_int
        L.oracle_e4m3_rne.argtypes = [ctypes.c_float]
        L.oracle_e4m3_rne.restype = ctypes.c_uint8
        L.oracle_e4m3_decode.argtypes = [ctypes.c_uint8]
        L.oracle_e4m3_decode.restype = ctypes.c_float
        L.oracle_blocked_offset.argtypes = [i64, i64, i64]
        L.oracle_blocked_offset.restype = i64
        L.oracle_mx_quant.argtypes = [p, i64, i64, i64, p, i64, i64, p, i64, i64]
        L.oracle_mx_quant.restype = ctypes.c_int
        L.oracle_mx_dequant.argtypes = [p, i64, i64, i64, p, i64, p]
        L.oracle_mx_dequant.restype = ctypes.c_int
        _lib = L
    return _lib


def scale_bytes(rows, cols):
    """Size of the blocked scale buffer of a [rows, cols] operand (mxfp8.py:83-84)."""
    return -(-rows // 128) * (cols // 128) * 512


def quant(x2d):
    """[R, C] bf16 (C % 128 == 0) -> (codes uint8 [R, C], blocked scales uint8 [ceil(R/128)*(C/128)*512]).

    Same contract as mxfp8.mx_quant (mxfp8.py:78-86) but on the CPU and returning raw bytes."""
    assert x2d.dtype == torch.bfloat16 and x2d.dim() == 2 and x2d.shape[1] % 128 == 0, (x2d.dtype, x2d.shape)
    x = x2d.detach().cpu().contiguous()
    R, C = x.shape
    q = torch.empty((R, C), dtype=torch.uint8)
    s = torch.zeros(scale_bytes(R, C), dtype=torch.uint8)
    rc = lib().oracle_mx_quant(x.data_ptr(), R, C, C, q.data_ptr(), C, 0, s.data_ptr(), C // 128, 0)
    assert rc == 0
    return q, s


def quant_into(x2d, q, s, q_col0, s_col_tiles):
    """Column-slice variant (fused_mlp.py:40-62): codes into q[:, q_col0:q_col0+C], scales into the blocked
    layout of the destination width (s_col_tiles tiles per row of tiles) starting at tile q_col0 // 128."""
    x = x2d.detach().cpu().contiguous()
    R, C = x.shape
    assert q.dtype == torch.uint8 and q.is_contiguous() and q_col0 % 128 == 0
    rc = lib().oracle_mx_quant(x.data_ptr(), R, C, C, q.data_ptr(), q.shape[1], q_col0, s.data_ptr(),
                               s_col_tiles, q_col0 // 128)
    assert rc == 0


def quant_t(x2d):
    """Quantization of x2dᵀ along its last axis (mxfp8.py:478, :490: quant_ref(w.t().contiguous()))."""
    return quant(x2d.t().contiguous())


def e8m0_ieee(amax):
    return lib().oracle_e8m0_ieee(float(amax))


def e8m0_closed(bits):
    return lib().oracle_e8m0_closed(int(bits))


def e4m3_rne(x):
    return int(lib().oracle_e4m3_rne(float(x)))


def e4m3_lut():
    """float32 [256]: value of every E4M3FN code (NaN for 0x7f / 0xff)."""
    return np.array([lib().oracle_e4m3_decode(c) for c in range(256)], dtype=np.float32)


def blocked_offset(i, b, n_col_tiles):
    """Scale byte offset of (row i, block b): mxfp8.py:74 / fused_mlp.py:59-61."""
    return ((i // 128) * n_col_tiles + b // 4) * 512 + (i % 32) * 16 + ((i % 128) // 32) * 4 + (b % 4)


def to_blocked_torchao(scales):
    """[R, nb] scale bytes (row-major, one per 32-block) -> flat blocked layout, built the way torchao 0.18.0's
    ``to_blocked`` does it (pad to 128 x 4, split into 128x4 tiles, each tile rearranged as 32 x (4 x 4)).
    An independent restatement of the same layout as ``blocked_offset``; padded entries are 0."""
    R, nb = scales.shape
    nr, nc = -(-R // 128), -(-nb // 4)
    padded = torch.zeros((nr * 128, nc * 4), dtype=scales.dtype)
    padded[:R, :nb] = scales
    blocks = padded.view(nr, 128, nc, 4).permute(0, 2, 1, 3)  # [nr, nc, 128, 4]
    rearranged = blocks.reshape(-1, 4, 32, 4).transpose(1, 2).reshape(-1, 32, 16)
    return rearranged.flatten()


def from_blocked(s_flat, rows, nblk, n_col_tiles=None):
    """Inverse of the blocked layout: flat bytes -> [rows, nblk] (one byte per 32-block)."""
    n_col_tiles = nblk // 4 if n_col_tiles is None else n_col_tiles
    i = torch.arange(rows).view(-1, 1)
    b = torch.arange(nblk).view(1, -1)
    off = blocked_offset(i, b, n_col_tiles)
    return s_flat.view(torch.uint8).reshape(-1)[off.reshape(-1)].view(rows, nblk)


_LUT = None


def dequant(q, s, rows, cols, n_col_tiles=None, ld=None):
    """fp32 [rows, cols] = E4M3(q) * 2^(e - 127); NaN where the scale byte is 0xFF."""
    global _LUT
    if _LUT is None:
        _LUT = torch.from_numpy(e4m3_lut())
    qb = q.view(torch.uint8).cpu()
    if ld is not None and ld != cols:
        qb = qb.view(rows, ld)[:, :cols]
    qb = qb.reshape(rows, cols)
    n_col_tiles = cols // 128 if n_col_tiles is None else n_col_tiles
    e = from_blocked(s.view(torch.uint8).cpu(), rows, cols // 32, n_col_tiles).to(torch.int32)
    vals = _LUT[qb.long()].view(rows, cols // 32, 32)
    out = torch.ldexp(vals, (e - 127).unsqueeze(-1).to(torch.float32))
    out = torch.where((e == 255).unsqueeze(-1), torch.full_like(out, float("nan")), out)
    return out.view(rows, cols)


def to_tiled(q):
    """Row-major codes [R, K] (uint8, K % 64 == 0) -> the MX-tiled GEMM operand layout as a flat uint8 array of
    ceil(R/16)*16*K bytes (padding rows zero): block (r//16, k//64) at ((r//16)*(K//64) + k//64)*1024, row r%16
    at +64*(r%16) of it, and the block's 16-code chunk c of that row at position c ^ ((r >> 2) & 3).  Written as
    a reshape/permute of the padded array.  No reference counterpart: the operand layout of this build's GEMM
    (include/mxfp8_mlp.h, mxfp8_quant_tiled); the reference's codes are row-major (mxfp8.py:46-86)."""
    q = np.asarray(q, dtype=np.uint8)
    R, K = q.shape
    Rp = -(-R // 16) * 16
    a = np.zeros((Rp, K), np.uint8)
    a[:R] = q
    a = a.reshape(Rp // 16, 16, K // 64, 4, 16)  # [rg, r16, kb, chunk, byte]
    out = np.empty_like(a)
    for r in range(16):
        sw = (r >> 2) & 3
        for c in range(4):
            out[:, r, :, c ^ sw, :] = a[:, r, :, c, :]
    return np.ascontiguousarray(out.transpose(0, 2, 1, 3, 4)).reshape(-1)  # [rg, kb, r16, position, byte]


def from_tiled(t, R, K):
    """Inverse of to_tiled: the first R rows of row-major codes [R, K]."""
    Rp = -(-R // 16) * 16
    a = np.asarray(t, dtype=np.uint8).reshape(Rp // 16, K // 64, 16, 4, 16).transpose(0, 2, 1, 3, 4)
    out = np.empty_like(a)
    for r in range(16):
        sw = (r >> 2) & 3
        for c in range(4):
            out[:, r, :, c, :] = a[:, r, :, c ^ sw, :]
    return out.reshape(Rp, K)[:R]


def to_ft(x):
    """Row-major bf16 [R, C] (as uint16, or any element array; C % 32 == 0) -> the fused-tile (FT) layout as a
    flat array of ceil(R/32)*32*C elements (padding rows zero): 32 x 32 blocks, block (r//32, c//32) at
    ((r//32)*(C//32) + c//32)*1024; inside it the 16 columns 16*lg + i of row r%32 belong to lane r%32 + 32*lg,
    and the block holds every lane's i = 0..7 (8 elements per lane, lane order), then every lane's i = 8..15.
    Written as a reshape/permute of the padded array.  No reference counterpart: the order in which this
    build's fused kernels read gu and dhm (include/mxfp8_mlp.h, MXFP8_GEMM_C_FT)."""
    x = np.asarray(x)
    R, C = x.shape
    Rp = -(-R // 32) * 32
    a = np.zeros((Rp, C), x.dtype)
    a[:R] = x
    # [rb, r32, cb, lg, half, e8] -> [rb, cb, half, lg, r32, e8]
    a = a.reshape(Rp // 32, 32, C // 32, 2, 2, 8).transpose(0, 2, 4, 3, 1, 5)
    return np.ascontiguousarray(a).reshape(-1)


def from_ft(t, R, C):
    """Inverse of to_ft: the first R rows of the row-major [R, C] matrix."""
    Rp = -(-R // 32) * 32
    a = np.asarray(t).reshape(Rp // 32, C // 32, 2, 2, 32, 8).transpose(0, 4, 1, 3, 2, 5)
    return np.ascontiguousarray(a).reshape(Rp, C)[:R]
