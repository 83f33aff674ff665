"""ctypes binding of libmxfp8_mlp.so, the gfx950 HIP library behind mxfp8.py and fused_mlp.py.

The C-ABI is declared in include/mxfp8_mlp.h.  Every call passes raw device pointers, sizes and the current
HIP stream of the tensors' device, so launches stay asynchronous and ordered with PyTorch's own work.  There
is no fallback: if the library is missing or does not match this module's ABI version, the first call raises.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmxfp8_mlp.so")
ABI_VERSION = 14
GEMM_A_TILED, GEMM_B_TILED, GEMM_WIDE, GEMM_C_FT, GEMM_B_PI = 1, 2, 4, 8, 16  # mxfp8_gemm_nt layout bits

_i64, _ptr, _f32, _int = ctypes.c_int64, ctypes.c_void_p, ctypes.c_float, ctypes.c_int

# name -> argument types, in the order of include/mxfp8_mlp.h
SIGNATURES = {
    "mxfp8_abi_version": [],
    "mxfp8_last_error": [],
    "mxfp8_quant_rows": [_ptr, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _i64, _ptr],
    "mxfp8_quant_dual": [_ptr, _i64, _i64, _i64, _ptr, _ptr, _ptr, _ptr, _ptr],
    "mxfp8_quant_tiled": [_ptr, _i64, _i64, _i64, _ptr, _ptr, _ptr],
    "mxfp8_tile_codes": [_ptr, _i64, _i64, _i64, _ptr, _ptr],
    "mxfp8_dequant": [_ptr, _i64, _i64, _i64, _ptr, _i64, _ptr, _ptr],
    "mxfp8_gemm_nt": [_ptr, _ptr, _i64, _ptr, _ptr, _i64, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr, _i64,
                      _i64, _f32, _i64, _ptr, _i64, _ptr],
    "mxfp8_gemm_workspace_size": [_i64, _i64, _i64],
    "mxfp8_gemm_swiglu_fwd": [_ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _ptr, _ptr, _ptr, _ptr, _i64, _f32, _f32, _ptr,
                              _ptr, _ptr, _ptr, _ptr],
    "mxfp8_gemm_swiglu_bwd": [_ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64] + [_ptr] * 11 + [_i64, _f32, _f32] + [_ptr] * 7,
    "mxfp8_gemm_nt_seg": [_ptr, _ptr, _i64, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _ptr, _ptr, _ptr, _ptr, _i64,
                          _ptr, _i64, _i64, _ptr, _f32, _i64, _ptr],
    "mxfp8_mlp_fwd_groups": [_i64, _i64, _i64],
    "mxfp8_mlp_fwd": [_ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _f32, _f32, _ptr, _ptr, _ptr, _i64, _ptr, _i64,
                      _ptr],
    "mxfp8_mlp_bwd": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _f32,
                      _f32, _i64, _i64, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _ptr],
    "mxfp8_sum_parts": [_ptr, _i64, _i64, _f32, _ptr, _int, _ptr],
    "mxfp8_lora_prep": [_ptr] * 6 + [_i64, _i64, _i64] + [_ptr] * 10 + [_ptr],
    "mxfp8_lora_nt": [_ptr, _i64, _i64, _i64, _ptr, _i64, _f32, _ptr, _ptr, _i64, _ptr],
    "mxfp8_quant_lora": [_ptr, _i64, _i64, _i64, _ptr, _ptr, _ptr, _i64, _f32, _ptr, _ptr, _i64, _ptr],
    "mxfp8_quant_lora_tp": [_ptr, _i64, _i64, _i64, _ptr, _ptr, _ptr, _i64, _f32, _ptr, _ptr, _i64, _ptr, _i64, _i64,
                            _ptr, _ptr],
    "mxfp8_res_lora": [_ptr, _ptr, _ptr, _i64, _ptr, _i64, _i64, _i64, _f32, _ptr, _ptr],
    "mxfp8_transpose_pad": [_ptr, _i64, _i64, _i64, _ptr, _i64, _ptr],
    "mxfp8_pack_bf16": [_ptr, _i64, _ptr],
    "mxfp8_lora_tn_chunks": [_i64, _i64],
    "mxfp8_swiglu": [_ptr, _ptr, _i64, _ptr, _ptr],
    "mxfp8_swiglu_bwd": [_ptr, _ptr, _ptr, _i64, _ptr, _ptr, _ptr],
    "mxfp8_lora_bwd_chunks": [_i64, _i64],
    "mxfp8_lora_bwd": [_ptr, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _i64, _ptr, _i64, _ptr, _i64, _f32, _ptr, _i64,
                       _ptr, _ptr, _ptr, _ptr],
    "mxfp8_lora_bwd_batch_chunks": [_i64, _i64],
    "mxfp8_lora_bwd_batch": [_ptr, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr],
    "mxfp8_lora_tn": [_ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _ptr, _f32, _i64, _i64, _ptr, _ptr],
    "mxfp8_lora_tn_batch": [_ptr, _i64, _i64, _i64, _i64, _ptr, _ptr],
    "mxfp8_gemm_nt_sum": [_ptr, _ptr, _i64, _ptr, _ptr, _i64, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _f32, _ptr,
                          _ptr, _i64, _i64, _f32, _i64, _i64, _ptr],
    "mxfp8_gemm_nt_tn": [_ptr, _ptr, _i64, _ptr, _ptr, _i64, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr, _i64,
                         _i64, _f32, _i64, _ptr, _i64, _i64, _i64, _i64, _ptr, _ptr],
    "mxfp8_lora_tn_noalloc": [_ptr, _i64, _i64, _i64, _ptr, _i64, _f32, _i64, _i64, _ptr, _ptr],
    "mxfp8_lora_tn_noalloc_chunks": [_i64, _i64, _i64],
    "mxfp8_mlp_bwd_finish": [_ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _f32, _f32, _ptr, _ptr, _ptr, _ptr,
                             _ptr, _ptr],
}

_RESTYPES = {"mxfp8_last_error": ctypes.c_char_p, "mxfp8_gemm_workspace_size": _i64, "mxfp8_mlp_fwd_groups": _i64,
             "mxfp8_lora_tn_chunks": _i64, "mxfp8_lora_bwd_chunks": _i64, "mxfp8_lora_bwd_batch_chunks": _i64,
             "mxfp8_lora_tn_noalloc_chunks": _i64}

_lib = None
_WORKSPACE = {}  # (device index, stream) -> zero-initialised uint8 workspace of the MX GEMM


class NativeError(RuntimeError):
    pass


def load(path=LIB_PATH):
    """Load and type the library (no GPU work)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise NativeError(f"{path} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
                          "or `make -C train-model-template_amd/csrc`; the MXFP8 path has no CPU fallback")
    L = ctypes.CDLL(path)
    for name, args in SIGNATURES.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, _int)
    v = L.mxfp8_abi_version()
    if v != ABI_VERSION:
        raise NativeError(f"{path}: ABI version {v}, expected {ABI_VERSION}; rebuild the library")
    _lib = L
    return L


def _check(rc, name):
    if rc != 0:
        raise NativeError(f"{name} failed with code {rc}: {_lib.mxfp8_last_error().decode()}")


_raw_stream = torch._C._cuda_getCurrentRawStream  # device index -> the current HIP stream, as an int


def _stream(t):
    return _raw_stream(t.get_device())


def _p(t):
    """A tensor's device address as an int (the signatures type it as a pointer), or None; an int passes
    through (an address inside a scratch buffer)."""
    if t is None or isinstance(t, int):
        return t
    return t.data_ptr()


def _gpu(t, what):
    if not t.is_cuda:
        raise NativeError(f"{what}: tensors must be on the GPU (the MXFP8 path has no CPU implementation)")


_FNS = {}  # entry point name -> typed ctypes function


def call(name, *args, like):
    """Call entry point `name` with `args` followed by the current stream of tensor `like`'s device."""
    fn = _FNS.get(name)
    if fn is None:
        fn = _FNS[name] = getattr(load(), name)
    if not like.is_cuda:
        _gpu(like, name)
    rc = fn(*args, _raw_stream(like.get_device()))
    if rc != 0:
        _check(rc, name)


def quant_rows(x, q, s, ld_q=None, s_col_tiles=None, s_tile0=0):
    """x [R, C] bf16 (row stride x.stride(0)) -> codes into q (a [R, >=C] uint8 view, row stride ld_q) and
    blocked scales into s."""
    R, C = x.shape
    ld_q = q.stride(0) if ld_q is None else ld_q
    s_col_tiles = C // 128 if s_col_tiles is None else s_col_tiles
    call("mxfp8_quant_rows", _p(x), R, C, x.stride(0), _p(q), ld_q, _p(s), s_col_tiles, s_tile0, like=x)


def quant_dual(x, q, s, qt, st):
    R, C = x.shape
    call("mxfp8_quant_dual", _p(x), R, C, x.stride(0), _p(q), _p(s), _p(qt), _p(st), like=x)


def quant_tiled(x, q, s):
    """x [R, C] bf16 -> codes in the MX-tiled layout into q (ceil(R/16)*16 * C bytes) and blocked scales."""
    R, C = x.shape
    call("mxfp8_quant_tiled", _p(x), R, C, x.stride(0), _p(q), _p(s), like=x)


def tile_codes(q, rows, cols, out):
    """Row-major codes (row stride q.stride(0)) -> the MX-tiled layout into out."""
    call("mxfp8_tile_codes", _p(q), rows, cols, q.stride(0), _p(out), like=out)


def dequant(q, s, rows, cols, ld_q, s_col_tiles, out):
    call("mxfp8_dequant", _p(q), rows, cols, ld_q, _p(s), s_col_tiles, _p(out), like=out)


def gemm_workspace(M, N, K, device):
    """The GEMM workspace for this shape on the current stream of `device`: one buffer per (device, stream),
    grown on demand and allocated zeroed (its arrival counters must start at zero; every call leaves them
    zero), so calls on one stream, which are ordered, share it safely."""
    need = load().mxfp8_gemm_workspace_size(M, N, K)
    if need <= 0:
        return None, 0
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, _raw_stream(idx))
    ws = _WORKSPACE.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(need, dtype=torch.uint8, device=device)
        _WORKSPACE[key] = ws
    return ws, ws.numel()


_SCRATCH = {}  # (device index, stream) -> float32 scratch of the partial-sum launch pairs


def scratch_f32(n, device):
    """At least n float32 of scratch memory on the current stream of `device`, shared by the launch pairs that
    pass partial sums from one kernel to the next (lora_bwd, lora_bwd_batch, lora_tn): launches on one stream
    run in order, so two pairs never use it at once.  Its contents are undefined; grown on demand (the caching
    allocator reuses a replaced buffer only for later work on the same stream)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, _raw_stream(idx))
    buf = _SCRATCH.get(key)
    if buf is None or buf.numel() < n:
        buf = _SCRATCH[key] = torch.empty(n, dtype=torch.float32, device=device)
    return buf


def gemm_nt(a, sa, lda, b, sb, ldb, M, N, K, c, lora=None, alpha=1.0, split=True, layout=0):
    """c[M, N] = bf16(A·Bᵀ) [+ alpha · P·Qᵀ with lora = (P [M, r], Q [N, r])].  layout bit 0 / 1: A / B codes
    MX-tiled; bit 2 (GEMM_WIDE): 8-wave 256 x 256 workgroups, whose tail tiles split along K through the cached
    workspace unless split=False."""
    if lora is None:
        p = q = None
        ldp = ldq = r = 0
    else:
        p, q = lora
        r = p.shape[1]
        ldp, ldq = p.stride(0), q.stride(0)
    _gpu(c, "mxfp8_gemm_nt")
    ws, ws_bytes = gemm_workspace(M, N, K, c.device) if split and layout & GEMM_WIDE else (None, 0)
    call("mxfp8_gemm_nt", _p(a), _p(sa), lda, _p(b), _p(sb), ldb, M, N, K, _p(c), c.stride(0), _p(p), ldp,
         _p(q), ldq, r, float(alpha), layout, _p(ws), ws_bytes, like=c)


def gemm_nt_seg(a, sa, lda, b, sb, ldb, M, N, K, outs, lora=None, alpha=1.0, layout=0, lora_cols=None, r=None):
    """gemm_nt with the N output columns split over `outs` (1..4 bf16 [M, n_k] matrices, any row stride; the widths
    sum to N, each a multiple of 128).  lora_cols (one per output) with rank r: output k adds the rank-r product
    over columns lora_cols[k] .. + r of P and Q instead of all of them."""
    n = len(outs)
    col0, c0 = [], 0
    for o in outs:
        col0.append(c0)
        c0 += o.shape[1]
    cols = (ctypes.c_int64 * n)(*col0)
    ptrs = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    lds = (ctypes.c_int64 * n)(*[o.stride(0) for o in outs])
    if lora is None:
        p = q = None
        ldp = ldq = r = 0
    else:
        p, q = lora
        r = p.shape[1] if lora_cols is None else r
        ldp, ldq = p.stride(0), q.stride(0)
    rcols = None if lora_cols is None else (ctypes.c_int64 * n)(*lora_cols)
    call("mxfp8_gemm_nt_seg", _p(a), _p(sa), lda, _p(b), _p(sb), ldb, M, N, K, n, cols, ptrs, lds, _p(p), ldp, _p(q),
         ldq, r, rcols, float(alpha), layout, like=outs[0])


GEMM_NT_SUM_MAX = 1 << 26  # M * r that mxfp8_gemm_nt_sum takes (64 K summing workgroups of 1024 values)


def gemm_nt_sum(a, sa, lda, b, sb, ldb, M, N, K, c, part, p_out, q, alpha=1.0, layout=0, part_scale=1.0,
                wait_limit=-1):
    """gemm_nt with the rank-16 epilogue whose P = p_out [M, 16] is summed from part [n, M, 16] in the same launch
    (include/mxfp8_mlp.h, mxfp8_gemm_nt_sum): p_out = bf16(part_scale · Σ part) as sum_parts writes it, then
    c = bf16(bf16(A·Bᵀ) + alpha · p_out · qᵀ).  wait_limit 0: every tile sums its own rows (tests)."""
    _gpu(c, "mxfp8_gemm_nt_sum")
    assert part.dtype == torch.float32 and part.is_contiguous() and p_out.is_contiguous() and p_out.shape == (M, 16)
    call("mxfp8_gemm_nt_sum", _p(a), _p(sa), lda, _p(b), _p(sb), ldb, M, N, K, _p(c), c.stride(0), _p(part),
         part.shape[0], float(part_scale), _p(p_out), _p(q), q.stride(0), 16, float(alpha), layout, int(wait_limit),
         like=c)


def gemm_swiglu_fwd(a, sa, b, sb, M, N, K, xs, bg, bu, ad, s_g, s_u, gu, q_h, s_h, part):
    """gate|up MX GEMM with the SwiGLU forward in its epilogue (include/mxfp8_mlp.h, mxfp8_gemm_swiglu_fwd)."""
    call("mxfp8_gemm_swiglu_fwd", _p(a), _p(sa), _p(b), _p(sb), M, N, K, _p(xs), _p(bg), _p(bu), _p(ad), ad.shape[0],
         float(s_g), float(s_u), _p(gu), _p(q_h), _p(s_h), _p(part), like=gu)


def gemm_swiglu_bwd(a, sa, b, sb, M, N, K, gu, xs, xsT, dxd, dxdT, bg, bgT, bu, buT, ad, adT, s_g, s_u, q, s, dxa_part,
                    dbg_part, dbu_part, dad_part):
    """dgrad MX GEMM of h with the SwiGLU backward in its epilogue (include/mxfp8_mlp.h, mxfp8_gemm_swiglu_bwd)."""
    call("mxfp8_gemm_swiglu_bwd", _p(a), _p(sa), _p(b), _p(sb), M, N, K, _p(gu), _p(xs), _p(xsT), _p(dxd), _p(dxdT),
         _p(bg), _p(bgT), _p(bu), _p(buT), _p(ad), _p(adT), ad.shape[0], float(s_g), float(s_u), _p(q), _p(s),
         _p(dxa_part), _p(dbg_part), _p(dbu_part), _p(dad_part), like=gu)


def mlp_fwd(gu, xs, bg, bu, ad, T, N, r, s_g, s_u, q, s, part, n_groups, h_out=None, q_layout=0):
    call("mxfp8_mlp_fwd", _p(gu), _p(xs), _p(bg), _p(bu), _p(ad), T, N, r, float(s_g), float(s_u), _p(q), _p(s),
         _p(part), n_groups, _p(h_out), q_layout, like=gu)


def mlp_bwd(gu, xs, xsT, dhm, dxd, dxdT, bg, bu, bgT, buT, ad, adT, T, N, r, s_g, s_u, SB, CG, q, s, dxa_part,
            dbg_part, dbu_part, dad_part, dgu_out=None, q_layout=0):
    call("mxfp8_mlp_bwd", _p(gu), _p(xs), _p(xsT), _p(dhm), _p(dxd), _p(dxdT), _p(bg), _p(bu), _p(bgT), _p(buT),
         _p(ad), _p(adT), T, N, r, float(s_g), float(s_u), SB, CG, _p(q), _p(s), _p(dxa_part), _p(dbg_part),
         _p(dbu_part), _p(dad_part), _p(dgu_out), q_layout, like=gu)


def sum_parts(part, n_parts, count, out, scale=1.0):
    """out (fp32 or bf16, `count` elements) = scale * Σ_p part[p] in ascending p."""
    assert out.dtype in (torch.float32, torch.bfloat16) and part.dtype == torch.float32
    call("mxfp8_sum_parts", _p(part), n_parts, count, float(scale), _p(out), int(out.dtype == torch.bfloat16),
         like=part)


def lora_prep(Ag, Au, Bg, Bu, Ad, Bd, out):
    """out: dict of bf16 tensors S, ST, bg, bu, bgT, buT, ad, adT, bd, bdT (see include/mxfp8_mlp.h)."""
    R, K = Ag.shape
    N = Bg.shape[0]
    call("mxfp8_lora_prep", *[_p(t) for t in (Ag, Au, Bg, Bu, Ad, Bd)], R, K, N,
         *[_p(out[k]) for k in ("S", "ST", "bg", "bu", "bgT", "buT", "ad", "adT", "bd", "bdT")], like=Ag)


def lora_nt(x, w, out, scale=1.0, outT=None):
    """out[t, ρ] = bf16(x[t] · w[ρ]) (then · scale); outT [rp, Tpad] optional (zero-padded transposed copy)."""
    T, K = x.shape
    call("mxfp8_lora_nt", _p(x), T, K, x.stride(0), _p(w), w.shape[0], float(scale), _p(out), _p(outT),
         outT.shape[1] if outT is not None else 0, like=x)


def quant_lora(x, q, s, w, out, scale=1.0, outT=None):
    """mxfp8.mx_quant_tiled(x) into (q, s) and lora_nt(x, w, out, scale, outT) from one read of x."""
    T, K = x.shape
    call("mxfp8_quant_lora", _p(x), T, K, x.stride(0), _p(q), _p(s), _p(w), w.shape[0], float(scale), _p(out),
         _p(outT), -(-T // 128) * 128, like=x)


def quant_lora_tp(x, q, s, w, out, tx, tout, scale=1.0, outT=None):
    """quant_lora(x, q, s, w, out, scale, outT) and, in the same launch, tout [C, Tpad] = txᵀ zero-padded
    (transpose_pad of tx [T, C])."""
    T, K = x.shape
    call("mxfp8_quant_lora_tp", _p(x), T, K, x.stride(0), _p(q), _p(s), _p(w), w.shape[0], float(scale), _p(out),
         _p(outT), -(-T // 128) * 128, _p(tx), tx.stride(0), tx.shape[1], _p(tout), like=x)


def res_lora(x, y, xa, b, out, scale):
    """out = bf16(x + bf16(y + scale · xa · bᵀ)); x, y, out [T, N], xa [T, r] (row stride any), b [N, r]."""
    T, N = x.shape
    call("mxfp8_res_lora", _p(x), _p(y), _p(xa), xa.stride(0), _p(b), T, N, b.shape[1], float(scale), _p(out),
         like=x)


def swiglu(g, u, h):
    """h = bf16(silu(g) · u) elementwise (bf16, contiguous, numel % 8 == 0)."""
    call("mxfp8_swiglu", _p(g), _p(u), g.numel(), _p(h), like=g)


def swiglu_bwd(g, u, dh, dg, du):
    call("mxfp8_swiglu_bwd", _p(g), _p(u), _p(dh), g.numel(), _p(dg), _p(du), like=g)


def lora_bwd_chunks(T, N):
    return int(load().mxfp8_lora_bwd_chunks(T, N))


def lora_bwd(dy, q, s, s_col_tiles, col_tile_off, xa, b, scale, dxa, db, part_dxa, part_db):
    """One read of dy [T, N]: MX codes/scales into q/s at column tile col_tile_off (q None: skipped) and, with xa,
    dxa = bf16(scale · dy·b), db = scale · dyᵀ·xa (fp32) through the partial buffers."""
    T, N = dy.shape
    lora = xa is not None
    call("mxfp8_lora_bwd", _p(dy), T, N, dy.stride(0), _p(q), q.stride(0) if q is not None else 0, _p(s),
         s_col_tiles, col_tile_off, _p(xa), xa.stride(0) if lora else 0, _p(b), b.shape[1] if lora else 0,
         float(scale), _p(dxa), dxa.stride(0) if lora else 0, _p(db), _p(part_dxa), _p(part_db), like=dy)


def lora_tn(x, p, out, part, scale=1.0, transpose=False):
    """out = bf16(pᵀ · x) (then · scale), [rp, K] or transposed; part: float scratch (lora_tn_chunks)."""
    T, K = x.shape
    rp = p.shape[1]
    chunks = part.numel() // (rp * K)
    call("mxfp8_lora_tn", _p(x), T, K, x.stride(0), _p(p), rp, chunks, _p(part), float(scale), int(transpose),
         int(out.dtype == torch.float32), _p(out), like=x)


class LoraTnJob(ctypes.Structure):
    """mxfp8_lora_tn_job of include/mxfp8_mlp.h."""
    _fields_ = [("x", _ptr), ("ld_x", _i64), ("p", _ptr), ("rp", _i64), ("scale", _f32), ("transpose", _i64),
                ("out_f32", _i64), ("out", _ptr)]


LORA_TN_MAX_JOBS = 4


def lora_tn_batch(jobs, part, chunks=None):
    """lora_tn of every job [(x, p, out, scale, transpose)] (the same [T, K] for all) in one launch, plus one launch
    of the chunk sums; chunks: token chunks (default lora_tn_chunks(T, K), lora_tn's chunking); part: float
    scratch of at least chunks * Σ rp * K."""
    arr, n, T, K, chunks = _tn_table(jobs, part, chunks)
    call("mxfp8_lora_tn_batch", ctypes.cast(arr, _ptr), n, T, K, chunks, _p(part), like=jobs[0][0])


def _tn_table(jobs, part, chunks):
    """(ctypes job array, n, T, K, chunks) of mxfp8_lora_tn_batch's jobs [(x, p, out, scale, transpose)]."""
    T, K = jobs[0][0].shape
    chunks = lora_tn_chunks(T, K) if chunks is None else int(chunks)
    if part.numel() < chunks * sum(p.shape[1] for _, p, _, _, _ in jobs) * K:
        raise NativeError("lora_tn_batch: partial buffer too small")
    table = [LoraTnJob(_p(x), x.stride(0), _p(p), p.shape[1], float(sc), int(tr), int(out.dtype == torch.float32),
                       _p(out)) for x, p, out, sc, tr in jobs]
    return (LoraTnJob * len(table))(*table), len(table), T, K, chunks


def gemm_nt_tn(a, sa, lda, b, sb, ldb, M, N, K, c, lora, jobs, part, alpha=1.0, layout=0, chunks=None):
    """gemm_nt (rank-16, 32 or 48 lora = (P, Q), 4-wave shape) and lora_tn_batch(jobs, part, chunks) in one launch,
    plus the batch's sums (include/mxfp8_mlp.h, mxfp8_gemm_nt_tn): the token reductions fill the GEMM's idle tail
    slots."""
    p, q = lora
    arr, n, T, Kt, chunks = _tn_table(jobs, part, chunks)
    _gpu(c, "mxfp8_gemm_nt_tn")
    call("mxfp8_gemm_nt_tn", _p(a), _p(sa), lda, _p(b), _p(sb), ldb, M, N, K, _p(c), c.stride(0), _p(p),
         p.stride(0), _p(q), q.stride(0), p.shape[1], float(alpha), layout, ctypes.cast(arr, _ptr), n, T, Kt, chunks,
         _p(part), like=c)


class LoraBwdJob(ctypes.Structure):
    """mxfp8_lora_bwd_job of include/mxfp8_mlp.h."""
    _fields_ = [("dy", _ptr), ("N", _i64), ("ld_dy", _i64), ("col_tile_off", _i64), ("xa", _ptr), ("ld_xa", _i64),
                ("b", _ptr), ("scale", _f32), ("dxa", _ptr), ("ld_dxa", _i64), ("db", _ptr), ("part_dxa", _ptr),
                ("part_db", _ptr)]


LORA_BWD_MAX_JOBS = 8


def lora_bwd_batch_chunks(T, n_total):
    return int(load().mxfp8_lora_bwd_batch_chunks(T, n_total))


def lora_bwd_batch(jobs, T, r, q, s):
    """jobs: [(dy, col_tile_off, xa, B, scale, dxa, db, part_dxa, part_db)] tensors as for lora_bwd; q [T, ΣN]
    uint8 codes and s its scales, or None."""
    table = [LoraBwdJob(_p(dy), dy.shape[1], dy.stride(0), off, _p(xa), xa.stride(0), _p(B), float(sc), _p(dxa),
                        dxa.stride(0), _p(db), _p(pdx), _p(pdb))
             for dy, off, xa, B, sc, dxa, db, pdx, pdb in jobs]
    arr = (LoraBwdJob * len(table))(*table)
    call("mxfp8_lora_bwd_batch", ctypes.cast(arr, _ptr), len(table), T, r, _p(q) if q is not None else None,
         q.stride(0) if q is not None else 0, _p(s) if s is not None else None,
         q.shape[1] // 128 if q is not None else 0, like=jobs[0][0])


class PackJob(ctypes.Structure):
    """mxfp8_pack_job of include/mxfp8_mlp.h."""
    _fields_ = [("src", _ptr), ("src_ld", _i64), ("src_f32", _i64), ("rows", _i64), ("cols", _i64), ("dst", _ptr),
                ("dst_ld", _i64), ("transpose", _i64)]


PACK_MAX_JOBS = 32


def pack_bf16(jobs):
    """Run the bf16 copies `jobs` = [(src, dst, transpose)] in as few launches as the job table allows: src a 2-D
    fp32 or bf16 tensor [rows, cols] with unit column stride, or None for zeros; dst a 2-D bf16 view, [rows, cols]
    or, when transpose, [cols, rows], with unit column stride.  Destinations must not overlap."""
    if jobs:
        pack_run(pack_table(jobs), like=jobs[0][1])


def pack_table(jobs):
    """The job tables of pack_bf16(jobs), built once: a list of (ctypes array, count), at most PACK_MAX_JOBS
    each.  They hold the tensors' addresses, so they stay valid while those tensors live at the same place."""
    table = []
    for src, dst, tr in jobs:
        assert dst.dtype == torch.bfloat16 and dst.dim() == 2 and dst.stride(1) == 1, (dst.dtype, dst.shape)
        rows, cols = (dst.shape[1], dst.shape[0]) if tr else tuple(dst.shape)
        if src is not None:
            assert src.dim() == 2 and src.stride(1) == 1 and tuple(src.shape) == (rows, cols), (src.shape, rows, cols)
            assert src.dtype in (torch.float32, torch.bfloat16) and src.device == dst.device
        table.append(PackJob(None if src is None else _p(src), 0 if src is None else src.stride(0),
                             int(src is not None and src.dtype == torch.float32), rows, cols, _p(dst), dst.stride(0),
                             int(bool(tr))))
    out = []
    for i in range(0, len(table), PACK_MAX_JOBS):
        chunk = table[i:i + PACK_MAX_JOBS]
        out.append(((PackJob * len(chunk))(*chunk), len(chunk)))
    return out


def pack_run(tables, like):
    """Launch the job tables of pack_table on the current stream of `like`'s device."""
    for arr, n in tables:
        call("mxfp8_pack_bf16", ctypes.addressof(arr), n, like=like)


def transpose_pad(x, out):
    """out [C, Tpad] = xᵀ of x [T, C] bf16, zero past T."""
    T, C = x.shape
    call("mxfp8_transpose_pad", _p(x), T, C, x.stride(0), _p(out), out.shape[1], like=x)


def lora_tn_noalloc(x, p, out, scale=1.0, transpose=False):
    """lora_tn with the chunk partials in the library's static scratch (nothing allocated)."""
    T, K = x.shape
    call("mxfp8_lora_tn_noalloc", _p(x), T, K, x.stride(0), _p(p), p.shape[1], float(scale), int(transpose),
         int(out.dtype == torch.float32), _p(out), like=x)


def lora_tn_noalloc_chunks(T, K, rp):
    return int(load().mxfp8_lora_tn_noalloc_chunks(T, K, rp))


def lora_tn_chunks(T, K):
    return int(load().mxfp8_lora_tn_chunks(T, K))


def mlp_bwd_finish(dxa_p, dbg_p, dbu_p, dad_p, T, N, r, s_g, s_u, dxa, xsd, dbg, dbu, dad):
    call("mxfp8_mlp_bwd_finish", _p(dxa_p), _p(dbg_p), _p(dbu_p), _p(dad_p), dxa_p.shape[0], dbg_p.shape[0], T, N, r,
         float(s_g), float(s_u), _p(dxa), _p(xsd), _p(dbg), _p(dbu), _p(dad), like=dxa)
