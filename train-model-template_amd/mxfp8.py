"""MXFP8 GEMMs (E4M3 codes, one E8M0 scale per 32 elements) for the FROZEN weights of LoRA layers, on MI355X.

Drop-in for /root/reference/scripts/mxfp8.py: same names, arguments, return types and layouts.  Every
quantization and MX GEMM runs in the hand-written gfx950 kernels of libmxfp8_mlp.so (see _native.py); there is
no CPU or Triton path, and a CPU tensor is an error.

Layouts (identical to the reference's cuBLAS-compatible ones):
  codes   float8_e4m3fn, row-major, quantized along the last dimension in blocks of 32 (the fused MLP path
          also keeps an MX-tiled copy, the GEMM's operand layout: mx_quant_tiled, tile_codes);
  scales  float8_e8m0fnu, flat, 128x4 blocked: byte of (row i, block b) at
          ((i // 128) * (C // 128) + b // 4) * 512 + (i % 32) * 16 + ((i % 128) // 32) * 4 + b % 4,
          padded rows (up to a multiple of 128) hold 0.

gate_proj + up_proj of one MLP share one quantized copy W_gu = [W_gate; W_up] [2N, K] and its transposed copy
W_guᵀ [K, 2N] (fused_mlp.py runs one forward GEMM and one K = 2N dgrad GEMM).  32-blocks never straddle the
gate/up boundary, so codes and scales equal those of separate copies byte for byte (mxfp8.py:20-23).
"""
import itertools
import os
import types
import weakref

import torch

import _native

F8, E8 = torch.float8_e4m3fn, torch.float8_e8m0fnu
STATS = {"quant": 0, "reuse": 0}  # how often an activation was quantized / reused (for checks)


def _cdiv(a, b):
    return -(-a // b)


def scale_numel(rows, cols):
    """Bytes of the blocked scale buffer of a [rows, cols] operand (mxfp8.py:83-84)."""
    return _cdiv(rows, 128) * (cols // 128) * 512


def mx_quant(x2d):
    """[R, K] contiguous bf16 (K % 128 == 0) -> (fp8 [R, K], flat e8m0 scales in the blocked layout).

    Replaces the Triton _quant_kernel launch of mxfp8.py:78-86."""
    R, K = x2d.shape
    assert x2d.dtype == torch.bfloat16 and x2d.is_contiguous() and K % 128 == 0, (x2d.dtype, x2d.shape)
    q = torch.empty((R, K), dtype=F8, device=x2d.device)
    s = torch.empty(scale_numel(R, K), dtype=torch.uint8, device=x2d.device)
    if R:
        _native.quant_rows(x2d, q, s)
    return q, s.view(E8)


def tiled_rows(R):
    """Rows held by an MX-tiled code buffer of R rows (16-row blocks)."""
    return _cdiv(R, 16) * 16


def ft_rows(R):
    """Rows held by a bf16 buffer of R rows in the fused-tile (FT) layout (32-row blocks)."""
    return _cdiv(R, 32) * 32


def mx_quant_tiled(x2d):
    """mx_quant with the codes in the MX-tiled operand layout of the GEMM (16-row x 64-code blocks of 1 KB, see
    include/mxfp8_mlp.h): same codes and scales in another byte order.  The code tensor is [ceil(R/16)*16, K]
    bytes; pass layout bits to mx_mm.  No reference counterpart (an internal layout of the fused path)."""
    R, K = x2d.shape
    assert x2d.dtype == torch.bfloat16 and x2d.stride(1) == 1 and K % 128 == 0, (x2d.dtype, x2d.shape)
    q = torch.empty((tiled_rows(R), K), dtype=F8, device=x2d.device)
    s = torch.empty(scale_numel(R, K), dtype=torch.uint8, device=x2d.device)
    if R:
        _native.quant_tiled(x2d, q, s)
    return q, s.view(E8)


def mx_quant_lora(x2d, w, scale=1.0, out_t=True):
    """mx_quant_tiled(x2d) and bf16(x2d · wᵀ) (then bf16(· scale)) from one read of x2d, w [rp, K] bf16 with
    rp in {16, 32, 64}: -> (q, s, out [R, rp], outT [rp, ceil(R/128)*128] zero-padded, or None)."""
    R, K = x2d.shape
    assert x2d.dtype == torch.bfloat16 and x2d.stride(1) == 1 and K % 128 == 0 and R > 0, (x2d.dtype, x2d.shape)
    rp = w.shape[0]
    dev = x2d.device
    q = torch.empty((tiled_rows(R), K), dtype=F8, device=dev)
    s = torch.empty(scale_numel(R, K), dtype=torch.uint8, device=dev)
    out = torch.empty((R, rp), dtype=torch.bfloat16, device=dev)
    outT = torch.empty((rp, _cdiv(R, 128) * 128), dtype=torch.bfloat16, device=dev) if out_t else None
    _native.quant_lora(x2d, q, s, w, out, scale=scale, outT=outT)
    return q, s.view(E8), out, outT


def mx_quant_lora_tp(x2d, w, tx, scale=1.0):
    """mx_quant_lora(x2d, w, scale) and, from the same launch, the zero-padded transpose [C, ceil(R/128)*128] of
    tx [R, C] bf16 (C in {16, 32, 64}): -> (q, s, out, outT, txT)."""
    R, K = x2d.shape
    assert x2d.dtype == torch.bfloat16 and x2d.stride(1) == 1 and K % 128 == 0 and R > 0, (x2d.dtype, x2d.shape)
    assert tx.dtype == torch.bfloat16 and tx.shape[0] == R and tx.stride(1) == 1 and tx.shape[1] in (16, 32, 64)
    rp = w.shape[0]
    dev = x2d.device
    tpad = _cdiv(R, 128) * 128
    q = torch.empty((tiled_rows(R), K), dtype=F8, device=dev)
    s = torch.empty(scale_numel(R, K), dtype=torch.uint8, device=dev)
    out = torch.empty((R, rp), dtype=torch.bfloat16, device=dev)
    outT = torch.empty((rp, tpad), dtype=torch.bfloat16, device=dev)
    txT = torch.empty((tx.shape[1], tpad), dtype=torch.bfloat16, device=dev)
    _native.quant_lora_tp(x2d, q, s, w, out, tx, txT, scale=scale, outT=outT)
    return q, s.view(E8), out, outT, txT


def res_lora(x, y, xa, B, scale):
    """x + (y + scale * xa @ Bᵀ) for x, y [T, N] bf16 contiguous, xa [T, r] (any row stride), B [N, r] contiguous:
    out = bf16(x + bf16(y + scale · xa·Bᵀ)), the LoRA-B addmm_ and the residual add in one pass
    (mxfp8.py:285-293).  r in {16, 32} (the LoRA ranks this build supports)."""
    T, N = x.shape
    assert T * N < 2 ** 31 and N % 128 == 0, (x.shape,)
    assert x.dtype == y.dtype == xa.dtype == B.dtype == torch.bfloat16 and x.is_contiguous() and y.is_contiguous()
    assert B.is_contiguous() and xa.stride(1) == 1 and B.shape == (N, xa.shape[1]) and xa.shape[0] == T
    assert xa.shape[1] in (16, 32), "res_lora: LoRA rank must be 16 or 32"
    out = torch.empty_like(x)
    if T:
        _native.res_lora(x, y, xa, B, out, scale)
    return out


def lora_bwd(dy, xa=None, B=None, scale=1.0, q=None, s=None, col_tile_off=0, dxa_out=None):
    """One read of dy [T, N] bf16 (unit column stride) for the backward of a LoRA-carrying MX linear
    (mxfp8.py:202-262, same arguments and result):
    - q/s given: MX codes of dy into columns col_tile_off*128 .. of q [T, ΣN] (row-major) and its scales into the
      blocked layout of q (q.shape[1] / 128 column tiles), byte for byte mx_quant(dy);
    - xa [T, r] (unit column stride, any row stride), B [N, r] contiguous given: writes bf16(scale · dy @ B) into
      dxa_out [T, r] (any row stride) and returns dB = scale · dyᵀ @ xa in fp32; otherwise returns None.
    r in {16, 32} (the LoRA ranks this build supports)."""
    T, N = dy.shape
    assert dy.dtype == torch.bfloat16 and dy.stride(1) == 1 and N % 128 == 0, (dy.dtype, dy.shape, dy.stride())
    has_lora, do_q = xa is not None, q is not None
    if not (has_lora or do_q) or T == 0:
        return None if not has_lora else torch.zeros((N, xa.shape[1]), dtype=torch.float32, device=dy.device)
    dev = dy.device
    db = part_dxa = part_db = None
    if do_q:
        assert q.is_contiguous() and q.dim() == 2 and q.shape[0] == T and s is not None
        assert s.numel() >= scale_numel(T, q.shape[1]) and (col_tile_off * 128 + N) <= q.shape[1]
    if has_lora:
        R = xa.shape[1]
        assert R in (16, 32), "lora_bwd: LoRA rank must be 16 or 32"
        assert xa.dtype == B.dtype == torch.bfloat16 and xa.stride(1) == 1 and B.is_contiguous()
        assert B.shape == (N, R) and xa.shape[0] == T and dxa_out is not None and dxa_out.shape == (T, R)
        assert dxa_out.stride(1) == 1 and dxa_out.dtype == torch.bfloat16
        db = torch.empty((N, R), dtype=torch.float32, device=dev)
        # the partial sums [N / 128, T, R] and [row chunks, N, R] live only until the launch's sum kernel
        n_dxa = _cdiv((N // 128) * T * R, 64) * 64
        part_dxa = _native.scratch_f32(n_dxa + _native.lora_bwd_chunks(T, N) * N * R, dev).data_ptr()
        part_db = part_dxa + 4 * n_dxa
    _native.lora_bwd(dy, q.view(torch.uint8) if do_q else None, s.view(torch.uint8) if do_q else None,
                     q.shape[1] // 128 if do_q else 0, col_tile_off, xa, B, scale, dxa_out, db, part_dxa, part_db)
    return db


def lora_bwd_batch(dys, xas, Bs, scales, dxa_outs, q=None, s=None, col_tile_offs=None):
    """lora_bwd of the layers of a group (one shared T and rank r) in one launch and one launch of their partial
    sums (mxfp8_lora_bwd_batch): every dy streams at once, with one row chunking for all.  Same arguments per
    layer as lora_bwd; returns the layers' dB (fp32).  d(xa) is the same bits as lora_bwd's; dB adds its row
    chunks in another grouping (fp32 rounding)."""
    T, R = dys[0].shape[0], xas[0].shape[1]
    assert 1 <= len(dys) <= _native.LORA_BWD_MAX_JOBS and R in (16, 32) and T > 0, (len(dys), R, T)
    if q is not None:
        assert q.is_contiguous() and q.dim() == 2 and q.shape[0] == T and s is not None
        assert s.numel() >= scale_numel(T, q.shape[1])
    Ns = [d.shape[1] for d in dys]
    rs = _native.lora_bwd_batch_chunks(T, sum(Ns))
    dev = dys[0].device
    # every job's partial sums ([N / 128, T, R] and [rs, N, R], live only until the sum launch) in the scratch
    sizes = [_cdiv(n // 128 * T * R, 64) * 64 + _cdiv(rs * n * R, 64) * 64 for n in Ns]
    addr = _native.scratch_f32(sum(sizes), dev).data_ptr()
    jobs, dbs = [], []
    for k, (dy, xa, B, sc, dxa) in enumerate(zip(dys, xas, Bs, scales, dxa_outs)):
        N = Ns[k]
        assert dy.dtype == xa.dtype == B.dtype == dxa.dtype == torch.bfloat16 and dy.shape[0] == T and N % 128 == 0
        assert dy.stride(1) == 1 and xa.stride(1) == 1 and B.is_contiguous() and B.shape == (N, R)
        assert xa.shape == (T, R) and dxa.shape == (T, R) and dxa.stride(1) == 1
        db = torch.empty((N, R), dtype=torch.float32, device=dev)
        part_dxa, part_db = addr, addr + 4 * _cdiv(N // 128 * T * R, 64) * 64
        addr += 4 * sizes[k]
        off = col_tile_offs[k] if col_tile_offs is not None else 0
        jobs.append((dy, off, xa, B, sc, dxa, db, part_dxa, part_db))
        dbs.append(db)
    _native.lora_bwd_batch(jobs, T, R, q.view(torch.uint8) if q is not None else None,
                           s.view(torch.uint8) if q is not None else None)
    return dbs


def tile_codes(q):
    """Row-major codes [R, K] (any row stride) -> the MX-tiled layout ([ceil(R/16)*16, K] bytes)."""
    R, K = q.shape
    out = torch.empty((tiled_rows(R), K), dtype=F8, device=q.device)
    if R:
        _native.tile_codes(q, R, K, out)
    return out


def quant_ref(x2d):
    """Quantization of a frozen weight (mxfp8.py:40-43: torchao to_mx RCEIL + to_blocked).  Same arithmetic
    and layout as mx_quant, which is what runs here."""
    x = x2d.contiguous()
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    return mx_quant(x)


def quant_both(w):
    """One read of a bf16 weight [R, C] -> (q [R, C], s) along C and (qt [C, R], st) along R, i.e.
    quant_ref(w) and quant_ref(w.t().contiguous()) of mxfp8.py:477-478 / :488-490 in one pass."""
    w = w.contiguous()
    R, C = w.shape
    assert w.dtype == torch.bfloat16 and R % 128 == 0 and C % 128 == 0, (w.dtype, w.shape)
    q = torch.empty((R, C), dtype=F8, device=w.device)
    s = torch.empty(scale_numel(R, C), dtype=torch.uint8, device=w.device)
    qt = torch.empty((C, R), dtype=F8, device=w.device)
    st = torch.empty(scale_numel(C, R), dtype=torch.uint8, device=w.device)
    _native.quant_dual(w, q, s, qt, st)
    return q, s.view(E8), qt, st.view(E8)


def dequant(q, s, shape):
    """fp32 tensor of `shape` [R, C] = E4M3(q) · 2^(e - 127) (NaN where e = 0xFF).  The reference has no such
    function; it dequantizes only inside torch._scaled_mm."""
    R, C = shape
    out = torch.empty((R, C), dtype=torch.float32, device=q.device)
    if R:
        _native.dequant(q, s, R, C, q.stride(0), C // 128, out)
    return out


GEMM_EVENTS = None  # set to a list to record (start event, end event, flops) around every MX GEMM launch


def mx_mm_seg(q, s, wq, ws, outs, lora=None, alpha=1.0, layout=0, m=None, lora_cols=None, r=None):
    """mx_mm whose N output columns go to the separate [M, n_k] tensors `outs` (consecutive column ranges, each a
    multiple of 128 wide); 4-wave shape, row-major outputs.  lora_cols / r: output k's rank-r window of the LoRA
    operands (mxfp8_gemm_nt_seg's seg_rcol)."""
    M, K = q.shape
    if m is not None:
        M = m
    N = wq.shape[0]
    assert sum(o.shape[1] for o in outs) == N and all(o.shape[0] == M for o in outs), ([o.shape for o in outs], N)
    if M:
        ev = GEMM_EVENTS
        if ev is not None:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
        _native.gemm_nt_seg(q, s, q.stride(0), wq, ws, wq.stride(0), M, N, K, outs, lora=lora, alpha=alpha,
                            layout=layout, lora_cols=lora_cols, r=r)
        if ev is not None:
            e1.record()
            ev.append((e0, e1, 2 * M * N * K))
    return outs


def mx_mm(q, s, wq, ws, out=None, lora=None, alpha=1.0, layout=0, m=None):
    """bf16 [M, N] = MX(q [M, K]) · MX(wq [N, K])ᵀ, i.e. torch._scaled_mm(q, wq.t(), s, ws, out_dtype=bf16).
    wq may be a row slice/stride view (row stride wq.stride(0)); optional rank-r epilogue
    out = bf16(out + alpha · P · Qᵀ) with lora = (P [M, r], Q [N, r]) (the addmm_ after the GEMM).
    layout bit 0 / 1: q / wq hold MX-tiled codes (mx_quant_tiled, tile_codes); then M = m (q has the rows
    padded to 16).  Bit 2: 8-wave 256 x 256 workgroups (see _native.gemm_nt).  Bit 3: out in the fused-tile
    layout (pass out with ft_rows(M) rows).  Bit 4: wq rows in the pi_col order of fused_dgrad_rows (Q in row
    order), out the same matrix stored in 16-byte pieces."""
    M, K = q.shape
    if m is not None:
        M = m
    N = wq.shape[0]
    assert wq.shape[1] == K and q.stride(1) == 1 and wq.stride(1) == 1, (q.shape, wq.shape)
    assert not (layout & 1) or q.shape[0] == tiled_rows(M), (q.shape, M)
    if out is None:
        out = torch.empty((ft_rows(M) if layout & 8 else M, N), dtype=torch.bfloat16, device=q.device)
    if M:
        ev = GEMM_EVENTS
        if ev is not None:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
        _native.gemm_nt(q, s, q.stride(0), wq, ws, wq.stride(0), M, N, K, out, lora=lora, alpha=alpha,
                        layout=layout)
        if ev is not None:
            e1.record()
            ev.append((e0, e1, 2 * M * N * K))
    return out


def mx_mm_sum(q, s, wq, ws, part, p_out, lq, alpha, layout, m, wait_limit=-1):
    """mx_mm with the rank-16 epilogue lora = (p_out, lq), its P = p_out summed from the fp32 partials part [n, m, 16]
    in the same launch (p_out = bf16(Σ part), as _native.sum_parts writes it): the MLP forward's xS_down sum and
    down GEMM (/root/reference/scripts/fused_mlp.py:214, :283-284).  Same results as sum_parts then mx_mm."""
    M, K = q.shape
    M = m
    N = wq.shape[0]
    assert wq.shape[1] == K and q.stride(1) == 1 and wq.stride(1) == 1, (q.shape, wq.shape)
    assert not (layout & 1) or q.shape[0] == tiled_rows(M), (q.shape, M)
    out = torch.empty((ft_rows(M) if layout & 8 else M, N), dtype=torch.bfloat16, device=q.device)
    ev = GEMM_EVENTS
    if ev is not None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
    _native.gemm_nt_sum(q, s, q.stride(0), wq, ws, wq.stride(0), M, N, K, out, part, p_out, lq, alpha=alpha,
                        layout=layout, wait_limit=wait_limit)
    if ev is not None:
        e1.record()
        ev.append((e0, e1, 2 * M * N * K))
    return out


def mx_mm_tn(q, s, wq, ws, lora, alpha, layout, m, tn_jobs, part):
    """mx_mm with the rank-16, 32 or 48 LoRA epilogue, and the token reductions _native.lora_tn_batch(tn_jobs,
    part) run in the same launch (in the workgroup slots the GEMM's last round of tiles leaves idle), plus their
    sums: the MLP backward's dx GEMM and its dB_d / dA reductions (/root/reference/scripts/fused_mlp.py:331,
    :316-318, :333), and the grouped linears' dx GEMM and dA (/root/reference/scripts/fused_linear.py:269, :271).
    Same results as mx_mm then lora_tn_batch."""
    M, K = q.shape
    M = m
    N = wq.shape[0]
    assert wq.shape[1] == K and q.stride(1) == 1 and wq.stride(1) == 1, (q.shape, wq.shape)
    assert not (layout & 1) or q.shape[0] == tiled_rows(M), (q.shape, M)
    out = torch.empty((ft_rows(M) if layout & 8 else M, N), dtype=torch.bfloat16, device=q.device)
    ev = GEMM_EVENTS
    if ev is not None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
    _native.gemm_nt_tn(q, s, q.stride(0), wq, ws, wq.stride(0), M, N, K, out, lora, tn_jobs, part, alpha=alpha,
                       layout=layout)
    if ev is not None:
        e1.record()
        ev.append((e0, e1, 2 * M * N * K))
    return out


def swiglu_gemm(q, s, hold, xs, bg, bu, ad, s_g, s_u, m):
    """The gate|up MX GEMM of the fused MLP with the SwiGLU forward in its epilogue: q, s the MX-tiled codes and
    scales of x [m, K]; hold the _GateUp copy (its fused-order operand).  -> (gu [ft_rows(m), 2N] bf16 in the
    fused-tile layout, q_h [tiled_rows(m), N] MX-tiled codes of h, s_h its blocked scales, part [2N/128, m, r]
    fp32 xS_down partials).  One launch for torch._scaled_mm + _fwd_kernel (fused_mlp.py:279-282, :65-109)."""
    n, K = hold.n, hold.w.shape[1]
    r = ad.shape[0]
    dev = q.device
    gu = torch.empty((ft_rows(m), 2 * n), dtype=torch.bfloat16, device=dev)
    qh = torch.empty((tiled_rows(m), n), dtype=F8, device=dev)
    sh = torch.empty(scale_numel(m, n), dtype=torch.uint8, device=dev)
    part = torch.empty((2 * n // 128, m, r), dtype=torch.float32, device=dev)
    ev = GEMM_EVENTS
    if ev is not None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
    _native.gemm_swiglu_fwd(q, s, hold.wf_tl, hold.wfs, m, n, K, xs, bg, bu, ad, s_g, s_u, gu, qh, sh, part)
    if ev is not None:
        e1.record()
        ev.append((e0, e1, 2 * m * 2 * n * K))
    return gu, qh, sh.view(E8), part


def swiglu_bwd_gemm(q, s, down, gu, xs, xsT, dxd, dxdT, bg, bgT, bu, buT, ad, adT, s_g, s_u, m):
    """The dgrad GEMM dhm = MX(dy) · W_down of the fused MLP with the SwiGLU backward in its epilogue: q, s the
    MX-tiled codes and scales of dy [m, K]; down the MX down_proj (its dgrad-order operand).  -> (q_dgu
    [tiled_rows(m), 2N] MX-tiled codes of dg | du, s_dgu its blocked scales, (dxa_p [N/128, m, 3r], dbg_p, dbu_p
    [ceil(m/256), N, r], dad_p [ceil(m/256), r, N]) fp32 partials).  One launch for torch._scaled_mm + _bwd_kernel
    (fused_mlp.py:307-314, :112-175); dhm is never stored."""
    wtf, wtfs = dgrad_rows_operand(down)
    n, K = wtf.shape
    r = ad.shape[0]
    dev = q.device
    qg = torch.empty((tiled_rows(m), 2 * n), dtype=F8, device=dev)
    sg = torch.empty(scale_numel(m, 2 * n), dtype=torch.uint8, device=dev)
    nsb = _cdiv(m, 256)
    dxa_p = torch.empty((n // 128, m, 3 * r), dtype=torch.float32, device=dev)
    dbg_p = torch.empty((nsb, n, r), dtype=torch.float32, device=dev)
    dbu_p = torch.empty((nsb, n, r), dtype=torch.float32, device=dev)
    dad_p = torch.empty((nsb, r, n), dtype=torch.float32, device=dev)
    ev = GEMM_EVENTS
    if ev is not None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
    _native.gemm_swiglu_bwd(q, s, wtf, wtfs, m, n, K, gu, xs, xsT, dxd, dxdT, bg, bgT, bu, buT,
                            ad, adT, s_g, s_u, qg, sg, dxa_p, dbg_p, dbu_p, dad_p)
    if ev is not None:
        e1.record()
        ev.append((e0, e1, 2 * m * n * K))
    return qg, sg.view(E8), (dxa_p, dbg_p, dbu_p, dad_p)


# ---------------------------------------------------------------- generic MX linear (mxfp8.py:296-341)
class _ActivationMemo:
    """The codes of the activation an MX linear quantized last, keyed by (weak reference, version).  Linears that
    read one input back to back (q/k/v, qkv/z, gate/up outside the fused MLP) quantize it once.  The weak
    reference keeps no activation alive, and a dead one never matches a new tensor that reuses the address; an
    in-place change bumps the version (mxfp8.py:296-312)."""

    __slots__ = ("ref", "version", "codes")

    def __init__(self):
        self.forget()

    def forget(self):
        self.ref, self.version, self.codes = None, -1, None

    def lookup(self, x):
        live = self.ref() if self.ref is not None else None
        return self.codes if (live is x and self.version == x._version) else None

    def remember(self, x, codes):
        self.ref, self.version, self.codes = weakref.ref(x), x._version, codes


_ACT = _ActivationMemo()


def _rows_bf16(t):
    """[..., C] -> a contiguous bf16 [R, C] matrix (a view when t already is one)."""
    t2 = t.reshape(-1, t.shape[-1])
    return t2 if t2.dtype == torch.bfloat16 and t2.is_contiguous() else t2.to(torch.bfloat16).contiguous()


def _quant_act(x):
    """(codes, scales) of a linear layer's input, reused when x is the live tensor quantized last, at the same
    version; STATS counts both cases."""
    codes = _ACT.lookup(x)
    if codes is not None:
        STATS["reuse"] += 1
        return codes
    codes = mx_quant(_rows_bf16(x))
    STATS["quant"] += 1
    _ACT.remember(x, codes)
    return codes


class _MXLinear(torch.autograd.Function):
    """x·Wᵀ of a frozen MX weight from the input's codes; backward dx = MX(dy)·W through the weight's second
    quantization axis (mx_wt).  The weight has no gradient (mxfp8.py:315-333)."""

    @staticmethod
    def forward(ctx, x, q, s, lin):
        ctx.lin = lin
        y = mx_mm(q, s, lin._mx_w, lin._mx_ws)
        return y.view(x.shape[:-1] + (y.shape[-1],))

    @staticmethod
    def backward(ctx, dy):
        qd, sd = mx_quant(_rows_bf16(dy))
        STATS["quant"] += 1
        dx = mx_mm(qd, sd, *mx_wt(ctx.lin))
        return dx.view(dy.shape[:-1] + (dx.shape[-1],)), None, None, None


@torch.compiler.disable
def _forward(self, x):
    """The forward enable_mxfp8 installs on a frozen linear (outside any torch.compile region, as the reference
    keeps it: mxfp8.py:336-341)."""
    return _MXLinear.apply(x, *_quant_act(x), self)


# ---------------------------------------------------------------- which linears, grouped how (mxfp8.py:345-366)
# leaf names of the decoder-layer linears that run on MX GEMMs
_NAMES = frozenset({"q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj", "in_proj_qkv",
                    "in_proj_z", "out_proj"})
# Sibling layers whose Wᵀ is kept once, concatenated along N, so that dx of the group is one GEMM over the
# concatenated dy codes.  Every N is a multiple of 128, so no 32-block straddles two layers and each layer's
# codes and scales equal its own quantization.  gate/up/down go through fused_mlp instead.
_CATS = (("in_proj_qkv", "in_proj_z"), ("q_proj", "k_proj", "v_proj"))
# Linears whose backward takes the grouped path of fused_linear._Group (one read of dy through lora_bwd)
FUSED_BWD = {"in_proj_qkv", "in_proj_z", "q_proj", "k_proj", "v_proj", "o_proj", "out_proj"}
FUSE_GU = os.environ.get("MXFP8_FUSE_GU", "1") != "0"
# what enable_mxfp8 attaches to a linear (disable_mxfp8 removes exactly these)
_MX_ATTRS = ("_mx_w", "_mx_ws", "_mx_wt", "_mx_wts", "_mx_w_tl", "_mx_wt_tl", "_mx_wtf_tl", "_mx_wtfs", "_mx_wp_tl",
             "_mx_wps", "_mx_cat", "_mx_gu", "_mx_fbwd", "_mx_ops", "_bf16_cpu", "forward")


def _mx_target(name, mod):
    """(leaf name, owner path) of a frozen base linear of a decoder layer that takes MX GEMMs, else None.  A PEFT
    wrapper's base_layer counts under the wrapper's name."""
    if not isinstance(mod, torch.nn.Linear) or mod.weight.requires_grad or ".layers." not in name:
        return None
    path = name.split(".")
    if path[-1] == "base_layer":
        path.pop()
    leaf = path.pop()
    return (leaf, ".".join(path)) if leaf in _NAMES else None


def _base_linears(model):
    """(name, linear) of every module _mx_target accepts, in module order."""
    return ((name, mod) for name, mod in model.named_modules() if _mx_target(name, mod) is not None)


def _col_tiles(scales, rows, cols, c0, c1):
    """The blocked scales of columns [c0, c1) of an MX operand [rows, cols] quantized along its columns: in every
    128-row tile row, the 512-byte tiles of that column range, cut out contiguously (c0, c1 multiples of 128).
    Byte for byte the quantization of those columns alone."""
    tiles = scales.view(torch.uint8).view(_cdiv(rows, 128), cols // 128, 512)
    return tiles[:, c0 // 128:c1 // 128].contiguous().view(-1).view(E8)


def fused_swiglu_rows(n, device=None):
    """Row order of W_gu = [W_gate; W_up] [2n, K] for the gate|up GEMM with the fused SwiGLU epilogue
    (mxfp8_gemm_swiglu_fwd): output tile t (128 columns) takes gate rows 64t..64t+63, then up rows n + 64t..,
    and inside each 32-row block row a is logical row pi_col(a) = ((a >> 2) & 1) * 16 + (a >> 3) * 4 + (a & 3), so
    that every lane of the epilogue holds 16 contiguous gate and up columns of one token."""
    c = torch.arange(2 * n, device=device)
    t, within = c // 128, c % 128
    half, blk, a = within // 64, (within % 64) // 32, within % 32
    pi = ((a >> 2) & 1) * 16 + (a >> 3) * 4 + (a & 3)
    return half * n + 64 * t + 32 * blk + pi


def fused_dgrad_rows(n, device=None):
    """Row order of W_downᵀ [n, K] for the dgrad GEMM with the fused SwiGLU backward (mxfp8_gemm_swiglu_bwd): inside
    each 32-row block row a is logical row pi_col(a), so that every lane of the epilogue holds 16 contiguous
    columns of dhm, the columns it also reads of gu."""
    c = torch.arange(n, device=device)
    a = c % 32
    return c - a + ((a >> 2) & 1) * 16 + (a >> 3) * 4 + (a & 3)


class _GateUp:
    """The one MX copy that gate_proj and up_proj of an MLP share (`_mx_gu = (hold, 0 | 1)`): W_gu = [W_gate;
    W_up] [2N, K] along K (w, ws) for the one forward GEMM and W_guᵀ [K, 2N] along 2N (wt, wts) for the one
    K = 2N dgrad GEMM, both from one read, with MX-tiled copies for the fused MLP (w_tl, wt_tl).  The scale tile
    rows of ws are ordered by row, so its first half is gate's (mxfp8.py:472-484).  half_t caches the per-half
    dgrad operands that mx_wt cuts out.  wf_tl / wfs: the forward operand again, in the row order of the GEMM
    with the fused SwiGLU epilogue (fused_swiglu_rows; the same codes, rows permuted, scales re-blocked)."""

    def __init__(self, gate_w, up_w):
        self.n = gate_w.shape[0]
        w = torch.cat([gate_w, up_w]).to(torch.bfloat16)
        self.w, self.ws, self.wt, self.wts = quant_both(w)
        self.w_tl, self.wt_tl = tile_codes(self.w), tile_codes(self.wt)
        self.wf_tl, self.wfs = mx_quant_tiled(w[fused_swiglu_rows(self.n, w.device)].contiguous())
        # the dgrad operand W_guᵀ [K, 2N] with its rows in the pi_col order (MXFP8_GEMM_B_PI)
        wt = w.t()
        self.wtp_tl, self.wtps = mx_quant_tiled(wt[fused_dgrad_rows(wt.shape[0], w.device)].contiguous())
        self.half_t = [None, None]

    def rows(self, i):
        half = self.ws.numel() // 2
        return self.w[i * self.n:(i + 1) * self.n], self.ws[i * half:(i + 1) * half]


class _Cat:
    """One MX copy of a group's weights concatenated along N, [ΣN, K]: the forward codes along K (w, ws; each
    layer's are a row range) and Wᵀ [K, ΣN] along ΣN (qt, st), from one read, with MX-tiled copies (w_tl, qt_tl).
    offs are the layers' first columns of Wᵀ (mxfp8.py:369-395)."""

    def __init__(self, lins):
        self.n = len(lins)
        self.offs = list(itertools.accumulate((lin.weight.shape[0] for lin in lins), initial=0))
        self.w, self.ws, self.qt, self.st = quant_both(torch.cat([lin.weight.data for lin in lins]).to(torch.bfloat16))
        self.w_tl, self.qt_tl = tile_codes(self.w), tile_codes(self.qt)
        self._cuts = {}

    def fwd_rows(self, k):
        """(codes, scales, tiled codes) of layer k's forward operand: rows offs[k]..offs[k+1] of w."""
        c0, c1 = self.offs[k], self.offs[k + 1]
        per_tile_row = (self.w.shape[1] // 128) * 512  # scale bytes of one 128-row tile row
        return self.w[c0:c1], self.ws[c0 // 128 * per_tile_row:c1 // 128 * per_tile_row], self.w_tl[c0:c1]

    def range(self, a, b):
        """(mat2 [N_a + .. + N_(b-1), K] as a column-major view of Wᵀ, scales) of layers a..b-1, the form
        torch._scaled_mm takes; the scales of a partial range are cut out on first use and kept."""
        c0, c1 = self.offs[a], self.offs[b]
        if (a, b) == (0, self.n):
            return self.qt.t(), self.st
        if (a, b) not in self._cuts:
            self._cuts[(a, b)] = _col_tiles(self.st, self.qt.shape[0], self.qt.shape[1], c0, c1)
        return self.qt[:, c0:c1].t(), self._cuts[(a, b)]


def is_mx(lin):
    return getattr(lin, "_mx_w", None) is not None


def _cat_span(lins):
    """(group, first index) when `lins` are consecutive layers of one concatenated group, else None."""
    tags = [lin.__dict__.get("_mx_cat") for lin in lins]
    if tags[0] is None:
        return None
    cat, k = tags[0]
    return (cat, k) if all(t is not None and t[0] is cat and t[1] == k + d for d, t in enumerate(tags)) else None


def mx_wt(lin):
    """(fp8 Wᵀ [K, N], scales): the B operand of dx = dy · W in mx_mm's form (mxfp8.py:402-415).  A gate/up half
    is a column view of the shared W_guᵀ (row stride 2N) with its scale tiles cut out on first use; a layer of a
    concatenated group, its column range of the group's Wᵀ; any other MX linear, its own Wᵀ."""
    pair = lin.__dict__.get("_mx_gu")
    if pair is not None:
        hold, i = pair
        if hold.half_t[i] is None:
            n, k = hold.n, hold.wt.shape[0]
            hold.half_t[i] = (hold.wt[:, i * n:(i + 1) * n], _col_tiles(hold.wts, k, 2 * n, i * n, (i + 1) * n))
        return hold.half_t[i]
    tag = lin.__dict__.get("_mx_cat")
    if tag is not None:
        mat2, sc = tag[0].range(tag[1], tag[1] + 1)
        return mat2.t(), sc
    return lin._mx_wt, lin._mx_wts


def wt_of(lin):
    """(mat2 [N, K] = Wᵀ as a column-major view, scales): mx_wt in the torch._scaled_mm form (mxfp8.py:418-426)."""
    wt, sc = mx_wt(lin)
    return wt.t(), sc


def group_wt(lins):
    """(mat2 [ΣN, K], scales) of dx = [dy_1 | dy_2 | ..] · [W_1; W_2; ..] for consecutive layers of one concatenated
    group, or of a single ungrouped layer; None otherwise (mxfp8.py:429-439)."""
    span = _cat_span(lins)
    if span is not None:
        return span[0].range(span[1], span[1] + len(lins))
    if len(lins) == 1 and "_mx_cat" not in lins[0].__dict__:
        return wt_of(lins[0])
    return None


def group_fwd_operand(lins):
    """(MX-tiled B operand [ΣN, K] of one forward GEMM over consecutive layers of a concatenated group, scales),
    or None when the layers are not such a range.  No reference counterpart (the reference runs one GEMM per
    layer)."""
    span = _cat_span(lins)
    if span is None:
        return None
    cat, k = span
    memo = cat.__dict__.setdefault("_ops", {})
    key = ("fwd", k, len(lins))
    if key not in memo:
        c0, c1 = cat.offs[k], cat.offs[k + len(lins)]
        per_tile_row = (cat.w.shape[1] // 128) * 512
        memo[key] = (cat.w_tl[c0:c1], cat.ws[c0 // 128 * per_tile_row:c1 // 128 * per_tile_row])
    return memo[key]


def group_operand(lins):
    """(B operand [K, ΣN] of mx_mm, scales, layout bit) of dx for `lins` (group_wt): the MX-tiled copy when the
    range is a whole concatenated group or a single layer that has one, else the row-major column view (row
    stride ΣN of the group).  Kept on the group (or the layer) after the first call: the MX copies are fixed
    from enable_mxfp8 on."""
    span = _cat_span(lins)
    memo = span[0].__dict__.setdefault("_ops", {}) if span is not None else lins[0].__dict__.setdefault("_mx_ops", {})
    key = ("dx", span[1] if span is not None else 0, len(lins))
    if key not in memo:
        memo[key] = _group_operand(lins)
    return memo[key]


def _group_operand(lins):
    g = group_wt(lins)
    if g is None:
        return None
    mat2, sc = g
    span = _cat_span(lins)
    if span is not None and span[1] == 0 and len(lins) == span[0].n:
        return span[0].qt_tl, sc, 2
    if span is None and "_mx_wt_tl" in lins[0].__dict__:
        return lins[0]._mx_wt_tl, sc, 2
    return mat2.t(), sc, 0


# ---------------------------------------------------------------- enable / disable (mxfp8.py:452-509)
def _dgrad_rows(lin, w):
    wt = w.t()
    lin._mx_wtf_tl, lin._mx_wtfs = mx_quant_tiled(wt[fused_dgrad_rows(wt.shape[0], w.device)].contiguous())


def _prep_single(lin, leaf):
    w = lin.weight.data.to(torch.bfloat16)
    lin._mx_w, lin._mx_ws, lin._mx_wt, lin._mx_wts = quant_both(w)
    lin._mx_w_tl, lin._mx_wt_tl = tile_codes(lin._mx_w), tile_codes(lin._mx_wt)
    if leaf == "down_proj":  # the fused MLP's operands in the pi_col row order (MXFP8_GEMM_B_PI)
        _dgrad_rows(lin, w)
        lin._mx_wp_tl, lin._mx_wps = mx_quant_tiled(w[fused_dgrad_rows(w.shape[0], w.device)].contiguous())


def dgrad_rows_operand(lin):
    """(codes, scales) of W_downᵀ in the dgrad row order (fused_dgrad_rows), MX-tiled: the B operand of the fused
    MLP's dhm GEMM (with MXFP8_GEMM_B_PI, or the fused SwiGLU backward).  Made at enable_mxfp8 for down_proj,
    else from the host copy of the bf16 weight on first use, and kept with the MX copies."""
    if "_mx_wtf_tl" not in lin.__dict__:
        _dgrad_rows(lin, lin._bf16_cpu.to(lin._mx_w.device, torch.bfloat16))
    return lin._mx_wtf_tl, lin._mx_wtfs


def _prep_gate_up(gate, up):
    hold = _GateUp(gate.weight.data, up.weight.data)
    for i, lin in enumerate((gate, up)):
        lin._mx_w, lin._mx_ws = hold.rows(i)
        lin._mx_gu = (hold, i)


def _prep_concat(lins):
    cat = _Cat(lins)
    for k, lin in enumerate(lins):
        lin._mx_w, lin._mx_ws, lin._mx_w_tl = cat.fwd_rows(k)
        lin._mx_cat = (cat, k)


def _install(lin, leaf):
    """Move the bf16 weight to host memory (an empty tensor of the same dtype and device stays for code that
    reads them) and route forward through the MX GEMM."""
    w = lin.weight.data
    lin._mx_fbwd = leaf in FUSED_BWD
    lin._bf16_cpu = w.to("cpu", copy=True)
    lin.weight.data = torch.empty((0,), dtype=w.dtype, device=w.device)
    lin.forward = types.MethodType(_forward, lin)


def enable_mxfp8(model):
    """Quantize every frozen base linear of the decoder layers along both axes, share one copy per gate/up pair
    and one concatenated Wᵀ per _CATS group, move the bf16 weights to host memory and patch forward
    (mxfp8.py:452-498).  Both axes of each weight come from one read (quant_both).  Returns the linear count."""
    found, owners = [], {}
    for name, lin in _base_linears(model):
        assert lin.bias is None
        assert lin.weight.is_cuda and lin.weight.shape[0] % 128 == 0 and lin.weight.shape[1] % 128 == 0, \
            lin.weight.shape
        leaf, owner = _mx_target(name, lin)
        found.append((leaf, lin))
        owners.setdefault(owner, {})[leaf] = lin
    prepared, n_cat, n_pair = set(), 0, 0
    for sib in owners.values():  # the siblings under one owner module
        for names in _CATS:
            if all(k in sib for k in names):
                grp = [sib[k] for k in names]
                _prep_concat(grp)
                prepared.update(id(lin) for lin in grp)
                n_cat += len(grp)
        gate, up = sib.get("gate_proj"), sib.get("up_proj")
        if FUSE_GU and gate is not None and up is not None and gate.weight.shape == up.weight.shape:
            _prep_gate_up(gate, up)
            prepared.update((id(gate), id(up)))
            n_pair += 1
    for leaf, lin in found:
        if id(lin) not in prepared:
            _prep_single(lin, leaf)
        _install(lin, leaf)
    torch.cuda.empty_cache()
    print(f"MXFP8: {len(found)} frozen linears on MX GEMMs (bf16 weights moved to host memory;"
          f" {n_cat} with a concatenated group Wᵀ, {n_pair} gate/up pairs shared)", flush=True)
    return len(found)


def disable_mxfp8(model):
    """Put the bf16 weights back on their device, drop the MX copies and the patched forward (mxfp8.py:501-509)."""
    for _, lin in _base_linears(model):
        saved = lin.__dict__.get("_bf16_cpu")
        if saved is None:
            continue
        lin.weight.data = saved.to(lin.weight.device)
        for a in _MX_ATTRS:
            lin.__dict__.pop(a, None)
    _ACT.forget()
    torch.cuda.empty_cache()
