"""Fused MXFP8 SwiGLU MLP with LoRA on gate/up/down in one autograd.Function, on MI355X (gfx950).

Drop-in for /root/reference/scripts/fused_mlp.py: same module names (ENABLED, ACTIVE, SAVED_LESS, mlp, _MLP,
mlp_fwd, mlp_bwd), same saved-tensor set, same return dtypes and the same None fallback contract of mlp().

  Every MX GEMM operand of the path is in the MX-tiled layout (mxfp8.mx_quant_tiled, tile_codes): the same codes
  and scales as mx_quant in 1 KB blocks the GEMM streams without strided row pieces.
  forward : xs = x·[A_g; A_u]ᵀ (bf16) with MX(x) from one read -> MX GEMM gate|up (W_gu [2N, K]) whose
            epilogue stores gu and applies the LoRA-B of gate and up, bf16 rounding, h = silu(g)·u, MX(h) and
            the xS_down partials -> MX GEMM down with the LoRA epilogue y = bf16(y + s_d · xS_down · B_dᵀ).
            h is not stored (backward recomputes it from gu).
  backward: MX(dy) with dxd = dy·B_d from one read -> MX GEMM dhm = dy·W_down (fused-tile layout) -> fused
            kernel reading gu and dhm once: recompute g, u, h; dh = dhm + dxd·A_d; SwiGLU backward; MX(dg | du)
            into one [T, 2N] buffer; dxa, dB, dA_d partials -> one K = 2N MX GEMM dx = [dg | du]·W_gu with the
            LoRA epilogue dx = bf16(dx + dxa·S).
  FUSED_EPILOGUE[0] = False (MXFP8_FUSED_EPILOGUE=0) runs the gate|up GEMM alone and the SwiGLU forward in the
  separate fused kernel (mlp_fwd), the reference's own split.  FUSED_BWD_EPILOGUE[0] = True
  (MXFP8_FUSED_BWD_EPILOGUE=1) moves the backward kernel's work into the dhm GEMM's epilogue (dhm never leaves
  the registers); it measured slower than the split at the headline shape (the epilogue's loads, stores and
  waits do not hide behind the co-resident workgroup's main loop), so it is off by default.  Every mode gives
  the same bits except the xS_down and dB / dA_d partial sums, which are grouped by other tiles.
  need_out=False (checkpoint recompute): only xs, MX(x) and the gate|up GEMM run (fused_mlp.py:286-288).
Every kernel of the path is hand-written HIP (libmxfp8_mlp.so, _native.py): the rank-r LoRA products come from
the quantizer (xs with MX(x), dxd with MX(dy)), the GEMM epilogues (y, dx) and the token-reduction kernel
(dB_d, dA); no BLAS or elementwise torch kernel runs inside a step.
"""
import os
import types

import torch

import _native
import mxfp8
from fused_linear import STATS, _cast, _part

_F8, _E8 = torch.float8_e4m3fn, torch.float8_e8m0fnu
ENABLED = [True]  # set False to compare against the unfused path in the same process
# the SwiGLU forward in the epilogue of the gate|up GEMM (False: the GEMM, then the separate forward kernel)
FUSED_EPILOGUE = [os.environ.get("MXFP8_FUSED_EPILOGUE", "1") != "0"]
# the down, dhm and dx GEMMs with their weight operand in the pi_col row order (MXFP8_GEMM_B_PI: 16-byte stores
# of y, dhm and dx; False: the weights in row order)
B_PI = [os.environ.get("MXFP8_B_PI", "1") != "0"]
# 8-wave backward workgroups summing two 128-column quads in LDS (half the dxa partial bytes)
WIDE_BWD = [os.environ.get("MXFP8_WIDE_BWD", "1") != "0"]
# the backward's token reductions (dB_d, dA) folded into the dx GEMM's launch, in the slots its last round of tiles
# leaves idle (mxfp8_gemm_nt_tn; False: their own launch before the GEMM)
FOLD_TN = [os.environ.get("MXFP8_FOLD_TN", "1") != "0"]
# the forward's xS_down partial sum computed by the first workgroups of the down GEMM's launch, which its tiles'
# epilogues wait for (mxfp8_gemm_nt_sum; False: the sum_parts launch before the GEMM)
FOLD_SUM = [os.environ.get("MXFP8_FOLD_SUM", "1") != "0"]
# the SwiGLU backward in the epilogue of the dhm GEMM (False: the GEMM, then the separate backward kernel)
FUSED_BWD_EPILOGUE = [os.environ.get("MXFP8_FUSED_BWD_EPILOGUE", "0") == "1"]
ACTIVE = [False]  # the fused path ran at least once (read by the step engine to shrink per-layer activations)
SAVED_LESS = 12288  # bytes per token per layer not saved compared with the unfused path (h [T, 6144] bf16)

_CUS = [None]
LAST = {}  # launch parameters of the last fused kernels (for inspection)


def _n_cu():
    if _CUS[0] is None:
        _CUS[0] = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    return _CUS[0]


def _cdiv(a, b):
    return -(-a // b)


def _divisors(n):
    return [d for d in range(1, n + 1) if n % d == 0]


def _fwd_groups(T, N, R=16):
    """Column groups of the forward kernel, chosen by the library from the kernel's occupancy on this device
    (mxfp8_mlp_fwd_groups: fewest rounds x tiles per group, at least 4 tiles per group)."""
    return int(_native.load().mxfp8_mlp_fwd_groups(T, N, R))


def _bwd_grid(T, N, R, wide=False):
    """(SB, CG) of the backward kernel (SB a multiple of 128; CG a multiple of 128 with two 4-wave workgroups per
    CU, or of 256 with one 8-wave workgroup per CU when wide).  Every workgroup of a round runs at the same pace,
    so the time goes as rounds x (SB/32 row blocks x column passes); pick the least of that, then the fewest
    partial-sum bytes (per super-block dB / dA_d partials; the dxa partials are one per 128 (wide: 256) columns
    whatever the grid; the trade-off of fused_mlp.py:218-232)."""
    tpad = _cdiv(T, 128) * 128
    cap = _n_cu() * (1 if wide else 2)
    cols = 256 if wide else 128
    best = None
    for cg in [cols * d for d in _divisors(N // cols)]:
        ncg = N // cg
        for sb in range(128, tpad + 128, 128):
            nsb = _cdiv(tpad, sb)
            work = _cdiv(nsb * ncg, cap) * (sb // 32) * (cg // cols)
            partial = nsb * N * R * 3 * 4
            key = (work, partial)
            if best is None or key < best[0]:
                best = (key, sb, cg)
    return best[1], best[2]


def mlp_fwd(gu, xs, bg, bu, ad, s_g, s_u, write_q, h_out=None, tiled=False, gu_ft=False):
    """gu [T, 2N] bf16, xs [T, 2R] bf16 (xa_gate | xa_up), bg/bu [N, R], ad [R, N] bf16 -> (q_h, s_h, xS_down
    bf16) (fused_mlp.py:198-215).  h_out (optional [T, N] bf16) receives h for checks; tiled=True writes q_h
    in the MX-tiled GEMM operand layout ([ceil(T/16)*16, N] bytes, see mxfp8.mx_quant_tiled); gu_ft=True reads
    gu in the fused-tile layout ([ceil(T/32)*32, 2N], T taken from xs)."""
    T, N2 = xs.shape[0], gu.shape[1]
    N, R = N2 // 2, ad.shape[0]
    dev = gu.device
    ng = _fwd_groups(T, N, R)
    if write_q:
        q = torch.empty((mxfp8.tiled_rows(T) if tiled else T, N), dtype=_F8, device=dev)
        s = torch.empty(_cdiv(T, 128) * (N // 128) * 512, dtype=torch.uint8, device=dev)
    else:
        q = s = None
    part = torch.empty((ng, T, R), dtype=torch.float32, device=dev)
    LAST["fwd"] = dict(n_groups=ng)
    _native.mlp_fwd(gu, xs, bg, bu, ad, T, N, R, s_g, s_u, q, s, part, ng, h_out,
                    q_layout=int(tiled) | (2 if gu_ft else 0))
    xsd = torch.empty((T, R), dtype=torch.bfloat16, device=dev)
    _native.sum_parts(part, ng, T * R, xsd)
    return (q, s.view(_E8), xsd) if write_q else (None, None, xsd)


def _bwd_launch(gu, xs, xsT, dhm, dxd, dxdT, bg, bu, bgT, buT, ad, adT, s_g, s_u, need_q, dgu_out, tiled,
                gu_ft=False, wide=None):
    """Run the backward kernel; -> (q, s, (dxa_p, dbg_p, dbu_p, dad_p)) with the partial sums unreduced.
    gu_ft: gu and dhm in the fused-tile layout (T taken from xs).  wide: 8-wave workgroups with one dxa partial
    per 256 columns (None: WIDE_BWD when N allows it and no dgu_out is asked for)."""
    T, N2 = xs.shape[0], gu.shape[1]
    N, R = N2 // 2, ad.shape[0]
    dev = gu.device
    tpad = _cdiv(T, 128) * 128
    if wide is None:
        wide = WIDE_BWD[0] and N % 256 == 0 and dgu_out is None
    SB, CG = _bwd_grid(T, N, R, wide)
    nsb, ncg = _cdiv(tpad, SB), N // CG
    LAST["bwd"] = dict(SB=SB, CG=CG, nsb=nsb, ncg=ncg, wide=wide)
    if need_q:
        q = torch.empty((mxfp8.tiled_rows(T) if tiled else T, N2), dtype=_F8, device=dev)
        s = torch.empty(_cdiv(T, 128) * (N2 // 128) * 512, dtype=torch.uint8, device=dev)
    else:
        q = s = None
    # one dxa partial per 128 (wide: 256) columns
    dxa_p = torch.empty((N // (256 if wide else 128), T, 3 * R), dtype=torch.float32, device=dev)
    dbg_p = torch.empty((nsb, N, R), dtype=torch.float32, device=dev)
    dbu_p = torch.empty((nsb, N, R), dtype=torch.float32, device=dev)
    dad_p = torch.empty((nsb, R, N), dtype=torch.float32, device=dev)
    _native.mlp_bwd(gu, xs, xsT, dhm, dxd, dxdT, bg, bu, bgT, buT, ad, adT, T, N, R, s_g, s_u, SB, CG, q, s,
                    dxa_p, dbg_p, dbu_p, dad_p, dgu_out, q_layout=int(tiled) | (2 if gu_ft else 0) | (4 if wide else 0))
    return q, (s.view(_E8) if need_q else None), (dxa_p, dbg_p, dbu_p, dad_p)


def _transposed_padded(t, tpad):
    """[C, tpad] = tᵀ of t [T, C] bf16, zero past T (mxfp8_transpose_pad)."""
    out = torch.empty((t.shape[1], tpad), dtype=t.dtype, device=t.device)
    _native.transpose_pad(t, out)
    return out


def mlp_bwd(gu, xs, dhm, dxd, bg, bu, ad, s_g, s_u, need_q, dgu_out=None, tiled=False, gu_ft=False):
    """-> (q_dgu [T, 2N] fp8, s_dgu, [dxa_gate | dxa_up | xS_down] [T, 3R] fp32 (dxa not yet scaled by s),
    dBg, dBu [N, R] fp32 (not scaled), dAd [R, N] fp32) (fused_mlp.py:235-259).  tiled=True writes q_dgu in
    the MX-tiled GEMM operand layout ([ceil(T/16)*16, 2N] bytes); gu_ft=True reads gu and dhm in the
    fused-tile layout (T taken from xs)."""
    T, N2 = xs.shape[0], gu.shape[1]
    N, R = N2 // 2, ad.shape[0]
    dev = gu.device
    tpad = _cdiv(T, 128) * 128
    # small transposed copies the kernel reads as matrix-instruction operands
    xsT, dxdT = _transposed_padded(xs, tpad), _transposed_padded(dxd, tpad)
    bgT, buT, adT = bg.t().contiguous(), bu.t().contiguous(), ad.t().contiguous()
    q, s, (dxa_p, dbg_p, dbu_p, dad_p) = _bwd_launch(gu, xs, xsT, dhm, dxd, dxdT, bg, bu, bgT, buT, ad, adT, s_g,
                                                     s_u, need_q, dgu_out, tiled, gu_ft)
    dxa = torch.empty((T, 3 * R), dtype=torch.float32, device=dev)
    dbg = torch.empty((N, R), dtype=torch.float32, device=dev)
    dbu = torch.empty((N, R), dtype=torch.float32, device=dev)
    dad = torch.empty((R, N), dtype=torch.float32, device=dev)
    _native.sum_parts(dxa_p, dxa_p.shape[0], T * 3 * R, dxa)
    _native.sum_parts(dbg_p, dbg_p.shape[0], N * R, dbg)
    _native.sum_parts(dbu_p, dbu_p.shape[0], N * R, dbu)
    _native.sum_parts(dad_p, dad_p.shape[0], R * N, dad)
    return q, s, dxa, dbg, dbu, dad


def _prep(Ag, Bg, Au, Bu, Ad, Bd, dt):
    """The step's bf16 forms of the LoRA weights (fused_mlp.py:272-276 _cast copies, plus the transposed copies
    the kernels index), from one kernel; cached per step like fused_linear._cast."""
    def make():
        dev = Ag.device
        R, K = Ag.shape
        N = Bg.shape[0]
        e = lambda *sh: torch.empty(sh, dtype=torch.bfloat16, device=dev)  # noqa: E731
        out = dict(S=e(2 * R, K), ST=e(K, 2 * R), bg=e(N, R), bu=e(N, R), bgT=e(R, N), buT=e(R, N), ad=e(R, N),
                   adT=e(N, R), bd=e(K, R), bdT=e(R, K))
        f = lambda t: t.detach().float().contiguous()  # noqa: E731
        _native.lora_prep(f(Ag), f(Au), f(Bg), f(Bu), f(Ad), f(Bd), out)
        return types.SimpleNamespace(**out)
    return _cast((("lora_prep", id(Ag), id(Au), id(Bg), id(Bu), id(Ad), id(Bd)), dt), make)


def _forms_key(S, bg, bu, ad, bd, dt):
    return (("lora_forms", id(S), id(bg), id(bu), id(ad), id(bd)), dt)


def _forms_of_saved(S, bg, bu, ad, bd, dt):
    """The step's bf16 weight forms (_prep) looked up from the five tensors _MLP saves.  The forward registers
    them under the ids of those tensors; when the saved tensors come back as other objects (a saved-tensor
    hook, e.g. checkpointing) or the cache was cleared, the transposed forms are rebuilt from the saved ones.
    Every entry keeps its five key tensors alive (`keep`), so no id in a live key can be reused by another
    tensor within the step, and a hit is accepted only when those are the very objects passed in."""
    keys = (S, bg, bu, ad, bd)

    def make():
        R = ad.shape[0]
        f = lambda t: t.float().contiguous()  # noqa: E731
        K, N = S.shape[1], bg.shape[0]
        e = lambda *sh: torch.empty(sh, dtype=torch.bfloat16, device=S.device)  # noqa: E731
        out = dict(S=e(2 * R, K), ST=e(K, 2 * R), bg=e(N, R), bu=e(N, R), bgT=e(R, N), buT=e(R, N), ad=e(R, N),
                   adT=e(N, R), bd=e(K, R), bdT=e(R, K))
        _native.lora_prep(f(S[:R]), f(S[R:]), f(bg), f(bu), f(ad), f(bd), out)
        return types.SimpleNamespace(keep=keys, **out)

    lw = _cast(_forms_key(*keys, dt), make)
    if len(lw.keep) != 5 or any(a is not b for a, b in zip(lw.keep, keys)):
        return make()  # not reachable while entries hold their keys; never trust an id match alone
    return lw


# GEMM layout of the MLP's own products: both operands MX-tiled, output in the fused-tile layout
_LAYOUT_FT = _native.GEMM_A_TILED | _native.GEMM_B_TILED | _native.GEMM_C_FT


class _MLP(torch.autograd.Function):
    """fused_mlp.py:262-336."""

    @staticmethod
    def forward(ctx, x, meta, need_out, Ag, Bg, Au, Bu, Ad, Bd):
        ctx.set_materialize_grads(False)
        hold, down, (s_g, s_u, s_d), dt = meta
        lead, K = x.shape[:-1], x.shape[-1]
        x2 = x.reshape(-1, K)
        if x2.dtype != dt or not x2.is_contiguous():
            x2 = x2.to(dt).contiguous()
        lw = _prep(Ag, Bg, Au, Bu, Ad, Bd, dt)  # every bf16 form of the LoRA weights, one kernel per step
        S, bg, bu, ad, bd = lw.S, lw.bg, lw.bu, lw.ad, lw.bd
        T, R = x2.shape[0], Ad.shape[0]
        # one read of x2: its MX operand (MX-tiled codes, the GEMM's operand layout; same codes and scales as
        # mx_quant) and xs = bf16(x2 · Sᵀ) [T, 2R] = xa_gate | xa_up, with the zero-padded transpose the backward
        # kernel reads
        q, sc, xs, _ = mxfp8.mx_quant_lora(x2, S, out_t=False)  # 2R in {32, 64} (r in {16, 32}, _r_ok)
        if need_out and FUSED_EPILOGUE[0]:
            # one launch: gu = gate | up [T, 2N] (fused-tile layout, the saved tensor) and, in the GEMM's epilogue,
            # the LoRA-B of gate and up, h = silu(g)·u, MX(h) and the per-tile xS_down partials
            gu, qh, sh, part = mxfp8.swiglu_gemm(q, sc, hold, xs, bg, bu, ad, s_g, s_u, T)
            del q, sc
            xsd = torch.empty((T, R), dtype=dt, device=x2.device)
            if not (R == 16 and FOLD_SUM[0] and T * R <= _native.GEMM_NT_SUM_MAX):  # else in the down launch
                _native.sum_parts(part, part.shape[0], T * R, xsd)
                part = None
        else:
            part = None
            # gu = gate | up [T, 2N] in the fused-tile layout the fused kernels read (32 x 32 blocks of 2 KB)
            gu = mxfp8.mx_mm(q, sc, hold.w_tl, hold.ws, layout=_LAYOUT_FT, m=T)
            del q, sc
            if need_out:
                qh, sh, xsd = mlp_fwd(gu, xs, bg, bu, ad, s_g, s_u, True, tiled=True, gu_ft=True)
        if need_out:
            # y = bf16(bf16(MX(h)·W_downᵀ) + s_d · xS_down · B_dᵀ): the addmm_ of fused_mlp.py:284 in the epilogue
            w, ws, lay = ((down._mx_wp_tl, down._mx_wps, 3 | _native.GEMM_B_PI)
                          if B_PI[0] and "_mx_wp_tl" in down.__dict__ else (down._mx_w_tl, down._mx_ws, 3))
            if part is not None:  # xsd = bf16(Σ part) summed by the first workgroups of the same launch
                y = mxfp8.mx_mm_sum(qh, sh, w, ws, part, xsd, bd, s_d, lay, T)
            else:
                y = mxfp8.mx_mm(qh, sh, w, ws, lora=(xsd, bd), alpha=s_d, layout=lay, m=T)
            del qh, sh, xsd, part
        else:  # graph only (checkpoint recompute / prefix backward): nobody reads y
            STATS["bỏ đầu ra"] = STATS.get("bỏ đầu ra", 0) + 1
            y = x2.new_empty(x2.shape[0], down.out_features)
        # the reference's saved set, the same in both modes (non-reentrant checkpointing compares metadata on
        # recompute); the transposed weight forms stay in the per-step cast cache, keyed by these tensors
        lw.keep = (S, bg, bu, ad, bd)  # the entry holds its key tensors (see _forms_of_saved)
        _cast(_forms_key(S, bg, bu, ad, bd, dt), lambda: lw)
        ctx.save_for_backward(x2, xs, gu, S, bg, bu, ad, bd)
        ctx.meta = (hold, down, (s_g, s_u, s_d), dt, lead, K, x.dtype)
        ctx.pdt = (Ag.dtype, Au.dtype, Bd.dtype)  # the dtypes autograd casts dA_g, dA_u and dB_d to
        return y.view(*lead, y.shape[-1])

    @staticmethod
    def backward(ctx, dy):
        if dy is None:
            return (None,) * 9
        x2, xs, gu, S, bg, bu, ad, bd = ctx.saved_tensors
        hold, down, (s_g, s_u, s_d), dt, lead, K, xdt = ctx.meta
        need_x = ctx.needs_input_grad[0]
        R = ad.shape[0]
        dy2 = dy.reshape(-1, dy.shape[-1]).to(dt)
        if not dy2.is_contiguous():
            dy2 = dy2.contiguous()
        T, N = dy2.shape[0], hold.n
        lw = _forms_of_saved(S, bg, bu, ad, bd, dt)
        # one read of dy2: its MX operand and dxd = bf16(bf16(dy2 · bd) · s_d) [T, R] with its zero-padded transpose,
        # and, from the same launch, xsT, the backward kernel's operand form of xs (zero-padded transpose)
        qd, sd, dxd, dxdT, xsT = mxfp8.mx_quant_lora_tp(dy2, lw.bdT, xs, scale=s_d)
        if need_x and R == 16 and FUSED_BWD_EPILOGUE[0]:
            # one launch: dhm = MX(dy) · W_down in registers and, in the GEMM's epilogue, the SwiGLU backward:
            # MX(dg | du) and the dxa / dB / dA_d partials
            qg, sg, parts = mxfp8.swiglu_bwd_gemm(qd, sd, down, gu, xs, xsT, dxd, dxdT, bg, lw.bgT, bu, lw.buT, ad,
                                                  lw.adT, s_g, s_u, T)
            del qd, sd
        else:
            # MX(dy) · W_down in the FT layout; with W_downᵀ in the dgrad row order the epilogue stores whole
            # 16-byte pieces (the same dhm)
            if B_PI[0]:
                dhm = mxfp8.mx_mm(qd, sd, *mxfp8.dgrad_rows_operand(down), layout=_LAYOUT_FT | _native.GEMM_B_PI,
                                  m=T)
            else:
                dhm = mxfp8.mx_mm(qd, sd, down._mx_wt_tl, down._mx_wts, layout=_LAYOUT_FT, m=T)
            del qd, sd
            qg, sg, parts = _bwd_launch(gu, xs, xsT, dhm, dxd, dxdT, bg, bu, lw.bgT, lw.buT, ad, lw.adT, s_g, s_u,
                                        need_x, None, True, gu_ft=True)
            del dhm
        # the partial sums, scaled and cast as fused_mlp.py:258, :319-326 do, in one kernel
        dxa = torch.empty((T, 2 * R), dtype=dt, device=dy2.device)  # bf16(s_g dxa_g | s_u dxa_u)
        xsd = torch.empty((T, R), dtype=dt, device=dy2.device)      # bf16(xS_down)
        dB_g = torch.empty((N, R), dtype=torch.float32, device=dy2.device)
        dB_u = torch.empty_like(dB_g)
        dA_d = torch.empty((R, N), dtype=torch.float32, device=dy2.device)
        _native.mlp_bwd_finish(*parts, T, N, R, s_g, s_u, dxa, xsd, dB_g, dB_u, dA_d)
        del parts
        # the token reductions: the bf16 values of the reference's bf16 GEMMs (fused_mlp.py:316-318, :333), held
        # in the dtype of the parameter they are the gradient of: autograd casts a bf16 return to an fp32
        # parameter's dtype anyway (bf16 -> fp32 is exact, so .grad is bit-identical), and the kernel writing the
        # fp32 holder directly saves those cast kernels (about 23 us per step at the headline shape).  Both in one
        # launch (and their chunk sums in one more): dB_d = bf16(bf16(dyᵀ xsd) s_d) and dA = bf16(dxaᵀ · x2)
        ag_dt, au_dt, bd_dt = ctx.pdt
        fp32_a = ag_dt == au_dt == torch.float32
        chunks = _native.lora_tn_chunks(T, K)
        part = torch.empty(chunks * 3 * R * K, dtype=torch.float32, device=dy2.device)
        dB_d = torch.empty((K, R), dtype=torch.float32 if bd_dt == torch.float32 else dt, device=dy2.device)
        dA = torch.empty((2 * R, K), dtype=torch.float32 if fp32_a else dt, device=dy2.device)
        tn_jobs = [(dy2, xsd, dB_d, s_d, True), (x2, dxa, dA, 1.0, False)]
        fold = need_x and 2 * R == 32 and FOLD_TN[0]  # else the reductions run here, before the dx GEMM
        if not fold and 2 * R <= 32:  # the batch takes ranks 16 and 32
            _native.lora_tn_batch(tn_jobs, part)
        elif not fold:
            _native.lora_tn(dy2, xsd, dB_d, part[:chunks * R * K], scale=s_d, transpose=True)
            _native.lora_tn(x2, dxa, dA, part[chunks * R * K:])
        dx = None
        if need_x:
            # dx = bf16(bf16(MX(dg | du) · W_gu) + dxa · S): one K = 2N GEMM with the addmm_ of
            # fused_mlp.py:331 in its epilogue
            w, ws, lay = ((hold.wtp_tl, hold.wtps, 3 | _native.GEMM_B_PI) if B_PI[0] else
                          (hold.wt_tl, hold.wts, 3))
            if fold:
                dx = mxfp8.mx_mm_tn(qg, sg, w, ws, (dxa, lw.ST), 1.0, lay, T, tn_jobs, part)
            else:
                dx = mxfp8.mx_mm(qg, sg, w, ws, lora=(dxa, lw.ST), alpha=1.0, layout=lay, m=T)
            del qg, sg
            dx = dx.view(*lead, K).to(xdt)
        grads = [dA[:R], dB_g, dA[R:], dB_u, dA_d, dB_d]
        ws_in = ctx.needs_input_grad[3:]
        return (dx, None, None, *[g if ws_in[k] else None for k, g in enumerate(grads)])


def _r_ok(r):
    return r in (16, 32)


def mlp(mlp_mod, x, need_out=True):
    """down(silu(gate(x)) * up(x)) through _MLP when gate/up/down are PEFT LoRA layers over MX weights with gate
    and up paired by mxfp8.enable_mxfp8, computing in bf16 on the GPU; otherwise None (the caller takes the
    unfused path) (fused_mlp.py:343-366)."""
    if not ENABLED[0]:
        return None
    parts = [_part(m) for m in (mlp_mod.gate_proj, mlp_mod.up_proj, mlp_mod.down_proj)]
    if any(p is None or p[1] is None for p in parts):
        return None
    (gb, Ag, Bg, s_g), (ub, Au, Bu, s_u), (db, Ad, Bd, s_d) = parts
    dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else x.dtype
    if dt != torch.bfloat16 or not x.is_cuda:
        return None
    pg, pu = getattr(gb, "_mx_gu", None), getattr(ub, "_mx_gu", None)
    if pg is None or pu is None or pg[0] is not pu[0] or (pg[1], pu[1]) != (0, 1) or not mxfp8.is_mx(db):
        return None
    hold = pg[0]
    if getattr(hold, "w_tl", None) is None or getattr(db, "_mx_wt_tl", None) is None:
        return None  # weights not prepared by this module's enable_mxfp8 (no MX-tiled copies)
    r = Ag.shape[0]
    T = x.numel() // x.shape[-1]
    if not (_r_ok(r) and Au.shape[0] == r and Ad.shape[0] == r and x.shape[-1] == hold.w.shape[1]
            and hold.n % 128 == 0 and x.shape[-1] % 128 == 0 and Ad.shape[1] == hold.n and T > 0
            and T * 2 * hold.n < 2 ** 31):
        return None  # (32-bit element indexing in the kernels; N and K in 128-wide MX tiles)
    STATS["mlp gộp"] = STATS.get("mlp gộp", 0) + 1
    ACTIVE[0] = True
    return _MLP.apply(x, (hold, db, (s_g, s_u, s_d), dt), need_out, Ag, Bg, Au, Bu, Ad, Bd)
