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
    rp in {16, 32}: -> (q, s, out [R, rp], outT [rp, ceil(R/128)*128] zero-padded, or None)."""
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
        part_dxa = torch.empty((N // 128, T, R), dtype=torch.float32, device=dev)
        part_db = torch.empty((_native.lora_bwd_chunks(T, N), N, R), dtype=torch.float32, device=dev)
    _native.lora_bwd(dy, q.view(torch.uint8) if do_q else None, s.view(torch.uint8) if do_q else None,
                     q.shape[1] // 128 if do_q else 0, col_tile_off, xa, B, scale, dxa_out, db, part_dxa, part_db)
    return db


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


def mx_mm_seg(q, s, wq, ws, outs, lora=None, alpha=1.0, layout=0, m=None):
    """mx_mm whose N output columns go to the separate [M, n_k] tensors `outs` (consecutive column ranges, each a
    multiple of 128 wide); 4-wave shape, row-major outputs."""
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
                            layout=layout)
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
    layout (pass out with ft_rows(M) rows)."""
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


# ---------------------------------------------------------------- generic MX linear (mxfp8.py:296-341)
_last = [None, 0, None, None]  # (weakref tensor, _version, q, s) of the last quantized activation


def _quant_act(x):
    """Quantize the input of a linear layer, reusing the last result if x is the same live tensor at the
    same version (qkv/z, q/k/v and gate/up share one input) (mxfp8.py:299-312)."""
    if _last[0] is not None and _last[0]() is x and _last[1] == x._version:
        STATS["reuse"] += 1
        return _last[2], _last[3]
    x2 = x.reshape(-1, x.shape[-1])
    if x2.dtype != torch.bfloat16 or not x2.is_contiguous():
        x2 = x2.to(torch.bfloat16).contiguous()
    q, s = mx_quant(x2)
    STATS["quant"] += 1
    _last[:] = [weakref.ref(x), x._version, q, s]
    return q, s


class _MXLinear(torch.autograd.Function):
    """x @ Wᵀ of a frozen MX weight, backward dx = MX(dy) @ W (mxfp8.py:315-333)."""

    @staticmethod
    def forward(ctx, x, q, s, lin):
        out = mx_mm(q, s, lin._mx_w, lin._mx_ws)
        ctx.lin = lin
        return out.view(*x.shape[:-1], out.shape[-1])

    @staticmethod
    def backward(ctx, dy):
        lin = ctx.lin
        n = dy.shape[-1]
        dy2 = dy.reshape(-1, n)
        if dy2.dtype != torch.bfloat16 or not dy2.is_contiguous():
            dy2 = dy2.to(torch.bfloat16).contiguous()
        q, s = mx_quant(dy2)
        STATS["quant"] += 1
        wt, wts = mx_wt(lin)
        dx = mx_mm(q, s, wt, wts)
        return dx.view(*dy.shape[:-1], dx.shape[-1]), None, None, None


@torch.compiler.disable
def _forward(self, x):
    q, s = _quant_act(x)
    return _MXLinear.apply(x, q, s, self)


_NAMES = {"q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj", "in_proj_qkv", "in_proj_z",
          "out_proj"}


def _base_linears(model):
    """Frozen base linears of the decoder layers (mxfp8.py:347-356)."""
    for name, m in model.named_modules():
        if not isinstance(m, torch.nn.Linear) or m.weight.requires_grad or ".layers." not in name:
            continue
        parts = name.split(".")
        leaf = parts[-2] if parts[-1] == "base_layer" else parts[-1]
        if leaf in _NAMES:
            yield name, m


def _leaf_parent(name):
    parts = name.split(".")
    if parts[-1] == "base_layer":
        return parts[-2], ".".join(parts[:-2])
    return parts[-1], ".".join(parts[:-1])


# Groups whose Wᵀ is kept once, concatenated along N, so that dx of the whole group is one GEMM over the
# concatenated dy codes (mxfp8.py:360-366).  Every N is a multiple of 128, so no 32-block straddles two layers and
# each layer's codes and scales equal its own quantization.  gate/up/down go through fused_mlp instead.
_CATS = (("in_proj_qkv", "in_proj_z"), ("q_proj", "k_proj", "v_proj"))
# Linears whose backward takes the grouped path of fused_linear._Group (one read of dy through lora_bwd)
FUSED_BWD = {"in_proj_qkv", "in_proj_z", "q_proj", "k_proj", "v_proj", "o_proj", "out_proj"}


class _Cat:
    """Wᵀ of a group concatenated along N: codes [K, ΣN] quantized along ΣN with their blocked scales, and the
    MX-tiled copy the whole-group GEMM reads (mxfp8.py:369-395)."""

    def __init__(self, qt, st, ns):
        self.qt, self.st = qt, st
        self.qt_tl = tile_codes(qt)
        self.offs = [0]
        for n in ns:
            self.offs.append(self.offs[-1] + n)
        self.n = len(ns)
        self._sub = {}

    def range(self, a, b):
        """(mat2 [N_a+..+N_{b-1}, K] column-major view, scales) of layers a..b-1, the torch._scaled_mm form.  The
        scales of a column range are its 128x4 tiles of every 128-row block, cut out contiguously on first use:
        byte for byte the quantization of that range alone."""
        c0, c1 = self.offs[a], self.offs[b]
        mat2 = self.qt[:, c0:c1].t()
        if (a, b) == (0, self.n):
            return mat2, self.st
        sc = self._sub.get((a, b))
        if sc is None:
            K, ntot = self.qt.shape
            blk = self.st.view(torch.uint8).view(_cdiv(K, 128), ntot // 128, 512)
            sc = self._sub[(a, b)] = blk[:, c0 // 128:c1 // 128].contiguous().view(-1).view(E8)
        return mat2, sc


def is_mx(lin):
    return getattr(lin, "_mx_w", None) is not None


def mx_wt(lin):
    """(fp8 Wᵀ [K, N] as the B operand of dx = dy @ W, scales).  For a gate/up pair: a column view of W_guᵀ
    (row stride 2N) plus that half's scale tiles cut out contiguously, made on first use and kept
    (mxfp8.py:402-415); for a layer of a concatenated group, its column range of the group's Wᵀ."""
    gu = lin.__dict__.get("_mx_gu")
    if gu is None:
        if "_mx_cat" in lin.__dict__:
            m, sc = wt_of(lin)
            return m.t(), sc
        return lin._mx_wt, lin._mx_wts
    hold, i = gu
    if hold.half_t[i] is None:
        n, k = hold.n, hold.wt.shape[0]
        s3 = hold.wts.view(torch.uint8).view(k // 128, 2 * n // 128, 512)
        hold.half_t[i] = (hold.wt[:, i * n:(i + 1) * n],
                          s3[:, i * (n // 128):(i + 1) * (n // 128)].reshape(-1).view(E8))
    return hold.half_t[i]


def wt_of(lin):
    """(mat2, scale) of dy @ W in torch._scaled_mm form: mat2 = Wᵀ codes as an [N, K] column-major view
    (mxfp8.py:418-426)."""
    c = lin.__dict__.get("_mx_cat")
    if c is not None:
        return c[0].range(c[1], c[1] + 1)
    wt, s = mx_wt(lin)
    return wt.t(), s


def group_wt(lins):
    """(mat2 [ΣN, K], scale) of dx = [dy_1|dy_2|..] @ [W_1; W_2; ..] for consecutive layers of one concatenated
    group (or a single layer); None when no concatenated copy fits (mxfp8.py:429-439)."""
    c = lins[0].__dict__.get("_mx_cat")
    if c is None:
        return wt_of(lins[0]) if len(lins) == 1 else None
    cat, k = c
    for d, lin in enumerate(lins):
        if lin.__dict__.get("_mx_cat") != (cat, k + d):
            return None
    return cat.range(k, k + len(lins))


def group_fwd_operand(lins):
    """(B operand [ΣN, K] of the forward GEMM of consecutive layers of one concatenated group (MX-tiled), scales),
    or None when the layers are not such a range."""
    c = lins[0].__dict__.get("_mx_cat")
    if c is None or getattr(c[0], "w_tl", None) is None:
        return None
    cat, k = c
    for d, lin in enumerate(lins):
        if lin.__dict__.get("_mx_cat") != (cat, k + d):
            return None
    c0, c1 = cat.offs[k], cat.offs[k + len(lins)]
    tile_b = (cat.w_tl.shape[1] // 128) * 512
    return cat.w_tl[c0:c1], cat.ws[c0 // 128 * tile_b:c1 // 128 * tile_b]


def group_operand(lins):
    """(B operand [K, ΣN] of mx_mm, scales, layout bit) for dx of `lins` (group_wt): the MX-tiled copy when the
    range is a whole concatenated group, else the row-major column view (row stride = the group's ΣN)."""
    g = group_wt(lins)
    if g is None:
        return None
    mat2, sc = g
    c = lins[0].__dict__.get("_mx_cat")
    if c is not None and c[1] == 0 and len(lins) == c[0].n:
        return c[0].qt_tl, sc, 2
    if c is None and "_mx_wt_tl" in lins[0].__dict__:
        return lins[0]._mx_wt_tl, sc, 2
    return mat2.t(), sc, 0


FUSE_GU = os.environ.get("MXFP8_FUSE_GU", "1") != "0"


def enable_mxfp8(model):
    """Quantize every frozen base linear of the decoder layers along both axes, pair gate/up into one shared
    copy, move the bf16 weights to host memory and patch forward (mxfp8.py:452-498).  Both axes of each weight
    come from one read (quant_both)."""
    lins = list(_base_linears(model))
    fam = {}
    for name, lin in lins:
        assert lin.bias is None
        w = lin.weight.data
        assert w.is_cuda and w.shape[0] % 128 == 0 and w.shape[1] % 128 == 0, w.shape
        leaf, parent = _leaf_parent(name)
        fam.setdefault(parent, {})[leaf] = lin
    in_cat, paired = set(), set()
    for d in fam.values():
        for names in _CATS:
            if all(k in d for k in names):
                # one read of the concatenated weight gives every layer's forward codes (rows of q) and the
                # group's Wᵀ along ΣN
                grp = [d[k] for k in names]
                w = torch.cat([lin.weight.data for lin in grp]).to(torch.bfloat16)  # [ΣN, K]
                q, sq, qt, st = quant_both(w)
                del w
                cat = _Cat(qt, st, [lin.weight.shape[0] for lin in grp])
                # the forward codes of the whole group (MX-tiled) for one GEMM over consecutive layers; each
                # layer's own codes and scales are row slices of them
                cat.w_tl, cat.ws = tile_codes(q), sq
                tile_b = (q.shape[1] // 128) * 512  # scale bytes of one 128-row tile row
                for k, lin in enumerate(grp):
                    c0, c1 = cat.offs[k], cat.offs[k + 1]
                    lin._mx_w, lin._mx_ws = q[c0:c1], sq[c0 // 128 * tile_b:c1 // 128 * tile_b]
                    lin._mx_w_tl = cat.w_tl[c0:c1]
                    lin._mx_cat = (cat, k)
                    in_cat.add(id(lin))
        gb, ub = d.get("gate_proj"), d.get("up_proj")
        if FUSE_GU and gb is not None and ub is not None and gb.weight.shape == ub.weight.shape:
            w = torch.cat([gb.weight.data, ub.weight.data]).to(torch.bfloat16)  # [2N, K]
            n = gb.weight.shape[0]
            hold = types.SimpleNamespace(n=n, half_t=[None, None])
            hold.w, hold.ws, hold.wt, hold.wts = quant_both(w)
            hold.w_tl, hold.wt_tl = tile_codes(hold.w), tile_codes(hold.wt)  # GEMM operand layout of the fused path
            del w
            ns = hold.ws.numel() // 2  # forward scales are ordered by tile row: first half = gate
            for i, lin in enumerate((gb, ub)):
                lin._mx_w, lin._mx_ws = hold.w[i * n:(i + 1) * n], hold.ws[i * ns:(i + 1) * ns]
                lin._mx_gu = (hold, i)
                paired.add(id(lin))
    for name, lin in lins:
        w = lin.weight.data
        if id(lin) not in paired and id(lin) not in in_cat:
            lin._mx_w, lin._mx_ws, lin._mx_wt, lin._mx_wts = quant_both(w.to(torch.bfloat16))
            lin._mx_w_tl, lin._mx_wt_tl = tile_codes(lin._mx_w), tile_codes(lin._mx_wt)
        lin._mx_fbwd = _leaf_parent(name)[0] in FUSED_BWD
        lin._bf16_cpu = w.to("cpu", copy=True)
        lin.weight.data = torch.empty((0,), dtype=w.dtype, device=w.device)
        lin.forward = types.MethodType(_forward, lin)
    torch.cuda.empty_cache()
    print(f"MXFP8: {len(lins)} frozen linears on MX GEMMs (bf16 weights moved to host memory;"
          f" {len(in_cat)} with a concatenated group Wᵀ, {len(paired) // 2} gate/up pairs shared)", flush=True)
    return len(lins)


def disable_mxfp8(model):
    """Restore the bf16 weights and the original forward (mxfp8.py:501-509)."""
    for _, lin in _base_linears(model):
        if hasattr(lin, "_bf16_cpu"):
            lin.weight.data = lin._bf16_cpu.to(lin.weight.device)
            for a in ("_mx_w", "_mx_ws", "_mx_wt", "_mx_wts", "_mx_w_tl", "_mx_wt_tl", "_mx_cat", "_mx_gu", "_mx_fbwd",
                      "_bf16_cpu", "forward"):
                if a in lin.__dict__:
                    delattr(lin, a)
    _last[:] = [None, 0, None, None]
    torch.cuda.empty_cache()
