"""Linear layers that share one input (q/k/v; qkv/z/b/a of a DeltaNet block; o_proj / out_proj) computed in ONE
autograd.Function, after /root/reference/scripts/fused_linear.py.

  - x is read once for every LoRA A of the group (and the weights of thin frozen linears, <= _THIN outputs): one
    GEMM x·Sᵀ with S the concatenated rows;
  - MX base layers share one quantization of x; the LoRA-B product rides in the MX GEMM's epilogue;
  - backward over MX layers (mxfp8.FUSED_BWD): each dy is read once by mxfp8.lora_bwd (MX codes into one buffer
    concatenated along the group's N, d(xa), dB), and dx of the group is ONE MX GEMM against the concatenated Wᵀ;
  - o_proj / out_proj may return a Deferred output (LoRA not yet added) that residual_add adds inside the residual
    kernel (mxfp8.res_lora).
Layers that cannot take this path (trainable base weights, DoRA, dropout > 0, several adapters) are called one by
one.  `_part`, `_cast` / `new_step` and `STATS` are also what the fused MLP path reads.
"""
import torch
from torch import nn

_THIN = 64  # a plain frozen Linear with at most this many outputs joins the S GEMM (in_proj_b/a: 16)
STATS = {"gộp": 0, "gọi thẳng": 0}  # path counters, same keys as the reference (fused / called directly)


def _part(m):
    """(base Linear, A, B, scaling) of a PEFT LoRA Linear; (m, None, None, 1.0) for a plain frozen Linear;
    None if the layer cannot take the fused path (fused_linear.py:30-48)."""
    base = getattr(m, "base_layer", None)
    if base is None:
        if type(m) is nn.Linear and m.bias is None and not m.weight.requires_grad:
            return m, None, None, 1.0
        return None
    if base.bias is not None or base.weight.requires_grad or m.merged or m.disable_adapters:
        return None
    ads = [a for a in m.active_adapters if a in m.lora_A]
    if len(ads) != 1:
        return None
    a = ads[0]
    drop = m.lora_dropout[a]
    if (a in getattr(m, "lora_variant", {}) or m.use_dora.get(a, False) or m.lora_B[a].bias is not None
            or not (isinstance(drop, nn.Identity) or getattr(drop, "p", 1) == 0)):
        return None
    return base, m.lora_A[a].weight, m.lora_B[a].weight, m.scaling[a]


# bf16 copies of the LoRA A/B parameters (fp32) and the concatenated S matrix, made once per training step
# instead of at every call.  The optimizer may update parameters in place without bumping _version, so the
# step driver calls new_step() at the start of each step (fused_linear.py:55-62).
_CAST = {}


def new_step():
    _CAST.clear()


def _cast(key, make):
    t = _CAST.get(key)
    if t is None:
        t = _CAST[key] = make()
    return t


def _mx(base):
    return getattr(base, "_mx_w", None) is not None


def _vec_ok(t):
    """A bf16 [rows, r] view the native kernels read with 16-byte loads: row stride % 8, 16-byte aligned."""
    return t.stride(1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0


def _rp(n):
    """Padded row count of S / column count of dS for the native rank-r kernels (16, 32 or 64), None above 64."""
    for rp in (16, 32, 64):
        if n <= rp:
            return rp
    return None


def _native_ok(x2, dt, n):
    """The thin GEMMs x·Sᵀ, dSᵀ·x and dS·S run on the library's kernels (mxfp8_lora_nt / mxfp8_lora_tn / the MX
    GEMM epilogue) when the math is bf16 on the GPU, S has at most 64 rows and d_model % 128 == 0."""
    return (x2.is_cuda and dt == torch.bfloat16 and _rp(n) is not None and x2.shape[0] > 0 and x2.shape[1] % 128 == 0
            and _vec_ok(x2))


def _s_pad(S, key, rp):
    """S zero-padded to rp rows (cached per step with the S it pads)."""
    return _cast(key + ("pad", rp), lambda: torch.cat([S, S.new_zeros(rp - S.shape[0], S.shape[1])]))


def _base_mm(base, x2, dt, q, T):
    """x2 @ Wᵀ of a base weight: the MX GEMM when enable_mxfp8 covers the layer (q = the group's tiled MX codes of
    x2), else a bf16 GEMM (fused_linear.py:72-76)."""
    if _mx(base):
        import mxfp8
        tl = getattr(base, "_mx_w_tl", None)
        if tl is not None:
            return mxfp8.mx_mm(q[0], q[1], tl, base._mx_ws, layout=3, m=T)
        return mxfp8.mx_mm(q[0], q[1], base._mx_w, base._mx_ws, layout=1, m=T)
    return x2 @ base.weight.to(dt).t()


def _fwd_merged(parts, lora, Bs, xS, q, T, dt, skey):
    """Outputs of the group's MX layers from ONE GEMM over their concatenated forward weight (a consecutive range of
    one mxfp8._CATS group), each written to its own contiguous tensor, with every layer's LoRA-B product in the
    epilogue: P = xS (the padded x·Sᵀ), Q = the layers' B placed block-diagonally at their S columns (zeros adding
    nothing), one alpha.  Same bits as one GEMM per layer.  None when the layers do not qualify (not a cat range,
    LoRA scalings that differ, xS not in the padded native form)."""
    import mxfp8
    mxi = [i for i, p in enumerate(parts) if _mx(p[0])]
    if len(mxi) < 2 or xS is None or not _vec_ok(xS) or xS.shape[1] not in (16, 32, 64):
        return None
    op = mxfp8.group_fwd_operand([parts[i][0] for i in mxi])
    if op is None:
        return None
    lora_of = {i: (j, o, r, s) for j, (i, o, r, s) in enumerate(lora)}
    scales = {lora_of[i][3] for i in mxi if i in lora_of}
    if len(scales) > 1:
        return None
    alpha = scales.pop() if scales else 1.0
    rp = xS.shape[1]
    widths = [parts[i][0].out_features for i in mxi]

    def qcat():
        Q = torch.zeros((sum(widths), rp), dtype=dt, device=xS.device)
        r0 = 0
        for i, n in zip(mxi, widths):
            if i in lora_of:
                j, o, r, s = lora_of[i]
                Q[r0:r0 + n, o:o + r] = Bs[j]
            r0 += n
        return Q

    Q = _cast(skey + ("qcat", tuple(mxi), rp), qcat)
    outs = [torch.empty((T, n), dtype=dt, device=xS.device) for n in widths]
    mxfp8.mx_mm_seg(q[0], q[1], op[0], op[1], outs, lora=(xS, Q), alpha=alpha, layout=3, m=T)
    return dict(zip(mxi, outs))


class _Group(torch.autograd.Function):
    """Forward/backward of a group of linears on one input (fused_linear.py:79-196)."""

    @staticmethod
    def forward(ctx, x, parts, need_out, defer, *ws):
        ctx.set_materialize_grads(False)  # an output nobody uses gets grad None, not zeros
        dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else x.dtype
        lead, K = x.shape[:-1], x.shape[-1]
        x2 = x.reshape(-1, K)
        if x2.dtype != dt or not x2.is_contiguous():
            x2 = x2.to(dt).contiguous()
        T = x2.shape[0]
        # rows of the thin matrix S: the A of every LoRA layer (in order), then the weights of thin plain linears
        rows, Bs, lora, thin = [], [], [], []
        off = 0
        for i, (base, A, B, s) in enumerate(parts):
            if A is not None:
                rows.append(A)
                Bs.append(_cast((id(B), dt), lambda B=B: B.detach().to(dt)))
                lora.append((i, off, A.shape[0], s))
                off += A.shape[0]
        for i, (base, A, B, s) in enumerate(parts):
            if A is None and not _mx(base) and base.weight.shape[0] <= _THIN:
                rows.append(base.weight)
                thin.append((i, off, base.weight.shape[0]))
                off += base.weight.shape[0]
        skey = (tuple(id(r) for r in rows), dt)
        S = _cast(skey, lambda: torch.cat([r.detach().to(dt) for r in rows])) if rows else None
        xS = None
        if rows and _native_ok(x2, dt, off):
            # bf16(x·Sᵀ) from one read of x (the extra columns of the padded product are zero)
            import _native
            rp = _rp(off)
            xS = torch.empty((T, rp), dtype=dt, device=x2.device)
            _native.lora_nt(x2, _s_pad(S, skey, rp), xS)
        elif rows:
            xS = x2 @ S.t()
        outs = [None] * len(parts)
        thin_ids = {i for i, _, _ in thin}
        lora_of = {i: (j, o, r, s) for j, (i, o, r, s) in enumerate(lora)}
        if need_out:
            q = None
            if any(_mx(p[0]) for p in parts) and T:
                import mxfp8
                q = mxfp8.mx_quant_tiled(x2)  # once for the whole group
            merged = _fwd_merged(parts, lora, Bs, xS, q, T, dt, skey) if (
                q is not None and defer is None and dt == torch.bfloat16) else None
            if merged:
                for i, y in merged.items():
                    outs[i] = y
            for i, (base, A, B, s) in enumerate(parts):
                if i in thin_ids or (merged and i in merged):
                    continue
                if i in lora_of and _mx(base) and dt == torch.bfloat16 and T:
                    j, o, r, s = lora_of[i]
                    if defer is not None:
                        defer[i] = (xS[:, o:o + r], Bs[j], s)  # residual_add adds the LoRA part
                    elif r in (16, 32, 64) and _vec_ok(xS[:, o:o + r]):
                        # bf16(bf16(x·Wᵀ) + s · xa·Bᵀ) in the GEMM epilogue: the addmm_ of the reference
                        import mxfp8
                        tl = getattr(base, "_mx_w_tl", None)
                        w, lay = (tl, 3) if tl is not None else (base._mx_w, 1)
                        outs[i] = mxfp8.mx_mm(q[0], q[1], w, base._mx_ws, lora=(xS[:, o:o + r], Bs[j]), alpha=s,
                                              layout=lay, m=T)
                        continue
                outs[i] = _base_mm(base, x2, dt, q, T) if T else x2.new_empty(0, base.out_features)
                if i in lora_of and (defer is None or i not in defer):
                    j, o, r, s = lora_of[i]
                    outs[i].addmm_(xS[:, o:o + r], Bs[j].t(), alpha=s)
        else:  # only the graph for backward is needed (x2, xS saved); nobody reads the outputs
            STATS["bỏ đầu ra"] = STATS.get("bỏ đầu ra", 0) + 1
            for i, (base, A, B, s) in enumerate(parts):
                if i not in thin_ids:
                    outs[i] = x2.new_empty(x2.shape[0], base.out_features)
        for i, o, n in thin:
            outs[i] = xS[:, o:o + n].contiguous()
        ctx.save_for_backward(x2, xS, S, *Bs)
        ctx.meta = (parts, lora, thin, lead, K, dt, x.dtype)
        ctx.skey = skey
        return tuple(y.view(*lead, y.shape[-1]) for y in outs)

    @staticmethod
    def backward(ctx, *dys):
        x2, xS, S, *Bs = ctx.saved_tensors
        parts, lora, thin, lead, K, dt, xdt = ctx.meta
        need_x = ctx.needs_input_grad[0]
        flat = [None if dy is None else dy.reshape(-1, dy.shape[-1]).to(dt) for dy in dys]
        plan = _fused_bwd_plan(parts, flat, dt, need_x)
        if plan is not None:
            return _fused_backward(ctx, x2, xS, S, Bs, flat, plan, need_x)
        dx = None
        if need_x:
            thin_ids = {i for i, _, _ in thin}
            for i, (base, A, B, s) in enumerate(parts):
                dy = flat[i]
                if dy is None or i in thin_ids:
                    continue
                if _mx(base):
                    import mxfp8
                    d = dy if dy.is_contiguous() else dy.contiguous()
                    qd, sd = mxfp8.mx_quant(d)
                    wt, wts = mxfp8.mx_wt(base)
                    g = mxfp8.mx_mm(qd, sd, wt, wts)
                    dx = g if dx is None else dx.add_(g)
                else:
                    w = base.weight.to(dt)
                    dx = dy @ w if dx is None else dx.addmm_(dy, w)
        # thin branches: columns of d(xS) for the LoRA layers (s · dy @ B) and thin linears (dy itself), with the
        # matching rows of S
        blocks, srows, grads = [], [], [None] * (2 * len(lora))
        act_lora = []
        for j, (i, o, r, s) in enumerate(lora):
            dy = flat[i]
            if dy is None:
                continue
            xa = xS[:, o:o + r]
            dB = dy.t() @ xa
            dxa = dy @ Bs[j]
            if s != 1:
                dB.mul_(s)
                dxa.mul_(s)
            grads[2 * j + 1] = dB
            blocks.append(dxa)
            srows.append((o, r))
            act_lora.append(j)
        n_act = sum(r for _, r in srows)
        if need_x:
            for i, o, n in thin:
                if flat[i] is not None:
                    blocks.append(flat[i])
                    srows.append((o, n))
        if blocks:
            dS = torch.cat(blocks, 1) if len(blocks) > 1 else blocks[0]
            if need_x:
                full = len(srows) == len(lora) + len(thin)  # every row of S in use, in order
                Sa = S if full else torch.cat([S[o:o + w] for o, w in srows])
                dx = dS @ Sa if dx is None else dx.addmm_(dS, Sa)
            if act_lora:
                dA = dS[:, :n_act].t() @ x2
                c = 0
                for j in act_lora:
                    r = lora[j][2]
                    grads[2 * j] = dA[c:c + r]
                    c += r
        # A / B may be fp32 parameters while the math runs in bf16: autograd casts the gradients to their dtype
        ws_in = ctx.needs_input_grad[4:]
        out = [None if (g is None or not ws_in[k]) else g for k, g in enumerate(grads)]
        dx = None if dx is None else dx.view(*lead, K).to(xdt)
        return (dx, None, None, None, *out)


def _cdiv(a, b):
    return -(-a // b)


def _fused_bwd_plan(parts, flat, dt, need_x):
    """Whether the grouped backward applies (fused_linear.py:203-216): bf16 math, a gradient for every output,
    every MX layer in mxfp8.FUSED_BWD and, when dx is needed, a concatenated Wᵀ covering exactly the group's MX
    layers in order.  Returns (MX layer indices, (B operand, scales, layout) or None), or None for the plain path."""
    if dt != torch.bfloat16 or any(dy is None for dy in flat):
        return None
    mxi = [i for i, p in enumerate(parts) if _mx(p[0])]
    if not mxi or not all(getattr(parts[i][0], "_mx_fbwd", False) for i in mxi):
        return None
    import mxfp8
    wt = mxfp8.group_operand([parts[i][0] for i in mxi]) if need_x else None
    if need_x and wt is None:
        return None
    return mxi, wt


def _fused_backward(ctx, x2, xS, S, Bs, flat, plan, need_x):
    """_Group.backward through mxfp8.lora_bwd (fused_linear.py:219-279): each dy is read ONCE (MX codes into a
    buffer concatenated along the group's N, d(xa), dB) and dx of the group is ONE MX GEMM with the concatenated
    Wᵀ (fp32 accumulation across the layers instead of a bf16 add per layer).  The columns of dS follow the rows
    of S (the LoRA d(xa) in order, then the thin linears' dy); dx.addmm_(dS, S) and dA = dSᵀ·x2 as in the plain
    path."""
    import mxfp8
    parts, lora, thin, lead, K, dt, xdt = ctx.meta
    mxi, wt = plan
    T, dev = x2.shape[0], x2.device
    lora_of = {i: (j, o, r, s) for j, (i, o, r, s) in enumerate(lora)}
    n_act = sum(r for _, _, r, _ in lora)
    n_cols = n_act + (sum(n for _, _, n in thin) if need_x else 0)
    plain = [i for i, p in enumerate(parts) if not _mx(p[0]) and i not in {t[0] for t in thin}]
    # dS·S rides in the dx GEMM's epilogue and dA = dSᵀ·x2 runs on the token-reduction kernel when dS fits a
    # padded width of 16/32/64 (zero columns) and no plain bf16 linear has to be added into dx first
    native = n_cols > 0 and _native_ok(x2, dt, n_cols) and not plain
    width = _rp(n_cols) if native else n_cols
    dS = torch.empty((T, width), dtype=dt, device=dev) if n_cols else None
    if native and width > n_cols:
        dS[:, n_cols:].zero_()
    grads = [None] * (2 * len(lora))
    q = s_buf = None
    if need_x:
        n_mx = sum(flat[i].shape[1] for i in mxi)
        q = torch.empty((T, n_mx), dtype=mxfp8.F8, device=dev)
        s_buf = torch.empty(_cdiv(T, 128) * (n_mx // 128) * 512, dtype=torch.uint8, device=dev)
    tile = 0
    for i in mxi:
        dy = flat[i] if flat[i].stride(1) == 1 else flat[i].contiguous()
        if i in lora_of:
            j, o, r, s = lora_of[i]
            if r in (16, 32) and _vec_ok(xS[:, o:o + r]):
                grads[2 * j + 1] = mxfp8.lora_bwd(dy, xS[:, o:o + r], Bs[j], s, q=q, s=s_buf, col_tile_off=tile,
                                                  dxa_out=dS[:, o:o + r])
            else:  # a rank or xa layout the fused kernel does not take: codes from it, the products as GEMMs
                if q is not None:
                    mxfp8.lora_bwd(dy, q=q, s=s_buf, col_tile_off=tile)
                xa = xS[:, o:o + r]
                grads[2 * j + 1] = (dy.t().float() @ xa.float()).mul_(s)
                dS[:, o:o + r] = (dy.float() @ Bs[j].float()).mul_(s)
        elif q is not None:
            mxfp8.lora_bwd(dy, q=q, s=s_buf, col_tile_off=tile)
        tile += dy.shape[1] // 128
    for j, (i, o, r, s) in enumerate(lora):  # LoRA on a non-MX base layer (rare): as the plain path
        if i in mxi:
            continue
        dy = flat[i]
        dB = dy.t() @ xS[:, o:o + r]
        dS[:, o:o + r] = dy @ Bs[j]
        if s != 1:
            dB.mul_(s)
            dS[:, o:o + r].mul_(s)
        grads[2 * j + 1] = dB
    dx = None
    if need_x:
        wq, ws, lay = wt
        for i, o, n in thin:
            dS[:, o:o + n].copy_(flat[i])
        if native:
            # bf16(bf16(MX GEMM) + dS·S): the dx.addmm_(dS, S) of the reference in the GEMM epilogue
            St = _cast(ctx.skey + ("padT", width), lambda: _s_pad(S, ctx.skey, width).t().contiguous())
            dx = mxfp8.mx_mm(q, s_buf.view(mxfp8.E8), wq, ws, layout=lay, lora=(dS, St), alpha=1.0)
        else:
            dx = mxfp8.mx_mm(q, s_buf.view(mxfp8.E8), wq, ws, layout=lay)
            for i in plain:  # plain bf16 linears (neither MX nor thin)
                dx.addmm_(flat[i], parts[i][0].weight.to(dt))
            if dS is not None:
                dx.addmm_(dS, S)
        del q, s_buf
    if lora:
        if native:
            import _native
            dA = torch.empty((width, K), dtype=dt, device=dev)
            part = torch.empty(_native.lora_tn_chunks(T, K) * width * K, dtype=torch.float32, device=dev)
            _native.lora_tn(x2, dS, dA, part)  # bf16(dSᵀ·x2)
        else:
            dA = dS[:, :n_act].t() @ x2
        for j, (i, o, r, s) in enumerate(lora):
            grads[2 * j] = dA[o:o + r]
    STATS["lan ngược gộp"] = STATS.get("lan ngược gộp", 0) + 1
    ws_in = ctx.needs_input_grad[4:]
    out = [None if (g is None or not ws_in[k]) else g for k, g in enumerate(grads)]
    dx = None if dx is None else dx.view(*lead, K).to(xdt)
    return (dx, None, None, None, *out)


# ---------------------------------------------------------------- residual + LoRA-B (fused_linear.py:282-312)
class Deferred(tuple):
    """(y, xa, B, scaling): the bf16 MX output of o_proj / out_proj WITHOUT its LoRA part; residual_add adds it."""


class _ResidualLoRA(torch.autograd.Function):
    """x + (y + s · xa @ Bᵀ) in ONE kernel (mxfp8.res_lora): the residual add reads y and x and writes the new x
    anyway; adding the rank-r product there drops the addmm_ that reads and writes [T, N] once more.  xa and B are
    detached: the LoRA gradients (dB, d(xa) -> dA, dx) come from _Group.backward with the same dy; here only dy
    passes through."""

    @staticmethod
    def forward(ctx, x, y, xa, B, s):
        import mxfp8
        N = x.shape[-1]
        return mxfp8.res_lora(x.reshape(-1, N), y.reshape(-1, N), xa, B, s).view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        return dy, dy, None, None, None


def residual_add(x, y):
    """x + y; when y is Deferred (group_linear(..., defer=True)) the LoRA part is added inside the residual
    kernel."""
    if not isinstance(y, Deferred):
        return x + y
    y, xa, B, s = y
    N = x.shape[-1]
    if (x.dtype == y.dtype == torch.bfloat16 and x.shape == y.shape and x.is_contiguous() and y.is_contiguous()
            and N % 128 == 0 and xa.stride(1) == 1 and B.is_contiguous() and xa.shape[1] in (16, 32)):
        STATS["residual LoRA"] = STATS.get("residual LoRA", 0) + 1
        return _ResidualLoRA.apply(x, y, xa, B, s)
    return x + torch.addmm(y.reshape(-1, N), xa, B.t(), alpha=s).view(y.shape)  # other dtype/shape: as before


def group_linear(x, mods, need_out=True, defer=False):
    """(m(x) for m in mods), computed as one group (fused_linear.py:315-330).
    need_out=False: only the graph for backward (outputs uninitialised), for the recomputation of a checkpointed
    segment's last layer whose outputs nobody reads (the gradients are the same).
    defer=True: MX bf16 outputs with LoRA come back as Deferred (LoRA not yet added), for a residual_add right
    after."""
    parts = tuple(_part(m) for m in mods)
    if any(p is None for p in parts):
        STATS["gọi thẳng"] += 1
        return tuple(m(x) for m in mods)
    STATS["gộp"] += 1
    ws = [w for p in parts if p[1] is not None for w in (p[1], p[2])]
    box = {} if defer and need_out else None
    outs = _Group.apply(x, parts, need_out, box, *ws)
    if not box:
        return outs
    return tuple(Deferred((y,) + box[i]) if i in box else y for i, y in enumerate(outs))
