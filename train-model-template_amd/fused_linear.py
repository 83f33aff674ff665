"""Linear layers that share one input (q/k/v; qkv/z/b/a of a DeltaNet block; o_proj / out_proj) computed in ONE
autograd.Function: the drop-in for /root/reference/scripts/fused_linear.py (group_linear, residual_add, Deferred,
_part, _cast, new_step, STATS).

A group is described once per call by a _Spec: which layers are MX, which carry a LoRA adapter, which are thin
frozen linears (<= _THIN outputs), and where each one's columns sit in the thin product xS = x·Sᵀ.  S stacks the
LoRA A rows of the adapter layers in layer order, then the thin linears' weights; the gradient layout of dS
follows the same columns.  On that layout:
  - forward reads x once for every A (and thin weight), quantizes x once for every MX layer, and puts each LoRA-B
    product in the MX GEMM's epilogue; consecutive layers of a concatenated group (mxfp8._CATS) run as one GEMM;
  - backward over MX layers (mxfp8.FUSED_BWD) reads each dy once (mxfp8.lora_bwd: MX codes into one buffer
    concatenated along the group's N, d(xa), dB) and computes dx of the group as ONE MX GEMM against the
    concatenated Wᵀ, with dS·S in its epilogue; other groups take the per-layer backward;
  - o_proj / out_proj may return a Deferred output (LoRA not yet added) that residual_add adds inside the residual
    kernel (mxfp8.res_lora).
Layers that cannot be grouped (trainable base weights, DoRA, dropout > 0, several adapters) are called one by one.
`_part`, `_cast` / `new_step` and `STATS` are also what the fused MLP path reads.
"""
import dataclasses
import os
import weakref

import torch
from torch import nn

_THIN = 64  # a plain frozen Linear with at most this many outputs joins the thin product (in_proj_b/a: 16)
# the per-step bf16 weight forms of a group from one mxfp8_pack_bf16 launch (False: one torch operation each)
PACK_FORMS = [os.environ.get("MXFP8_PACK_FORMS", "1") != "0"]
# the grouped backward's dA = dSᵀ·x2 in the workgroup slots its dx GEMM's last round of tiles leaves idle, one
# launch (mxfp8_gemm_nt_tn; False: its own launch after the GEMM)
FOLD_TN = [os.environ.get("MXFP8_GROUP_FOLD_TN", "1") != "0"]
STATS = {"gộp": 0, "gọi thẳng": 0}  # path counters, the reference's keys (grouped / called directly)


def _part(m):
    """(base Linear, A, B, scaling) of a PEFT LoRA Linear; (m, None, None, 1.0) for a plain frozen Linear;
    None if the layer cannot be grouped (fused_linear.py:30-48)."""
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


def _cdiv(a, b):
    return -(-a // b)


# ------------------------------------------------------------------------------------------- layout
@dataclasses.dataclass(frozen=True)
class _Slot:
    """Columns [col, col + width) of xS = x·Sᵀ that belong to layer `layer`: the rows of its LoRA A (an adapter,
    `index`-th of the group, scaled by `scale`) or the whole output of a thin frozen linear."""
    layer: int
    col: int
    width: int
    index: int = -1
    scale: float = 1.0

    @property
    def cols(self):
        return slice(self.col, self.col + self.width)


class _Spec:
    """The layout of one group (see the module docstring)."""

    def __init__(self, parts):
        self.parts = parts
        self.adapters, self.thin = [], []
        col = 0
        for i, (base, A, B, s) in enumerate(parts):
            if A is not None:
                self.adapters.append(_Slot(i, col, A.shape[0], len(self.adapters), s))
                col += A.shape[0]
        for i, (base, A, B, s) in enumerate(parts):
            if A is None and not _mx(base) and base.weight.shape[0] <= _THIN:
                self.thin.append(_Slot(i, col, base.weight.shape[0]))
                col += base.weight.shape[0]
        self.width = col
        self.adapter_cols = sum(sl.width for sl in self.adapters)
        self.thin_ids = frozenset(sl.layer for sl in self.thin)
        self._adapter = {sl.layer: sl for sl in self.adapters}
        self.mx = [i for i, p in enumerate(parts) if _mx(p[0])]
        self.plain = [i for i, p in enumerate(parts) if not _mx(p[0]) and i not in self.thin_ids]

    def adapter(self, i):
        return self._adapter.get(i)

    def s_sources(self):
        """The tensors whose rows make S, in column order."""
        return [self.parts[sl.layer][1] for sl in self.adapters] + [self.parts[sl.layer][0].weight for sl in self.thin]


# ------------------------------------------------------------------------------------------- native helpers
def _vec_ok(t):
    """A bf16 [rows, r] view the native kernels read with 16-byte loads: row stride % 8, 16-byte aligned."""
    return t.stride(1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0


def _rp(n):
    """Padded row count of S / column count of dS for the native rank-r kernels (16, 32 or 64), None above 64."""
    return next((rp for rp in (16, 32, 64) if n <= rp), None)


def _native_ok(x2, dt, n):
    """The thin GEMMs x·Sᵀ, dSᵀ·x and dS·S run on the library's kernels (mxfp8_lora_nt / mxfp8_lora_tn / the MX
    GEMM epilogue) when the math is bf16 on the GPU, S has at most 64 rows and d_model % 128 == 0."""
    return (x2.is_cuda and dt == torch.bfloat16 and _rp(n) is not None and x2.shape[0] > 0 and x2.shape[1] % 128 == 0
            and _vec_ok(x2))


def _same_buffer(a, b):
    """a and b are views of one allocation."""
    return a.untyped_storage().data_ptr() == b.untyped_storage().data_ptr()


def _s_pad(S, key, rp):
    """S zero-padded to rp rows (cached per step with the S it pads)."""
    return _cast(key + ("pad", rp), lambda: torch.cat([S, S.new_zeros(rp - S.shape[0], S.shape[1])]))


# The layout of a group's weight forms, kept across steps: the buffer, its views and the pack job table, keyed
# by the addresses, shapes, strides and dtypes of the group's sources (the optimizer updates parameters in
# place, at the same addresses).  Each step relaunches the pack into the same buffer, unless a backward of an
# earlier step may still read it: every forward saves its own views of the buffer and the plan keeps weak
# references to them (`readers`); autograd drops saved tensors when that backward has run (or when its graph
# dies), so a live reader at the next step's pack means a graph whose backward is still to come (a retained
# graph, a deferred prefix backward, overlapped micro-batches), and that step packs into a fresh buffer
# instead, leaving the pending backward the weights of its own step, as the reference's per-step copies do.
_PLANS = {}
_PLANS_MAX = 256


def _build_forms(spec, K, dev):
    """The buffer and views of the group's weight forms and the pack jobs that fill them."""
    import types
    rp, width = _rp(spec.width), spec.width
    a8 = lambda n: _cdiv(n, 8) * 8  # noqa: E731  (16-byte aligned views)
    sizes = [rp * K, K * rp] + [spec.parts[sl.layer][2].shape[0] * sl.width for sl in spec.adapters]
    n_q = sum(spec.parts[i][0].out_features for i in spec.mx) if len(spec.mx) >= 2 else 0
    sizes.append(n_q * rp)
    buf = torch.empty(sum(a8(n) for n in sizes), dtype=torch.bfloat16, device=dev)
    views, off = [], 0
    for n in sizes:
        views.append(buf[off:off + n])
        off += a8(n)
    S_pad, St = views[0].view(rp, K), views[1].view(K, rp)
    Bs = [v.view(-1, sl.width) for v, sl in zip(views[2:-1], spec.adapters)]
    Q = views[-1].view(n_q, rp) if n_q else None
    jobs = []
    for sl, src in zip(spec.adapters + spec.thin, spec.s_sources()):
        jobs += [(src.detach(), S_pad[sl.cols], False), (src.detach(), St[:, sl.cols], True)]
    if rp > width:
        jobs += [(None, S_pad[width:], False), (None, St[:, width:], True)]
    for sl, b in zip(spec.adapters, Bs):
        jobs.append((spec.parts[sl.layer][2].detach(), b, False))
    row = 0
    for i in (spec.mx if n_q else ()):
        n, sl = spec.parts[i][0].out_features, spec.adapter(i)
        if sl is None:
            jobs.append((None, Q[row:row + n], False))
        else:
            if sl.col:
                jobs.append((None, Q[row:row + n, :sl.col], False))
            jobs.append((spec.parts[i][2].detach(), Q[row:row + n, sl.cols], False))
            if sl.col + sl.width < rp:
                jobs.append((None, Q[row:row + n, sl.col + sl.width:], False))
        row += n
    return types.SimpleNamespace(S_pad=S_pad, S=S_pad[:width], St=St, Bs=Bs, Q=Q, rp=rp), jobs


def _group_forms(spec, skey, K, dev):
    """Every per-step bf16 form of the group's weights from ONE launch (mxfp8_pack_bf16), cached per step under
    skey: S_pad [rp, K] (the A rows and thin weights in column order, zero rows up to rp = _rp(width)), St =
    S_padᵀ [K, rp] (the backward's dS·S operand), each adapter's B [n, r] in Bs, and Q [Σ n, rp] with the MX
    layers' B placed block-diagonally at their S columns (the merged forward GEMM's epilogue operand; None
    for fewer than two MX layers).  The buffer and the job table persist across steps (_PLANS); the torch path
    builds these with one operation each."""
    def make():
        import _native
        srcs = spec.s_sources() + [spec.parts[sl.layer][2] for sl in spec.adapters]
        sig = (K, dev, tuple((sl.col, sl.width) for sl in spec.adapters + spec.thin),
               tuple(spec.parts[i][0].out_features for i in spec.mx),
               tuple((t.data_ptr(), tuple(t.shape), tuple(t.stride()), t.dtype) for t in srcs))
        plan = _PLANS.get(sig)
        if plan is not None:
            plan[0].readers[:] = [r for r in plan[0].readers if r() is not None]
            if plan[0].readers:  # an earlier step's backward still reads this buffer: pack into a fresh one
                plan = None
        if plan is None:
            if len(_PLANS) >= _PLANS_MAX:
                _PLANS.clear()
            forms, jobs = _build_forms(spec, K, dev)
            forms.readers = []
            plan = _PLANS[sig] = (forms, _native.pack_table(jobs))
        _native.pack_run(plan[1], like=plan[0].S_pad)
        return plan[0]
    return _cast(skey + ("forms",), make)


def _packable(spec, x2, dt):
    """The per-step weight forms come from one mxfp8_pack_bf16 launch: the native thin product applies and every
    source is fp32 or bf16."""
    return (PACK_FORMS[0] and bool(spec.adapters or spec.thin) and _native_ok(x2, dt, spec.width)
            and all(t.dtype in (torch.float32, torch.bfloat16) for t in spec.s_sources())
            and all(spec.parts[sl.layer][2].dtype in (torch.float32, torch.bfloat16) for sl in spec.adapters))


def _thin_product(x2, S, skey, width, dt, S_pad=None):
    """bf16(x2 · Sᵀ): one read of x2 on the library's rank-r kernel (S zero-padded to 16/32/64 rows, so xS has
    zero columns past `width`) when it applies, else a torch GEMM."""
    if not _native_ok(x2, dt, width):
        return x2 @ S.t()
    import _native
    rp = _rp(width)
    xS = torch.empty((x2.shape[0], rp), dtype=dt, device=x2.device)
    _native.lora_nt(x2, _s_pad(S, skey, rp) if S_pad is None else S_pad, xS)
    return xS


def _mx_out(base, codes, T, lora=None, alpha=1.0):
    """MX GEMM of one layer from the group's tiled codes of x (its MX-tiled weight copy when it has one)."""
    import mxfp8
    tl = getattr(base, "_mx_w_tl", None)
    w, layout = (tl, 3) if tl is not None else (base._mx_w, 1)
    return mxfp8.mx_mm(codes[0], codes[1], w, base._mx_ws, lora=lora, alpha=alpha, layout=layout, m=T)


def _base_mm(base, x2, dt, codes, T):
    """x2 · Wᵀ of a base weight: the MX GEMM when enable_mxfp8 covers the layer, else a bf16 GEMM
    (fused_linear.py:72-76)."""
    return _mx_out(base, codes, T) if _mx(base) else x2 @ base.weight.to(dt).t()


# ------------------------------------------------------------------------------------------- forward
def _fwd_merged(spec, Bs, xS, codes, T, dt, skey):
    """The outputs of the group's MX layers from ONE GEMM over their concatenated forward weight (a consecutive
    range of one mxfp8._CATS group), each written to its own contiguous tensor, with every layer's LoRA-B
    product in the epilogue: P = xS, Q = the layers' B placed block-diagonally at their S columns (zeros add
    nothing), one alpha.  Same bits as one GEMM per layer.  None when the layers do not qualify (not a cat
    range, LoRA scalings that differ, xS not in the padded native form)."""
    import mxfp8
    if len(spec.mx) < 2 or xS is None or not _vec_ok(xS) or xS.shape[1] not in (16, 32, 64):
        return None
    op = mxfp8.group_fwd_operand([spec.parts[i][0] for i in spec.mx])
    if op is None:
        return None
    slots = [spec.adapter(i) for i in spec.mx]
    scales = {sl.scale for sl in slots if sl is not None}
    if len(scales) > 1:
        return None
    alpha = scales.pop() if scales else 1.0
    widths = [spec.parts[i][0].out_features for i in spec.mx]
    rp = xS.shape[1]

    def block_diagonal_b():
        Q = torch.zeros((sum(widths), rp), dtype=dt, device=xS.device)
        row = 0
        for sl, n in zip(slots, widths):
            if sl is not None:
                Q[row:row + n, sl.cols] = Bs[sl.index]
            row += n
        return Q

    forms = _CAST.get(skey + ("forms",))
    if forms is not None and forms.Q is not None and forms.rp == rp:
        Q = forms.Q
    else:
        Q = _cast(skey + ("qcat", tuple(spec.mx), rp), block_diagonal_b)
    outs = [torch.empty((T, n), dtype=dt, device=xS.device) for n in widths]
    # every layer with an adapter of one width: each output tile takes the rank-width window of xS and Q at its
    # layer's own columns (the rest of its Q row is zero) instead of all rp columns
    ranks = {sl.width for sl in slots if sl is not None}
    if all(sl is not None for sl in slots) and len(ranks) == 1 and ranks <= {16, 32, 64}:
        cols = dict(lora_cols=[sl.col for sl in slots], r=ranks.pop())
    else:
        cols = {}
    mxfp8.mx_mm_seg(codes[0], codes[1], op[0], op[1], outs, lora=(xS, Q), alpha=alpha, layout=3, m=T, **cols)
    return dict(zip(spec.mx, outs))


def _forward_outputs(spec, x2, xS, Bs, skey, defer, dt, codes=None):
    """Every non-thin output of the group (fused_linear.py:104-117); codes: the MX-tiled codes of x2 when the
    caller already has them."""
    T = x2.shape[0]
    outs = [None] * len(spec.parts)
    if spec.mx and T:
        import mxfp8
        if codes is None:
            codes = mxfp8.mx_quant_tiled(x2)  # once for the whole group
        if defer is None and dt == torch.bfloat16:
            for i, y in (_fwd_merged(spec, Bs, xS, codes, T, dt, skey) or {}).items():
                outs[i] = y
    for i, (base, A, B, s) in enumerate(spec.parts):
        if outs[i] is not None or i in spec.thin_ids:
            continue
        sl = spec.adapter(i)
        on_mx_bf16 = sl is not None and _mx(base) and dt == torch.bfloat16 and T > 0
        if on_mx_bf16 and defer is not None:  # residual_add adds the LoRA part later
            defer[i] = (xS[:, sl.cols], Bs[sl.index], sl.scale)
            outs[i] = _mx_out(base, codes, T)
        elif on_mx_bf16 and sl.width in (16, 32, 64) and _vec_ok(xS[:, sl.cols]):
            # bf16(bf16(x·Wᵀ) + s · xa·Bᵀ) in the GEMM epilogue: the reference's addmm_
            outs[i] = _mx_out(base, codes, T, lora=(xS[:, sl.cols], Bs[sl.index]), alpha=sl.scale)
        else:
            outs[i] = _base_mm(base, x2, dt, codes, T) if T else x2.new_empty(0, base.out_features)
            if sl is not None:
                outs[i].addmm_(xS[:, sl.cols], Bs[sl.index].t(), alpha=sl.scale)
    return outs


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
        spec = _Spec(parts)
        src = spec.s_sources()
        skey = (tuple(id(t) for t in src), dt)
        codes = None
        forms = None
        if _packable(spec, x2, dt):
            forms = _group_forms(spec, skey, K, x2.device)
            Bs, S = forms.Bs, forms.S
            if spec.mx:
                # one read of x2 for both the MX layers' codes and xS (mxfp8_quant_lora); also when the outputs
                # are not needed (a checkpoint's recompute), so xS, which backward reads, has the same bits in
                # both modes
                import mxfp8
                q, sc, xS, _ = mxfp8.mx_quant_lora(x2, forms.S_pad, out_t=False)
                codes = (q, sc) if need_out else None
            else:
                xS = _thin_product(x2, S, skey, spec.width, dt, S_pad=forms.S_pad)
        else:
            Bs = [_cast((id(parts[sl.layer][2]), dt), lambda B=parts[sl.layer][2]: B.detach().to(dt))
                  for sl in spec.adapters]
            S = _cast(skey, lambda: torch.cat([t.detach().to(dt) for t in src])) if src else None
            xS = _thin_product(x2, S, skey, spec.width, dt) if src else None
        if need_out:
            outs = _forward_outputs(spec, x2, xS, Bs, skey, defer, dt, codes)
        else:  # only the graph for backward is needed (x2, xS saved); nobody reads the outputs
            STATS["bỏ đầu ra"] = STATS.get("bỏ đầu ra", 0) + 1
            outs = [None if i in spec.thin_ids else x2.new_empty(x2.shape[0], p[0].out_features)
                    for i, p in enumerate(parts)]
        for sl in spec.thin:
            outs[sl.layer] = xS[:, sl.cols].contiguous()
        if forms is not None:  # views of the persistent buffer: saved as views of their own, tracked (see _PLANS)
            S, Bs = S.view(S.shape), [b.view(b.shape) for b in Bs]
            forms.readers.append(weakref.ref(S))
        ctx.save_for_backward(x2, xS, S, *Bs)
        ctx.spec, ctx.skey, ctx.meta = spec, skey, (lead, K, dt, x.dtype)
        return tuple(y.view(*lead, y.shape[-1]) for y in outs)

    @staticmethod
    def backward(ctx, *dys):
        x2, xS, S, *Bs = ctx.saved_tensors
        spec, (lead, K, dt, xdt) = ctx.spec, ctx.meta
        need_x = ctx.needs_input_grad[0]
        flat = [None if dy is None else dy.reshape(-1, dy.shape[-1]).to(dt) for dy in dys]
        plan = _fused_bwd_plan(spec, flat, dt, need_x)
        if plan is not None:
            dx, grads = _fused_backward(spec, ctx.skey, x2, xS, S, Bs, flat, plan, need_x, dt)
            STATS["lan ngược gộp"] = STATS.get("lan ngược gộp", 0) + 1
        else:
            dx, grads = _plain_backward(spec, x2, xS, S, Bs, flat, need_x, dt)
        # A / B may be fp32 parameters while the math runs in bf16: autograd casts the gradients to their dtype
        wanted = ctx.needs_input_grad[4:]
        grads = [g if (g is not None and wanted[k]) else None for k, g in enumerate(grads)]
        return (None if dx is None else dx.view(*lead, K).to(xdt), None, None, None, *grads)


# ------------------------------------------------------------------------------------------- backward
def _add_dgrad(dx, base, dy, dt):
    """dx += dy · W of one base layer (MX: the quantized dy times the weight's second axis; bf16: addmm_)."""
    if _mx(base):
        import mxfp8
        qd, sd = mxfp8.mx_quant(dy if dy.is_contiguous() else dy.contiguous())
        g = mxfp8.mx_mm(qd, sd, *mxfp8.mx_wt(base))
        return g if dx is None else dx.add_(g)
    w = base.weight.to(dt)
    return dy @ w if dx is None else dx.addmm_(dy, w)


def _plain_backward(spec, x2, xS, S, Bs, flat, need_x, dt):
    """Per-layer backward (fused_linear.py:128-196): the base layers' dgrads, then the thin branch as one
    product dS = [s·dy·B of each adapter | dy of each thin linear] against the matching rows of S, and
    dA = dS_adaptersᵀ · x2."""
    dx = None
    if need_x:
        for i, (base, A, B, s) in enumerate(spec.parts):
            if flat[i] is not None and i not in spec.thin_ids:
                dx = _add_dgrad(dx, base, flat[i], dt)
    grads = [None] * (2 * len(spec.adapters))
    cols, used, live = [], [], []
    for sl in spec.adapters:
        dy = flat[sl.layer]
        if dy is None:
            continue
        dB, dxa = dy.t() @ xS[:, sl.cols], dy @ Bs[sl.index]
        if sl.scale != 1:
            dB.mul_(sl.scale)
            dxa.mul_(sl.scale)
        grads[2 * sl.index + 1] = dB
        cols.append(dxa)
        used.append(sl)
        live.append(sl)
    if need_x:
        for sl in spec.thin:
            if flat[sl.layer] is not None:
                cols.append(flat[sl.layer])
                used.append(sl)
    if not cols:
        return dx, grads
    dS = cols[0] if len(cols) == 1 else torch.cat(cols, 1)
    if need_x:
        rows = S if len(used) == len(spec.adapters) + len(spec.thin) else torch.cat([S[sl.cols] for sl in used])
        dx = dS @ rows if dx is None else dx.addmm_(dS, rows)
    if live:
        dA = dS[:, :sum(sl.width for sl in live)].t() @ x2
        c = 0
        for sl in live:
            grads[2 * sl.index] = dA[c:c + sl.width]
            c += sl.width
    return dx, grads


def _fused_bwd_plan(spec, flat, dt, need_x):
    """The B operand of the group's one dx GEMM ((codes, scales, layout), or None without dx) when the grouped
    backward applies (fused_linear.py:203-216): bf16 math, a gradient for every output, every MX layer in
    mxfp8.FUSED_BWD and, for dx, a concatenated Wᵀ covering exactly the group's MX layers in order.  None for
    the per-layer backward."""
    if dt != torch.bfloat16 or any(dy is None for dy in flat) or not spec.mx:
        return None
    if not all(getattr(spec.parts[i][0], "_mx_fbwd", False) for i in spec.mx):
        return None
    if not need_x:
        return (None,)
    import mxfp8
    wt = mxfp8.group_operand([spec.parts[i][0] for i in spec.mx])
    return None if wt is None else (wt,)


def _lora_bwd_batchable(spec, flat, xS):
    """The adapter slots of the group's MX layers when their lora_bwd calls can run as one batch: 2..8 MX layers,
    each with an adapter of one common rank 16 or 32 whose xS columns the kernel reads with 16-byte loads, and
    row-contiguous, 16-byte aligned dy; else None."""
    import _native
    slots = [spec.adapter(i) for i in spec.mx]
    if not 2 <= len(slots) <= _native.LORA_BWD_MAX_JOBS or any(sl is None for sl in slots):
        return None
    if len({sl.width for sl in slots}) != 1 or slots[0].width not in (16, 32):
        return None
    if not all(_vec_ok(xS[:, sl.cols]) for sl in slots):
        return None
    if not all(flat[i].stride(1) == 1 and flat[i].stride(0) % 8 == 0 and flat[i].data_ptr() % 16 == 0
               for i in spec.mx):
        return None
    return slots


def _fused_backward(spec, skey, x2, xS, S, Bs, flat, plan, need_x, dt):
    """Grouped backward through mxfp8.lora_bwd (fused_linear.py:219-279): each MX dy is read ONCE (its MX codes
    into a buffer concatenated along the group's N, its d(xa) into dS, its dB), then dx of the group is ONE MX
    GEMM with the concatenated Wᵀ (fp32 accumulation across the layers instead of a bf16 add per layer).  dS·S
    rides in that GEMM's epilogue and dA = dSᵀ·x2 runs on the token-reduction kernel when dS fits a padded
    width of 16/32/64 and no plain bf16 linear has to be added into dx first."""
    import mxfp8
    (wt,) = plan
    T, K, dev = x2.shape[0], x2.shape[1], x2.device
    n_cols = spec.adapter_cols + (sum(sl.width for sl in spec.thin) if need_x else 0)
    native = n_cols > 0 and _native_ok(x2, dt, n_cols) and not spec.plain
    width = _rp(n_cols) if native else n_cols
    # the dx GEMM's rank-r epilogue reads only the n_cols used columns of dS and St when n_cols is a rank it
    # takes (q|k|v at r = 16: 48), so the padding of dS stays unwritten; the token reduction's rows past n_cols,
    # computed from it, are dropped
    r_dx = n_cols if n_cols in (16, 32, 48, 64) else width
    dS = torch.empty((T, width), dtype=dt, device=dev) if n_cols else None
    if native and r_dx > n_cols:
        dS[:, n_cols:].zero_()
    grads = [None] * (2 * len(spec.adapters))
    q = sbuf = None
    if need_x:
        n_mx = sum(flat[i].shape[1] for i in spec.mx)
        q = torch.empty((T, n_mx), dtype=mxfp8.F8, device=dev)
        sbuf = torch.empty(_cdiv(T, 128) * (n_mx // 128) * 512, dtype=torch.uint8, device=dev)
    tile = 0
    batch = _lora_bwd_batchable(spec, flat, xS)
    if batch:
        # every MX layer's lora_bwd in one launch (mxfp8_lora_bwd_batch)
        offs, t = [], 0
        for i in spec.mx:
            offs.append(t)
            t += flat[i].shape[1] // 128
        dbs = mxfp8.lora_bwd_batch([flat[i] for i in spec.mx], [xS[:, sl.cols] for sl in batch],
                                   [Bs[sl.index] for sl in batch], [sl.scale for sl in batch],
                                   [dS[:, sl.cols] for sl in batch], q=q, s=sbuf, col_tile_offs=offs)
        for sl, db in zip(batch, dbs):
            grads[2 * sl.index + 1] = db
    for i in (() if batch else spec.mx):
        dy = flat[i] if flat[i].stride(1) == 1 else flat[i].contiguous()
        sl = spec.adapter(i)
        if sl is not None and sl.width in (16, 32) and _vec_ok(xS[:, sl.cols]):
            grads[2 * sl.index + 1] = mxfp8.lora_bwd(dy, xS[:, sl.cols], Bs[sl.index], sl.scale, q=q, s=sbuf,
                                                     col_tile_off=tile, dxa_out=dS[:, sl.cols])
        else:
            if q is not None:
                mxfp8.lora_bwd(dy, q=q, s=sbuf, col_tile_off=tile)
            if sl is not None:  # a rank or xa layout the fused kernel does not take: the products as GEMMs
                grads[2 * sl.index + 1] = (dy.t().float() @ xS[:, sl.cols].float()).mul_(sl.scale)
                dS[:, sl.cols] = (dy.float() @ Bs[sl.index].float()).mul_(sl.scale)
        tile += dy.shape[1] // 128
    mx_ids = set(spec.mx)
    for sl in spec.adapters:  # LoRA on a non-MX base layer (rare): as the per-layer backward
        if sl.layer in mx_ids:
            continue
        dy = flat[sl.layer]
        dB = dy.t() @ xS[:, sl.cols]
        dS[:, sl.cols] = dy @ Bs[sl.index]
        if sl.scale != 1:
            dB.mul_(sl.scale)
            dS[:, sl.cols].mul_(sl.scale)
        grads[2 * sl.index + 1] = dB
    dx = dA = None
    a32 = bool(spec.adapters) and all(spec.parts[sl.layer][1].dtype == torch.float32 for sl in spec.adapters)

    def tn_job():
        # bf16(dSᵀ·x2), held in fp32 when every A is an fp32 parameter: autograd would cast each bf16 slice to its
        # parameter's dtype anyway (exactly), one kernel per adapter.  (job, its partial-sum scratch)
        import _native
        out = torch.empty((width, K), dtype=torch.float32 if a32 else dt, device=dev)
        n_part = _native.lora_tn_chunks(T, K) * width * K
        part = _native.scratch_f32(n_part, dev)[:n_part]  # partial sums, read by the launch's sum kernel
        return (x2, dS, out, 1.0, False), part

    if need_x:
        wq, ws, lay = wt
        for sl in spec.thin:
            dS[:, sl.cols].copy_(flat[sl.layer])
        codes = (q, sbuf.view(mxfp8.E8))
        if native:
            # bf16(bf16(MX GEMM) + dS·S): the reference's dx.addmm_(dS, S) in the GEMM epilogue
            # this step's St only if the saved S is a view of the same buffer: a backward that runs after the next
            # step's forward has the saved S of its own step (see _PLANS), so it builds St from that S
            forms = _CAST.get(skey + ("forms",))
            if forms is not None and forms.rp == width and _same_buffer(S, forms.S_pad):
                St = forms.St
            else:
                ent = _CAST.get(skey + ("padT", width))
                if ent is None or ent[0] is not S:
                    pad = torch.cat([S, S.new_zeros(width - S.shape[0], S.shape[1])]) if width > S.shape[0] else S
                    ent = _CAST[skey + ("padT", width)] = (S, pad.t().contiguous())
                St = ent[1]
            lora = (dS[:, :r_dx], St[:, :r_dx])
            import _native
            if spec.adapters and FOLD_TN[0] and r_dx in (16, 32, 48) and not lay & _native.GEMM_WIDE:
                # the dA reduction in the dx GEMM's launch: the same bits as the two calls below
                job, part = tn_job()
                dA = job[2]
                dx = mxfp8.mx_mm_tn(*codes, wq, ws, lora, 1.0, lay, T, [job], part)
            else:
                dx = mxfp8.mx_mm(*codes, wq, ws, layout=lay, lora=lora, alpha=1.0)
        else:
            dx = mxfp8.mx_mm(*codes, wq, ws, layout=lay)
            for i in spec.plain:  # plain bf16 linears (neither MX nor thin)
                dx.addmm_(flat[i], spec.parts[i][0].weight.to(dt))
            if dS is not None:
                dx.addmm_(dS, S)
        del codes, q, sbuf
    if spec.adapters:
        if native and dA is None:
            import _native
            job, part = tn_job()
            dA = job[2]
            _native.lora_tn(x2, dS, dA, part)
        elif not native:
            dA = dS[:, :spec.adapter_cols].t() @ x2
        for sl in spec.adapters:
            grads[2 * sl.index] = dA[sl.cols]
    return dx, grads


# ------------------------------------------------------------------------------------------- residual + LoRA-B
class Deferred(tuple):
    """(y, xa, B, scaling): the bf16 MX output of o_proj / out_proj WITHOUT its LoRA part; residual_add adds it
    (fused_linear.py:282-284)."""


class _ResidualLoRA(torch.autograd.Function):
    """x + (y + s · xa·Bᵀ) in ONE kernel (mxfp8.res_lora): the residual add reads y and x and writes the new x
    anyway, so adding the rank-r product there saves a read and a write of [T, N].  xa and B are detached: the
    LoRA gradients (dB, d(xa) -> dA, dx) come from _Group.backward with the same upstream gradient, which passes
    through here to both x and y (fused_linear.py:287-300)."""

    @staticmethod
    def forward(ctx, x, y, xa, B, s):
        import mxfp8
        n = x.shape[-1]
        return mxfp8.res_lora(x.reshape(-1, n), y.reshape(-1, n), xa, B, s).view(x.shape)

    @staticmethod
    def backward(ctx, g):
        return g, g, None, None, None


def _res_kernel_ok(x, y, xa, B):
    return (x.dtype == y.dtype == torch.bfloat16 and x.shape == y.shape and x.is_contiguous() and y.is_contiguous()
            and x.shape[-1] % 128 == 0 and xa.stride(1) == 1 and B.is_contiguous() and xa.shape[1] in (16, 32))


def residual_add(x, y):
    """x + y; a Deferred y gets its LoRA part added inside the residual kernel when it qualifies, else by a torch
    addmm first (fused_linear.py:303-312)."""
    if not isinstance(y, Deferred):
        return x + y
    y0, xa, B, s = y
    if _res_kernel_ok(x, y0, xa, B):
        STATS["residual LoRA"] = STATS.get("residual LoRA", 0) + 1
        return _ResidualLoRA.apply(x, y0, xa, B, s)
    n = x.shape[-1]
    return x + torch.addmm(y0.reshape(-1, n), xa, B.t(), alpha=s).view(y0.shape)


def group_linear(x, mods, need_out=True, defer=False):
    """The outputs m(x) of every module in `mods`, computed as one group (fused_linear.py:315-330).
    need_out=False builds only the graph for backward (outputs uninitialised), for the recomputation of a
    checkpointed segment's last layer whose outputs nobody reads; the gradients are the same.
    defer=True returns MX bf16 outputs with LoRA as Deferred (LoRA not yet added), for a residual_add right
    after."""
    parts = tuple(_part(m) for m in mods)
    if any(p is None for p in parts):
        STATS["gọi thẳng"] += 1
        return tuple(m(x) for m in mods)
    STATS["gộp"] += 1
    ws = [t for base, A, B, s in parts if A is not None for t in (A, B)]
    box = {} if defer and need_out else None
    outs = _Group.apply(x, parts, need_out, box, *ws)
    if not box:
        return outs
    return tuple(Deferred((y,) + box[i]) if i in box else y for i, y in enumerate(outs))
