"""GPU checks of mxfp8_gemm_nt_tn: the LoRA-epilogue MX GEMM whose launch also runs the token reductions of
mxfp8_lora_tn_batch in workgroups past its tiles (the MLP backward's dx GEMM with its dB_d / dA reductions,
/root/reference/scripts/fused_mlp.py:331, :316-318, :333, at epilogue rank 32; the grouped linears' dx GEMMs with
dA, fused_linear.py:269, :271, at ranks 16 and 48 with a rank-64 reduction).  The folded launch computes what the
two separate calls compute, with the same kernels' arithmetic in the same order, so the bar is bit-identical
outputs:
  - the GEMM output and both reductions against mxfp8_gemm_nt followed by mxfp8_lora_tn_batch, at the MLP's
    configuration-3 dx shape (672 tiles: the reductions run in the last round's idle slots), at a small shape
    whose few tiles leave most slots free from the start, with T not a multiple of 32 or 128, and at T = 1;
  - the whole fused MLP step with the fold on and off (fused_mlp.FOLD_TN): output, dx and every LoRA gradient.
The same bar for mxfp8_gemm_nt_sum (the forward's down GEMM whose launch also sums its epilogue operand from the
xS_down partials, :214, :283-284) against mxfp8_sum_parts then mxfp8_gemm_nt, and for both entry points captured
into a HIP graph and replayed with new inputs."""
import pytest
import torch

import _native
import fused_linear
import fused_mlp
import mxfp8
import workloads

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K,Kt", [(10752, 2048, 12288, 2048), (300, 256, 512, 1024), (1, 128, 256, 128),
                                      (2000, 1024, 2048, 768)])
def test_gemm_nt_tn_matches_separate_calls(M, N, K, Kt, gpu):
    g = torch.Generator().manual_seed(M + N + K)
    a = (torch.randn(M, K, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    b = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(gpu)
    qa, sa = mxfp8.mx_quant_tiled(a)
    qb, sb = mxfp8.mx_quant_tiled(b)
    P = (torch.randn(M, 32, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    Q = (torch.randn(N, 32, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    # the MLP's two reductions: dB_d = bf16(bf16(dyᵀ xsd) s) [Kt, 16] transposed, dA = bf16(dxaᵀ x) [32, Kt] fp32
    x0 = torch.randn(M, Kt, generator=g).to(torch.bfloat16).to(gpu)
    p0 = (torch.randn(M, 16, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    x1 = torch.randn(M, Kt, generator=g).to(torch.bfloat16).to(gpu)
    p1 = (torch.randn(M, 32, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    chunks = _native.lora_tn_chunks(M, Kt)
    part = torch.empty(chunks * 48 * Kt, device=gpu)

    ref_c = mxfp8.mx_mm(qa, sa, qb, sb, lora=(P, Q), alpha=2.0, layout=3, m=M)
    r0 = torch.empty((Kt, 16), dtype=torch.bfloat16, device=gpu)
    r1 = torch.empty((32, Kt), dtype=torch.float32, device=gpu)
    _native.lora_tn_batch([(x0, p0, r0, 2.0, True), (x1, p1, r1, 1.0, False)], part)
    torch.cuda.synchronize()

    o0 = torch.full_like(r0, float("nan"))
    o1 = torch.full_like(r1, float("nan"))
    part.fill_(float("nan"))  # the folded launch must write every partial it sums
    c = mxfp8.mx_mm_tn(qa, sa, qb, sb, (P, Q), 2.0, 3, M, [(x0, p0, o0, 2.0, True), (x1, p1, o1, 1.0, False)], part)
    torch.cuda.synchronize()
    assert torch.equal(c.view(torch.int16), ref_c.view(torch.int16))
    assert torch.equal(o0.view(torch.int16), r0.view(torch.int16))
    assert torch.equal(o1.view(torch.int32), r1.view(torch.int32))


@pytest.mark.parametrize("r,M,N,K,Kt,rps,layout", [
    (48, 10752, 2048, 3072, 2048, (64,), 2),  # the grouped q|k|v dx GEMM at configuration 3 and its dA
    (16, 10752, 2048, 2048, 2048, (16,), 2),  # the o_proj dx GEMM and its dA
    (48, 300, 256, 512, 1024, (64, 16), 3),
    (16, 1, 128, 256, 128, (64, 32, 16), 3),
    (32, 2000, 1024, 2048, 768, (64, 32), 2),
    (48, 50000, 256, 256, 2048, (64, 16), 3)])  # x of 205 MB: the reductions' one-step register ring
def test_gemm_nt_tn_other_ranks_match_separate_calls(r, M, N, K, Kt, rps, layout, gpu):
    """The epilogue ranks 16 and 48 and the rank-64 reduction (the grouped linears' backward): the GEMM with its
    epilogue operands as column views of wider buffers whose columns past r hold NaN (the padded dS and Sᵀ), and
    the reductions, against mx_mm then lora_tn_batch."""
    g = torch.Generator().manual_seed(M + N + K + r)
    a = (torch.randn(M, K, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    b = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(gpu)
    qa, sa = mxfp8.mx_quant_tiled(a) if layout & 1 else mxfp8.mx_quant(a)
    qb, sb = mxfp8.mx_quant_tiled(b)
    P = (torch.randn(M, 64, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    Q = (torch.randn(N, 64, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    P[:, r:] = float("nan")
    Q[:, r:] = float("nan")
    lora = (P[:, :r], Q[:, :r])
    xs = [torch.randn(M, Kt, generator=g).to(torch.bfloat16).to(gpu) for _ in rps]
    ps = [(torch.randn(M, rp, generator=g) * 0.1).to(torch.bfloat16).to(gpu) for rp in rps]
    part = torch.empty(_native.lora_tn_chunks(M, Kt) * sum(rps) * Kt, device=gpu)

    def outs(fill):
        return [torch.full(((Kt, rp) if j % 2 else (rp, Kt)), fill, dtype=torch.bfloat16 if j % 2 else torch.float32,
                           device=gpu) for j, rp in enumerate(rps)]

    def jobs(o):
        return [(x, p, oo, 2.0 if j % 2 else 1.0, bool(j % 2)) for j, (x, p, oo) in enumerate(zip(xs, ps, o))]

    ref_c = mxfp8.mx_mm(qa, sa, qb, sb, lora=lora, alpha=1.0, layout=layout, m=M)
    ref = outs(0.0)
    _native.lora_tn_batch(jobs(ref), part)
    torch.cuda.synchronize()
    got = outs(float("nan"))
    part.fill_(float("nan"))
    c = mxfp8.mx_mm_tn(qa, sa, qb, sb, lora, 1.0, layout, M, jobs(got), part)
    torch.cuda.synchronize()
    assert torch.equal(c.view(torch.int16), ref_c.view(torch.int16))
    assert not torch.isnan(c).any()
    for j, (o, w) in enumerate(zip(got, ref)):
        assert torch.equal(o.view(torch.int16), w.view(torch.int16)), j


def _grads(m):
    return [m.gate_proj.lora_A["default"].weight.grad, m.gate_proj.lora_B["default"].weight.grad,
            m.up_proj.lora_A["default"].weight.grad, m.up_proj.lora_B["default"].weight.grad,
            m.down_proj.lora_A["default"].weight.grad, m.down_proj.lora_B["default"].weight.grad]


@pytest.mark.parametrize("T", [2048, 1000])
def test_mlp_step_with_and_without_the_fold(T, gpu, monkeypatch):
    model, inps = workloads.build_model(3, T=T, device=gpu)
    mxfp8.enable_mxfp8(model)
    mod = model.layers[0].mlp
    x, dy = inps[0]["x"].to(gpu), inps[0]["dy"].to(gpu)
    outs = []
    for fold in (False, True):
        monkeypatch.setattr(fused_mlp, "FOLD_TN", [fold])
        fused_linear.new_step()
        for p in model.parameters():
            p.grad = None
        xi = x.clone().requires_grad_(True)
        y = fused_mlp.mlp(mod, xi)
        y.backward(dy)
        torch.cuda.synchronize()
        outs.append([y.detach(), xi.grad] + [t.detach().clone() for t in _grads(mod)])
    for k, (a, b) in enumerate(zip(*outs)):
        assert torch.equal(a, b), k


@pytest.mark.parametrize("M,N,K,n_parts", [(10752, 2048, 6144, 96), (1000, 256, 128, 7), (1, 128, 256, 3),
                                           (4097, 1024, 512, 24)])
@pytest.mark.parametrize("wait_limit", [-1, 0])
def test_gemm_nt_sum_matches_separate_calls(M, N, K, n_parts, wait_limit, gpu):
    """mxfp8_gemm_nt_sum against mxfp8_sum_parts then mxfp8_gemm_nt: P and the GEMM output bit-identical, with the
    tiles waiting for the summing workgroups (K = 128: the tiles reach their epilogue almost at once) and with
    wait_limit 0, where every tile sums its own rows of P from the partials; three launches into one P buffer, so a
    tile that read an earlier launch's P (a stale cache line) or flag would fail."""
    g = torch.Generator().manual_seed(M + N + K + n_parts)
    a = (torch.randn(M, K, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    b = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(gpu)
    qa, sa = mxfp8.mx_quant_tiled(a)
    qb, sb = mxfp8.mx_quant_tiled(b)
    Q = (torch.randn(N, 16, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    p_out = torch.full((M, 16), float("nan"), dtype=torch.bfloat16, device=gpu)
    # three launches into the same P buffer with new partials each time: a later launch finds the earlier ones'
    # flags and P values, and must read neither
    for it in range(3):
        part = torch.randn(n_parts, M, 16, generator=g).to(gpu)
        p_ref = torch.empty((M, 16), dtype=torch.bfloat16, device=gpu)
        _native.sum_parts(part, n_parts, M * 16, p_ref)
        ref_c = mxfp8.mx_mm(qa, sa, qb, sb, lora=(p_ref, Q), alpha=2.0, layout=3, m=M)
        torch.cuda.synchronize()
        c = mxfp8.mx_mm_sum(qa, sa, qb, sb, part, p_out, Q, 2.0, 3, M, wait_limit=wait_limit)
        torch.cuda.synchronize()
        assert torch.equal(p_out.view(torch.int16), p_ref.view(torch.int16)), it
        assert torch.equal(c.view(torch.int16), ref_c.view(torch.int16)), it


@pytest.mark.parametrize("T", [2048, 1000])
def test_mlp_step_with_and_without_the_forward_sum_fold(T, gpu, monkeypatch):
    model, inps = workloads.build_model(3, T=T, device=gpu)
    mxfp8.enable_mxfp8(model)
    mod = model.layers[0].mlp
    x, dy = inps[0]["x"].to(gpu), inps[0]["dy"].to(gpu)
    outs = []
    for fold in (False, True):
        monkeypatch.setattr(fused_mlp, "FOLD_SUM", [fold])
        fused_linear.new_step()
        for p in model.parameters():
            p.grad = None
        xi = x.clone().requires_grad_(True)
        y = fused_mlp.mlp(mod, xi)
        y.backward(dy)
        torch.cuda.synchronize()
        outs.append([y.detach(), xi.grad] + [t.detach().clone() for t in _grads(mod)])
    for k, (a, b) in enumerate(zip(*outs)):
        assert torch.equal(a, b), k


def test_gemm_nt_sum_on_two_streams_at_once(gpu):
    """Two mxfp8_gemm_nt_sum launches in flight together on two streams (default priority), each with its own
    inputs, K = 128 so that tiles reach their epilogue while summing workgroups still run: each launch publishes in
    its own slice of the flag array, and both results are bit-identical to their separate references."""
    M, N, K, n_parts = 4000, 512, 128, 12
    g = torch.Generator().manual_seed(7)
    cases = []
    for _ in range(2):
        a = (torch.randn(M, K, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
        b = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(gpu)
        qa, sa = mxfp8.mx_quant_tiled(a)
        qb, sb = mxfp8.mx_quant_tiled(b)
        part = torch.randn(n_parts, M, 16, generator=g).to(gpu)
        Q = (torch.randn(N, 16, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
        p_ref = torch.empty((M, 16), dtype=torch.bfloat16, device=gpu)
        _native.sum_parts(part, n_parts, M * 16, p_ref)
        ref = mxfp8.mx_mm(qa, sa, qb, sb, lora=(p_ref, Q), alpha=1.0, layout=3, m=M)
        cases.append((qa, sa, qb, sb, part, Q, p_ref, ref))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = []
    for rep in range(3):
        res = [None, None]
        for k, st in enumerate(streams):
            with torch.cuda.stream(st):
                qa, sa, qb, sb, part, Q, _, _ = cases[k]
                p_out = torch.empty((M, 16), dtype=torch.bfloat16, device=gpu)
                res[k] = (p_out, mxfp8.mx_mm_sum(qa, sa, qb, sb, part, p_out, Q, 1.0, 3, M))
        torch.cuda.synchronize()
        outs.append(res)
    for res in outs:
        for k, (p_out, c) in enumerate(res):
            assert torch.equal(p_out.view(torch.int16), cases[k][6].view(torch.int16)), k
            assert torch.equal(c.view(torch.int16), cases[k][7].view(torch.int16)), k


def _capture(fn):
    """fn() captured into a HIP graph (after one warm-up call on the capture stream); returns (graph, its output)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


def test_gemm_nt_sum_under_graph_capture(gpu):
    """mxfp8_gemm_nt_sum captured into a HIP graph and replayed four times, new partials copied in eagerly before
    each replay and the eager references computed between replays: every replay's P and GEMM output bit-identical
    to mxfp8_sum_parts then mxfp8_gemm_nt on that replay's partials.  A replay repeats the captured launch's
    arguments, so a flag matched against a captured launch id would already hold it from the replay before (K =
    128: the tiles reach their epilogue while the sums run), and a tile would read the previous replay's P."""
    M, N, K, n_parts = 4000, 512, 128, 12
    gen = torch.Generator().manual_seed(11)
    a = (torch.randn(M, K, generator=gen) * 0.1).to(torch.bfloat16).to(gpu)
    b = (torch.randn(N, K, generator=gen) * 0.02).to(torch.bfloat16).to(gpu)
    qa, sa = mxfp8.mx_quant_tiled(a)
    qb, sb = mxfp8.mx_quant_tiled(b)
    Q = (torch.randn(N, 16, generator=gen) * 0.1).to(torch.bfloat16).to(gpu)
    part = torch.randn(n_parts, M, 16, generator=gen).to(gpu)
    p_out = torch.empty((M, 16), dtype=torch.bfloat16, device=gpu)
    graph, c = _capture(lambda: mxfp8.mx_mm_sum(qa, sa, qb, sb, part, p_out, Q, 1.5, 3, M))
    for it in range(4):
        part.copy_(torch.randn(n_parts, M, 16, generator=gen).to(gpu))
        p_ref = torch.empty((M, 16), dtype=torch.bfloat16, device=gpu)
        _native.sum_parts(part, n_parts, M * 16, p_ref)
        ref = mxfp8.mx_mm(qa, sa, qb, sb, lora=(p_ref, Q), alpha=1.5, layout=3, m=M)
        torch.cuda.synchronize()
        p_out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(p_out.view(torch.int16), p_ref.view(torch.int16)), it
        assert torch.equal(c.view(torch.int16), ref.view(torch.int16)), it
    del graph


def test_gemm_nt_tn_under_graph_capture(gpu):
    """mxfp8_gemm_nt_tn captured into a HIP graph and replayed three times with new token-side inputs copied in
    before each replay: the GEMM output and both reductions bit-identical to the separate eager calls."""
    M, N, K, Kt = 1000, 256, 512, 768
    gen = torch.Generator().manual_seed(12)
    a = (torch.randn(M, K, generator=gen) * 0.1).to(torch.bfloat16).to(gpu)
    b = (torch.randn(N, K, generator=gen) * 0.02).to(torch.bfloat16).to(gpu)
    qa, sa = mxfp8.mx_quant_tiled(a)
    qb, sb = mxfp8.mx_quant_tiled(b)
    P = (torch.randn(M, 32, generator=gen) * 0.1).to(torch.bfloat16).to(gpu)
    Q = (torch.randn(N, 32, generator=gen) * 0.1).to(torch.bfloat16).to(gpu)
    x0 = torch.empty((M, Kt), dtype=torch.bfloat16, device=gpu)
    p0 = torch.empty((M, 16), dtype=torch.bfloat16, device=gpu)
    x1 = torch.empty((M, Kt), dtype=torch.bfloat16, device=gpu)
    p1 = torch.empty((M, 32), dtype=torch.bfloat16, device=gpu)
    chunks = _native.lora_tn_chunks(M, Kt)
    part = torch.empty(chunks * 48 * Kt, device=gpu)
    o0 = torch.empty((Kt, 16), dtype=torch.bfloat16, device=gpu)
    o1 = torch.empty((32, Kt), dtype=torch.float32, device=gpu)

    def fill():
        x0.copy_(torch.randn(M, Kt, generator=gen).to(torch.bfloat16))
        p0.copy_((torch.randn(M, 16, generator=gen) * 0.1).to(torch.bfloat16))
        x1.copy_(torch.randn(M, Kt, generator=gen).to(torch.bfloat16))
        p1.copy_((torch.randn(M, 32, generator=gen) * 0.1).to(torch.bfloat16))

    fill()
    graph, c = _capture(lambda: mxfp8.mx_mm_tn(qa, sa, qb, sb, (P, Q), 2.0, 3, M,
                                               [(x0, p0, o0, 2.0, True), (x1, p1, o1, 1.0, False)], part))
    for it in range(3):
        fill()
        ref_c = mxfp8.mx_mm(qa, sa, qb, sb, lora=(P, Q), alpha=2.0, layout=3, m=M)
        r0 = torch.empty((Kt, 16), dtype=torch.bfloat16, device=gpu)
        r1 = torch.empty((32, Kt), dtype=torch.float32, device=gpu)
        _native.lora_tn_batch([(x0, p0, r0, 2.0, True), (x1, p1, r1, 1.0, False)], torch.empty_like(part))
        torch.cuda.synchronize()
        o0.fill_(float("nan"))
        o1.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(c.view(torch.int16), ref_c.view(torch.int16)), it
        assert torch.equal(o0.view(torch.int16), r0.view(torch.int16)), it
        assert torch.equal(o1.view(torch.int32), r1.view(torch.int32)), it
    del graph
