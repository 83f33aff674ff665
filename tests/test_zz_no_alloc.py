"""GPU test of the allocation-free token reduction mxfp8_lora_tn_noalloc, called through the C-ABI (_native):
its output must equal, bit for bit, that of the allocating entry point mxfp8_lora_tn run with the same chunk
count (the same kernels and summation order), on two calls in a row whose second input is smaller, so that the
shared static scratch left by the first call cannot leak into the second.  A float64 product bounds both."""
import pytest
import torch

import _native

pytestmark = pytest.mark.gpu

CASES = [  # (T, K, rp, scale, transpose, out dtype): the second call is the smaller one
    (10752, 2048, 32, 1.0, False, torch.bfloat16),  # dA = bf16(dxaᵀ · x) at the headline shape
    (300, 1024, 16, 2.0, True, torch.float32),      # dB_d = bf16(bf16(dyᵀ · xsd) · s), transposed, fp32 holder
]


def _inputs(T, K, rp, seed, dev):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16).to(dev)
    p = (torch.randn(T, rp, generator=g) * 0.1).to(torch.bfloat16).to(dev)
    return x, p


def test_noalloc_matches_allocating_entry_point_twice(gpu):
    for n, (T, K, rp, scale, transpose, dt) in enumerate(CASES):
        x, p = _inputs(T, K, rp, 100 + n, gpu)
        shape = (K, rp) if transpose else (rp, K)
        got = torch.empty(shape, dtype=dt, device=gpu)
        _native.lora_tn_noalloc(x, p, got, scale=scale, transpose=transpose)
        chunks = _native.lora_tn_noalloc_chunks(T, K, rp)
        assert chunks > 0
        part = torch.empty(chunks * rp * K, dtype=torch.float32, device=gpu)
        ref = torch.empty(shape, dtype=dt, device=gpu)
        _native.lora_tn(x, p, ref, part, scale=scale, transpose=transpose)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (T, K, rp, (got.float() - ref.float()).abs().max().item())
        want = p.double().t().cpu() @ x.double().cpu()
        want = want.to(torch.bfloat16).double() * scale
        want = want.t() if transpose else want
        err = (got.double().cpu() - want).abs()
        assert (err <= want.abs() * 2.0 ** -7 + 1e-3 * want.abs().max()).all(), err.max().item()
