"""The block-pair fast memory at the full benchmark shapes (110M: B=16,
T=1024, A=3072, D=768; 42M: B=16, T=1024, A=2048, D=512; 15M: B=32, T=256,
A=1152, D=288; v and fast in bf16; needs an MI355X), through a property that
holds at any size: batch rows are independent. Every per-row output and
gradient of the full-batch call (q, fast, dr, dv) equals, bit for bit, that
of a B=1 call on the same row: a tile's arithmetic does not depend on which
workgroup runs it or what runs beside it. dg and dw are sums over the rows;
they match the sums of the row calls' within fp32 rounding. The B=1 call of
the same product form and shape is held to the float64 oracle in
test_gpu_parity (PATH_CASES).

Only the full shapes run all rows of jobs in the XCD-local order, dv on the
device's second stream (B T^2 D >= 2e9: the 110M and 42M shapes) and, at the
110M shape, the scores' tile copies of v on the CUs the 160 score tiles leave
idle, so those are what this test adds.
"""
import pytest
import torch

from helpers import fm_inputs, rel, say

pytestmark = pytest.mark.gpu

import kernel  # noqa: E402
import ulm_native as nat  # noqa: E402


SHAPES = [(16, 1024, 3072, 768), (16, 1024, 2048, 512), (32, 256, 1152, 288)]


@pytest.mark.parametrize("B,T,A,D", SHAPES)
def test_full_shape_rows_match_single_row_calls(B, T, A, D, monkeypatch):
    say(f"full-shape row independence: block-pair form, B={B} T={T} A={A} D={D}, v bf16")
    monkeypatch.setenv("ULM_FM_PATH", "pair")
    assert nat.lib().ulm_fm_path(B, T, A, D) == 2
    r, v, g, w = fm_inputs(B, T, A, D, seed=B + T + A, device="cuda")
    r, g, w = r.float(), g.float(), w.float()
    v = v.to(torch.bfloat16)
    gen = torch.Generator(device="cuda").manual_seed(16)
    dq = torch.randn(B, T, A, device="cuda", generator=gen)
    df = torch.randn(B, T, D, device="cuda", generator=gen).to(torch.bfloat16)

    def call(rows):
        ins = [r[rows].contiguous().requires_grad_(), v[rows].contiguous().requires_grad_(),
               g.clone().requires_grad_(), w.clone().requires_grad_()]
        q, fast = kernel.unified_memory(*ins)
        grads = torch.autograd.grad((q, fast), ins, (dq[rows].contiguous(), df[rows].contiguous()))
        return (q.detach(), fast.detach()) + tuple(grads)

    q, fast, dr, dv, dg, dw = call(slice(None))
    torch.cuda.synchronize()
    assert fast.dtype == torch.bfloat16 and dv.dtype == torch.bfloat16
    dg_rows = torch.zeros((), dtype=torch.float64, device="cuda")
    dw_rows = torch.zeros(A, dtype=torch.float64, device="cuda")
    for b in range(B):
        q1, f1, dr1, dv1, dg1, dw1 = call(slice(b, b + 1))
        for name, full, one in (("q", q, q1), ("fast", fast, f1), ("dr", dr, dr1), ("dv", dv, dv1)):
            assert torch.equal(full[b:b + 1], one), (name, b)
        dg_rows += dg1.double()
        dw_rows += dw1.double()
    torch.cuda.synchronize()
    errs = {"dg": rel(dg, dg_rows), "dw": rel(dw, dw_rows)}
    say(f"  per-row outputs equal; dg, dw against the row sums {errs}")
    assert max(errs.values()) < 1e-5, errs
    assert torch.isfinite(dr).all() and dr.abs().max() > 0
