"""The deferred decode state (ulm_decode_dots / ulm_decode_read /
ulm_decode_flush) against ulm_decode_state position by position (needs an
MI355X): the same write S <- lam S + v r_prev^T and read-out x + S q + ymu
(model.py:107-109, run.c:244-255), the writes held as pending terms and
written back every 16 positions. Outputs and, after each write-back, the state
itself agree within fp32 rounding (1e-6). Widths: 3072 slots (12 16-byte
slices per lane), 712 and 1000 (a row cut inside a lane's last slice), 4096
(the largest), 256; feature counts off the 16 rows of a workgroup."""
import math

import pytest
import torch

from helpers import rel, say

pytestmark = pytest.mark.gpu

import kernel  # noqa: E402
import ulm_native as nat  # noqa: E402

J = 16


@pytest.mark.parametrize("N,D,A", [(3, 40, 3072), (2, 17, 712), (1, 8, 4096), (4, 24, 256), (2, 9, 1000)])
def test_deferred_state_matches_direct(N, D, A):
    say(f"deferred decode state N={N} D={D} A={A}, {J} terms per write-back")
    assert nat.lib().ulm_decode_max_pending() == J
    dev = "cuda"
    gen = torch.Generator(device=dev).manual_seed(N * 1000 + D + A)
    S = torch.randn(N, D, A, device=dev, generator=gen) * 0.1
    Sb = S.clone()
    pv = torch.zeros(J, N, D, device=dev)
    pr = torch.zeros(J, N, A, device=dev)
    g = torch.tensor([math.log(0.97)], device=dev)
    m = 0
    for t in range(2 * J + 3):
        v = torch.randn(N, D, device=dev, generator=gen)
        rp = torch.rand(N, A, device=dev, generator=gen) / A
        q = torch.rand(N, A, device=dev, generator=gen)
        x = torch.randn(N, D, device=dev, generator=gen)
        ymu = torch.randn(N, D, device=dev, generator=gen)
        ref = kernel.decode_state(S, v, rp, q, g, x, ymu)
        pv[m].copy_(v)
        pr[m].copy_(rp)
        m += 1
        got = kernel.decode_deferred(Sb, pv, pr, m, m == J, q, g, x, ymu)
        torch.cuda.synchronize()
        err = rel(got, ref)
        assert err < 1e-6, (t, m, err)
        if m == J:
            serr = rel(Sb, S)
            say(f"  write-back at position {t}: state rel {serr:.2e}, output rel {err:.2e}")
            assert serr < 1e-6, (t, serr)
            m = 0
