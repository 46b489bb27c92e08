"""The deferred decode state (ulm_decode_dots / ulm_decode_read /
ulm_decode_flush) against ulm_decode_state position by position (needs an
MI355X): the same write S <- lam S + v r_prev^T and read-out x + S q + ymu
(model.py:107-109, run.c:244-255), the writes held as pending terms and
written back every 16 positions. Outputs (to 1e-6 of the size of the terms
they sum) and, after each write-back, the state itself (1e-6 relative) agree
within fp32 rounding. Widths: 3072 slots (12 16-byte slices per lane), 712 and
1000 (a row cut inside a lane's last slice), 4096 (the largest), 256, and
seeded draws; feature counts off the 16 rows of a workgroup."""
import math

import pytest
import torch

from helpers import rel, say

pytestmark = pytest.mark.gpu

import kernel  # noqa: E402
import ulm_native as nat  # noqa: E402

J = 16


def _random_state_cases(n, seed):
    """Seeded (N, D, A) draws within the deferred form's limits (A % 4 == 0,
    A <= 4096): feature counts on and off the kernels' row groups."""
    import random
    rng = random.Random(seed)
    return [(rng.choice([1, 2, 3, 5, 8]), rng.choice([1, 7, 16, 17, 33, 64, 100]),
             4 * rng.randint(1, 1024)) for _ in range(n)]


def _read_err(got, ref, S, q, x, ymu):
    """|got - ref| over the size of what the read-out sums, |x| + |ymu| +
    |S| |q|: an output of a few elements whose A-term sum cancels would make
    a plain relative error measure the cancellation, not the kernels."""
    scale = x.abs() + ymu.abs() + torch.bmm(S.abs(), q.abs()[:, :, None])[:, :, 0]
    return ((got - ref).norm() / scale.norm()).item()


@pytest.mark.parametrize("N,D,A", [(3, 40, 3072), (2, 17, 712), (1, 8, 4096), (4, 24, 256), (2, 9, 1000)]
                         + _random_state_cases(10, 5))
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
        err = _read_err(got, ref, S, q, x, ymu)
        assert err < 1e-6, (t, m, err)
        if m == J:
            serr = rel(Sb, S)
            say(f"  write-back at position {t}: state rel {serr:.2e}, output rel {err:.2e}")
            assert serr < 1e-6, (t, serr)
            m = 0
