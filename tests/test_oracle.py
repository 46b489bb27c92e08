"""Pins the float64 oracle (CPU only).

Each oracle function is checked against something other than its own formula:
a brute-force scalar loop, the recurrent (U, c) form, closed-form special
cases, finite differences, the reference's invariant tests (test_all.py:100-137)
and the logits of the reference's own run.c (golden fixture + live build).
"""
import math
import os
import tempfile

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import fastmem as fm
from oracle import runc, ulme

TOL = 1e-8  # test_all.py:22


def _inputs(B=2, T=11, A=5, D=3, seed=0, lam=0.8):
    g = torch.Generator().manual_seed(seed)
    r = torch.rand(B, T, A, generator=g, dtype=torch.float64)
    r = r / (1 + r.sum(-1, keepdim=True))
    v = torch.randn(B, T, D, generator=g, dtype=torch.float64)
    w = torch.rand(A, generator=g, dtype=torch.float64) * 3 + 0.1
    return r, v, torch.tensor(math.log(lam), dtype=torch.float64), w


def _brute(r, v, lam, w):
    """Scalar double loop straight from the definitions (kernel.py:4-9)."""
    B, T, A = r.shape
    D = v.shape[-1]
    r, v, w, lam = r.tolist(), v.tolist(), w.tolist(), float(lam)
    key = lambda b, s, a: r[b][s - 1][a] if s > 0 else 0.0
    q = [[[0.0] * A for _ in range(T)] for _ in range(B)]
    f = [[[0.0] * D for _ in range(T)] for _ in range(B)]
    for b in range(B):
        for t in range(T):
            for a in range(A):
                c = w[a] + sum(lam ** (t - s) * key(b, s, a) for s in range(t + 1))
                q[b][t][a] = r[b][t][a] / c
            for s in range(t + 1):
                dot = sum(q[b][t][a] * key(b, s, a) for a in range(A))
                for d in range(D):
                    f[b][t][d] += lam ** (t - s) * dot * v[b][s][d]
    return torch.tensor(q, dtype=torch.float64), torch.tensor(f, dtype=torch.float64)


def _recurrent(r, v, lam, w):
    """Token-by-token U/c recursion with the prior folded in (model.py:107-109)."""
    B, T, A = r.shape
    U = torch.zeros(B, v.shape[-1], A, dtype=torch.float64)  # mu = 0: U holds S only
    c = w.expand(B, A).clone()
    rp = torch.zeros(B, A, dtype=torch.float64)
    qs, fs = [], []
    for t in range(T):
        U = lam * U + v[:, t, :, None] * rp[:, None, :]
        c = lam * c + (1 - lam) * w + rp
        q = r[:, t] / c
        qs.append(q)
        fs.append((U @ q[:, :, None]).squeeze(-1))
        rp = r[:, t]
    return torch.stack(qs, 1), torch.stack(fs, 1)


def test_dense_matches_bruteforce():
    r, v, g, w = _inputs(B=2, T=7, A=3, D=2)
    q, f = fm.dense_fast_memory(r, v, g.exp(), w)
    qb, fb = _brute(r, v, g.exp(), w)
    assert (q - qb).abs().max() < 1e-12
    assert (f - fb).abs().max() < 1e-12


@pytest.mark.parametrize("mistake", ["no_shift", "reversed_decay", "no_prior", "transposed_scores"])
def test_bruteforce_detects_planted_mistakes(mistake):
    """A mistake planted in a copy of the dense form is caught by the brute force."""
    r, v, g, w = _inputs(B=1, T=6, A=3, D=2)
    lam = g.exp()
    T = r.shape[1]
    k = r if mistake == "no_shift" else fm.shift_keys(r)
    M = fm.decay_mask(T, lam)
    if mistake == "reversed_decay":
        M = M.transpose(0, 1)
    c = (0.0 if mistake == "no_prior" else w) + M @ k
    q = r / (c + (1.0 if mistake == "no_prior" else 0.0))
    S = q @ k.transpose(1, 2)
    if mistake == "transposed_scores":
        S = S.transpose(1, 2)
    f = (S * M) @ v
    qb, fb = _brute(r, v, lam, w)
    assert max((q - qb).abs().max().item(), (f - fb).abs().max().item()) > 1e-6


def test_recurrent_form_matches_dense():
    r, v, g, w = _inputs(B=3, T=20, A=6, D=4)
    q, f = fm.dense_fast_memory(r, v, g.exp(), w)
    qr, fr = _recurrent(r, v, g.exp(), w)
    assert (q - qr).abs().max() < 1e-12
    assert (f - fr).abs().max() < 1e-12


@pytest.mark.parametrize("T", [1, 2, 37])
def test_state_reads_out_the_last_position(T):
    """fast_{T-1} = S_{T-1} q_{T-1} and q_{T-1} = r_{T-1} / c_{T-1}, against the dense form."""
    r, v, g, w = _inputs(B=2, T=T, A=6, D=4, lam=0.7)
    q, f = fm.dense_fast_memory(r, v, g.exp(), w)
    S, c = fm.fast_memory_state(r, v, g.exp(), w)
    assert (torch.einsum("bda,ba->bd", S, q[:, -1]) - f[:, -1]).abs().max() < 1e-12
    assert (r[:, -1] / c - q[:, -1]).abs().max() < 1e-12


def test_state_matches_block_decode_state():
    """The state of one block after T calls of block_step (its U minus the prior
    mu w, and its c) from that block's own addresses and values."""
    p = fm.tiny_params(seed=3, n_layers=1)
    pre = "layers.0."
    B, T = 2, 23
    x = torch.randn(B, T, p[pre + "norm.weight"].shape[0], generator=torch.Generator().manual_seed(5),
                    dtype=torch.float64)
    st = fm.init_state(p, pre, B)
    rs, vs = [], []
    for t in range(T):
        h = fm.rmsnorm(x[:, t], p[pre + "norm.weight"], 1e-5)
        win = torch.cat([st["buf"], h[:, :, None]], dim=-1)
        u = (win * p[pre + "conv.weight"][:, 0, :]).sum(-1)
        rs.append(fm.address(torch.nn.functional.linear(u, p[pre + "key.weight"], p[pre + "key.bias"]),
                             p[pre + "log_eps"]))
        vs.append(torch.nn.functional.linear(h, p[pre + "val.weight"]))
        fm.block_step(p, pre, x[:, t], st)
    lam = torch.exp(fm.decay_log(p[pre + "log_rate"]))
    w = fm.prior_mass(p[pre + "log_w"])
    S, c = fm.fast_memory_state(torch.stack(rs, 1), torch.stack(vs, 1), lam, w)
    assert (S - (st["U"] - p[pre + "mu.weight"] * w)).abs().max() < 1e-12
    assert (c - st["c"]).abs().max() < 1e-12


@pytest.mark.parametrize("chunk", [1, 7, 16, 64])
def test_chunked_equals_dense(chunk):
    r, v, g, w = _inputs(B=2, T=150, A=9, D=5)
    q, f = fm.fast_memory(r, v, g, w, "dense")
    qc, fc = fm.fast_memory(r, v, g, w, "chunked", chunk)
    assert (q - qc).abs().max() < TOL
    assert (f - fc).abs().max() < TOL


def test_la_dense_and_role_table():
    """la_dense(q, k, v) is fast, and the three backward products of the role
    table (docs/kernel.md:22-27) are the autograd gradients of it."""
    r, v, g, w = _inputs(B=2, T=30, A=6, D=4)
    lam = g.exp()
    q, f = fm.dense_fast_memory(r, v, lam, w)
    k = fm.shift_keys(r)
    assert (fm.la_dense(q, k, v, lam) - f).abs().max() < 1e-13
    do = torch.randn(f.shape, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    q_, k_, v_ = (x.clone().requires_grad_(True) for x in (q, k, v))
    (fm.la_dense(q_, k_, v_, lam) * do).sum().backward()
    assert (fm.la_dense(do, v, k, lam) - q_.grad).abs().max() < 1e-12
    assert (fm.la_dense(v, do, q, lam, reverse=True) - k_.grad).abs().max() < 1e-12
    assert (fm.la_dense(k, q, do, lam, reverse=True) - v_.grad).abs().max() < 1e-12


def test_special_case_lam_to_zero():
    """lam -> 0: c_t = w + k_t and fast_t = (q_t . k_t) v_t."""
    r, v, _, w = _inputs(T=9)
    g = torch.tensor(-60.0, dtype=torch.float64)
    q, f = fm.fast_memory(r, v, g, w, "chunked", 4)
    k = fm.shift_keys(r)
    assert (q - r / (w + k)).abs().max() < 1e-14
    assert (f - (q * k).sum(-1, keepdim=True) * v).abs().max() < 1e-14


def test_special_case_lam_one():
    """lam = 1: prefix sums."""
    r, v, _, w = _inputs(T=13)
    g = torch.tensor(0.0, dtype=torch.float64)
    q, f = fm.fast_memory(r, v, g, w, "chunked", 5)
    k = fm.shift_keys(r)
    qe = r / (w + k.cumsum(1))
    fe = torch.stack([(qe[:, t:t + 1] @ k[:, :t + 1].transpose(1, 2)) @ v[:, :t + 1] for t in range(13)], 1)[:, :, 0]
    assert (q - qe).abs().max() < 1e-13
    assert (f - fe).abs().max() < 1e-13


def test_special_case_single_step_and_zero_rows():
    r, v, g, w = _inputs(T=1)
    q, f = fm.fast_memory(r, v, g, w)
    assert (q - r / w).abs().max() < 1e-15 and f.abs().max() == 0
    r, v, g, w = _inputs(T=10)
    r[:, 4] = 0
    q, f = fm.fast_memory(r, v, g, w)
    assert q[:, 4].abs().max() == 0 and f[:, 4].abs().max() == 0


def test_address_invariants():
    g = torch.Generator().manual_seed(3)
    pre = torch.randn(4, 7, 50, generator=g, dtype=torch.float64)
    r = fm.address(pre, torch.tensor(0.0, dtype=torch.float64))
    assert (r >= 0).all() and (r[pre <= 0] == 0).all()
    assert (r.sum(-1) < 1).all()
    z = pre.clamp(min=0) ** 2
    assert (r.sum(-1) - z.sum(-1) / (1 + z.sum(-1))).abs().max() < 1e-14
    r_lo = fm.address(pre, torch.tensor(-10.0, dtype=torch.float64))   # eps = e^-10
    assert (r_lo.sum(-1) - 1).abs().max() < 1e-3
    assert torch.allclose(fm.address(pre, torch.tensor(-30.0, dtype=torch.float64)), r_lo)  # clamp


def test_gradcheck_fast_memory():
    r, v, g, w = _inputs(B=1, T=7, A=3, D=2)
    args = tuple(x.clone().requires_grad_(True) for x in (r, v, g, w))
    assert torch.autograd.gradcheck(lambda *a: fm.fast_memory(*a, "chunked", 3), args)


def test_gradcheck_address():
    g = torch.Generator().manual_seed(5)
    pre = torch.randn(3, 6, generator=g, dtype=torch.float64).requires_grad_(True)
    le = torch.tensor(0.3, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(fm.address, (pre, le))


def test_dg_identity_matches_autograd():
    """The reference's positional form of d/dg (kernel.py:173-175) equals autograd."""
    r, v, g, w = _inputs(B=2, T=40, A=6, D=4)
    gen = torch.Generator().manual_seed(9)
    dq = torch.randn(r.shape, generator=gen, dtype=torch.float64)
    df = torch.randn(v.shape, generator=gen, dtype=torch.float64)
    _, _, dg, _ = fm.fast_memory_grads(r, v, g, w, dq, df, "dense")
    dg_id, _ = fm.dg_identity(r, v, g, w, dq, df)
    assert abs(dg.item() - dg_id.item()) < 1e-10 * max(1.0, abs(dg.item()))


def test_dg_bf16_floor_without_rounding_is_the_exact_dg():
    """dg_bf16_floor's positional identity (tau = (T-1)/2, the kernel's) with
    float64 operands equals autograd's dg; rounding only its operands then
    moves it by the bf16 floor the GPU dg check allows."""
    r, v, g, w = _inputs(B=2, T=70, A=6, D=4)
    gen = torch.Generator().manual_seed(11)
    dq = torch.randn(r.shape, generator=gen, dtype=torch.float64)
    df = torch.randn(v.shape, generator=gen, dtype=torch.float64)
    _, _, dg, _ = fm.fast_memory_grads(r, v, g, w, dq, df, "dense")
    exact = fm.dg_bf16_floor(r, v, g, w, dq, df, round_bf16=False)
    assert abs(dg.item() - exact.item()) < 1e-10 * max(1.0, abs(dg.item()))
    rounded = fm.dg_bf16_floor(r, v, g, w, dq, df)
    assert 0 < abs(rounded.item() - dg.item()) < 0.1 * abs(dg.item())


def test_pair_form_without_rounding_is_autograd():
    """pair_form_grads' closed-form gradients (summed over pairs for the decay)
    equal float64 autograd of the dense form, with and without dq_out, and
    pair_form's autograd wrapper returns the same."""
    r, v, g, w = _inputs(B=2, T=70, A=6, D=4)
    gen = torch.Generator().manual_seed(12)
    dq = torch.randn(r.shape, generator=gen, dtype=torch.float64)
    df = torch.randn(v.shape, generator=gen, dtype=torch.float64)
    for dq_out in (dq, None):
        q, fast, dr, dv, dg, dw = fm.pair_form_grads(r, v, g, w, dq_out, df, roundings=())
        qe, fe = fm.fast_memory(r, v, g, w, "dense")
        ref = fm.fast_memory_grads(r, v, g, w, dq_out, df, "dense")
        for got, exp in zip((q, fast, dr, dv, dg, dw), (qe, fe) + tuple(ref)):
            assert (got - exp).abs().max() < 1e-12 * max(1.0, exp.abs().max().item())
    leaves = [t.clone().requires_grad_() for t in (r, v, g, w)]
    q, fast = fm.pair_form(*leaves, roundings=())
    ((q * dq).sum() + (fast * df).sum()).backward()
    for t, exp in zip(leaves, fm.fast_memory_grads(r, v, g, w, dq, df, "dense")):
        assert (t.grad - exp).abs().max() < 1e-12 * max(1.0, exp.abs().max().item())


@pytest.mark.parametrize("rounding,moves,keeps", [
    ("qk", {"fast", "dv", "dg"}, {"q", "dr", "dw"}),   # P, hence fast, dv and the pair sum
    ("P", {"fast", "dv", "dg"}, {"q", "dr", "dw"}),
    ("v", {"fast", "dr", "dg", "dw"}, {"q", "dv"}),
    ("dfast", {"dr", "dv", "dg", "dw"}, {"q", "fast"}),
    ("dS", {"dr", "dg", "dw"}, {"q", "fast", "dv"}),
    ("qk_bwd", {"dr", "dg", "dw"}, {"q", "fast", "dv"}),
])
def test_each_pair_rounding_moves_only_what_reads_it(rounding, moves, keeps):
    """A planted bf16 rounding of one operand changes exactly the outputs that
    read that operand (a rounding applied at the wrong place fails this)."""
    r, v, g, w = _inputs(B=2, T=70, A=6, D=4)
    gen = torch.Generator().manual_seed(13)
    dq = torch.randn(r.shape, generator=gen, dtype=torch.float64)
    df = torch.randn(v.shape, generator=gen, dtype=torch.float64)
    names = ("q", "fast", "dr", "dv", "dg", "dw")
    exact = dict(zip(names, fm.pair_form_grads(r, v, g, w, dq, df, roundings=())))
    got = dict(zip(names, fm.pair_form_grads(r, v, g, w, dq, df, roundings=(rounding,))))
    for n in moves:
        assert (got[n] - exact[n]).abs().max() > 0, n
    for n in keeps:
        assert torch.equal(got[n], exact[n]), n


# ----- model level (test_all.py:100-137)

def _tokens(B=3, T=40, V=97, seed=0):
    return torch.randint(0, V, (B, T), generator=torch.Generator().manual_seed(seed))


def test_model_chunked_equals_dense():
    p = fm.tiny_params()
    x = _tokens()
    a, _ = fm.lm_forward(p, x, form="chunked", chunk=7)
    b, _ = fm.lm_forward(p, x, form="dense")
    assert (a - b).abs().max() < TOL


def test_parallel_equals_recurrent():
    p = fm.tiny_params()
    x = _tokens()
    a, _ = fm.lm_forward(p, x, form="chunked", chunk=16)
    assert (a - fm.forward_recurrent(p, x)).abs().max() < TOL


def test_causality():
    p = fm.tiny_params()
    x = _tokens()
    x2 = x.clone()
    x2[:, 25:] = _tokens(3, 15, seed=1)
    a, _ = fm.lm_forward(p, x, form="chunked", chunk=7)
    b, _ = fm.lm_forward(p, x2, form="chunked", chunk=7)
    assert (a[:, :25] - b[:, :25]).abs().max() < TOL


def test_gradients_finite():
    p = {k: v.clone().requires_grad_(True) for k, v in fm.tiny_params().items()}
    x = _tokens()
    _, loss = fm.lm_forward(p, x, x, form="chunked", chunk=7)
    loss.backward()
    for name, t in p.items():
        assert t.grad is not None and torch.isfinite(t.grad).all(), name


def _block_inputs(seed=3, B=2, T=70, dim=32, hidden=48):
    p = fm.tiny_params(seed, dim=dim, n_layers=1, hidden_dim=hidden)
    x = torch.randn(B, T, dim, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)
    return p, x


def _autocast_block_ref(p, x):
    """The block with its three products run by torch's CPU bf16 autocast
    (bf16 operands, fp32 accumulation, bf16 outputs) and the conv in fp32
    with a bf16 output, the rest in float64."""
    g = lambda n: p["layers.0." + n].float()
    bf = torch.bfloat16
    h = fm.rmsnorm(x.float(), g("norm.weight"), 1e-5)
    u = fm.causal_conv(h, g("conv.weight")).to(bf)
    with torch.autocast("cpu", dtype=bf):
        pre = F.linear(u, g("key.weight"))
        v = F.linear(h, g("val.weight"))
    assert pre.dtype == bf and v.dtype == bf
    r = fm.address(pre.double() + p["layers.0.key.bias"], p["layers.0.log_eps"])
    w = fm.prior_mass(p["layers.0.log_w"])
    q, fast = fm.fast_memory(r, v.double(), fm.decay_log(p["layers.0.log_rate"]), w)
    if fast.requires_grad:
        # the fused block hands the fast memory its upstream gradient in bf16
        fast.register_hook(lambda d: d.to(bf).to(d.dtype))
    with torch.autocast("cpu", dtype=bf):
        mu = F.linear((q * w).float(), g("mu.weight"))
    return x + mu.double() + fast


def test_block_autocast_emulation_matches_torch_autocast(monkeypatch):
    """block_forward(autocast=True) against the block whose products torch's
    own bf16 autocast computes: 30x closer to it than the exact block is
    (what remains is mostly the mu output, rounded by autocast, kept fp32
    by the fused block).
    A rounding left out (planted here: the value weight kept exact) moves the
    emulation away from torch's result by far more than that."""
    p, x = _block_inputs()
    rel = lambda a, b: ((a - b).norm() / b.norm()).item()
    exact = fm.block_forward(p, "layers.0.", x)
    emu = fm.block_forward(p, "layers.0.", x, autocast=True)
    ref = _autocast_block_ref(p, x)
    assert rel(exact, ref) > 1e-4
    assert rel(emu, ref) < 0.03 * rel(exact, ref)
    keep = p["layers.0.val.weight"]
    rounding = fm.round_bf16
    monkeypatch.setattr(fm, "round_bf16", lambda t: t if t is keep else rounding(t))
    planted = fm.block_forward(p, "layers.0.", x, autocast=True)
    assert rel(planted, ref) > 10 * rel(emu, ref)


def _head_grads(p, x, block):
    gen = torch.Generator().manual_seed(5)
    head = torch.randn(11, x.shape[-1], generator=gen, dtype=torch.float64)
    target = torch.randint(0, 11, (x.shape[0] * x.shape[1],), generator=gen)
    pp = {k: v.clone().requires_grad_() for k, v in p.items()}
    xx = x.clone().requires_grad_()
    F.cross_entropy((block(pp, xx) @ head.t()).reshape(-1, 11), target).backward()
    return {"x": xx.grad, **{k: v.grad for k, v in pp.items() if v.grad is not None}}


def test_block_autocast_gradients_match_torch_autocast(monkeypatch):
    """The backward roundings of block_forward(autocast=True) against the same
    torch-autocast block, under a classifier loss. The scalar and bias
    gradients, which torch's autocast rounds nowhere else, come 30x closer to
    torch's than the exact block's; the weight and input gradients at least
    2x (torch also rounds the weight gradients and the products' input
    gradients to bf16, which the fused block keeps in fp32). Dropping the
    gradient roundings (planted: round_grad_bf16 as the identity) undoes the
    agreement of the decay gradient."""
    p, x = _block_inputs()
    rel = lambda a, b: ((a - b).norm() / b.norm()).item()
    ref = _head_grads(p, x, _autocast_block_ref)
    exact = _head_grads(p, x, lambda pp, xx: fm.block_forward(pp, "layers.0.", xx))
    emu = _head_grads(p, x, lambda pp, xx: fm.block_forward(pp, "layers.0.", xx, autocast=True))
    assert set(ref) == set(emu)
    for k in ref:
        tight = k.split(".")[-1] in ("bias", "log_eps", "log_rate", "log_w")
        assert rel(emu[k], ref[k]) < (1 / 30 if tight else 0.5) * rel(exact[k], ref[k]), k
    monkeypatch.setattr(fm, "round_grad_bf16", lambda t: t)
    planted = _head_grads(p, x, lambda pp, xx: fm.block_forward(pp, "layers.0.", xx, autocast=True))
    k = "layers.0.log_rate"
    assert rel(planted[k], ref[k]) > 10 * rel(emu[k], ref[k])


def test_round_grad_bf16_is_torch_cast_backward():
    """round_grad_bf16: the identity forward, and the backward of torch's own
    bf16 round trip x.to(bf16).to(float64) on the gradient."""
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(64, dtype=torch.float64, generator=gen).requires_grad_()
    d = torch.randn(64, dtype=torch.float64, generator=gen)
    y = fm.round_grad_bf16(x)
    assert torch.equal(y, x)
    (gx,) = torch.autograd.grad(y, x, d)
    x2 = x.detach().to(torch.bfloat16).requires_grad_()
    (g2,) = torch.autograd.grad(x2.to(torch.float64), x2, d)
    assert torch.equal(gx, g2.double()) and not torch.equal(gx, d)


def test_round_bf16_is_forward_only():
    """round_bf16 leaves bf16 values unchanged and passes the gradient
    through unrounded."""
    x = torch.randn(4, 8, dtype=torch.float64).to(torch.bfloat16).double()
    assert torch.equal(fm.round_bf16(x), x)
    y = torch.randn(4, 8, dtype=torch.float64, requires_grad=True)
    fm.round_bf16(y).sum().backward()
    assert torch.equal(y.grad, torch.ones_like(y))     # the rounding passes gradients unchanged


# ----- the reference's own C decoder

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "runc_decode.npz")


def _golden():
    z = np.load(GOLDEN)
    p = {k[len("param/"):]: torch.from_numpy(z[k]).double() for k in z.files if k.startswith("param/")}
    return p, torch.from_numpy(z["tokens"]), z["logits"]


def test_recurrent_matches_runc_golden():
    """forward_recurrent of the oracle against logits written by run.c itself."""
    p, tokens, logits = _golden()
    got = fm.forward_recurrent(p, tokens[None])[0].numpy()
    scale = np.abs(logits).max()
    assert np.abs(got - logits).max() < 1e-5 * scale


def test_parallel_matches_runc_golden():
    p, tokens, logits = _golden()
    got, _ = fm.lm_forward(p, tokens[None], form="chunked", chunk=64)
    assert np.abs(got[0].numpy() - logits).max() < 1e-5 * np.abs(logits).max()


@pytest.mark.skipif(not runc.available(), reason="oracle/_ref/librunc_ref.so not built")
def test_recurrent_matches_runc_live():
    """A fresh seeded model with an untied classifier, through run.c."""
    p = fm.tiny_params(seed=11, dim=16, n_layers=2, hidden_dim=20, vocab_size=41, dtype=torch.float32)
    p["output.weight"] = torch.randn(41, 16, generator=torch.Generator().manual_seed(2)) * 0.1
    tokens = _tokens(1, 30, 41, seed=4)[0]
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "m.bin")
        ulme.write_ulme_v1(p, path, max_seq_len=30)
        magic, version, cfg = ulme.read_header(path)
        assert (magic, version, cfg[-1]) == (ulme.MAGIC, 1, 0)
        ref = runc.RuncReference(path).logits(tokens.tolist())
    got = fm.forward_recurrent({k: v.double() for k, v in p.items()}, tokens[None])[0].numpy()
    assert np.abs(got - ref).max() < 1e-5 * np.abs(ref).max()
