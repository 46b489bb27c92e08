"""UnifiedBlock around the fast memory (needs an MI355X): the fused RMSNorm +
causal conv kernels against float64 autograd of the oracle's rmsnorm and
causal_conv, and one whole block (model.py:77-85) forward and backward against
the oracle's block_forward.

Tolerances: the norm/conv kernels compute in fp32 (1e-5, fp32 outputs); the
block's GEMMs and fast-memory products take bf16 (autocast) or fp32 operands
with fp32 accumulation, held to the reference's 1e-2 (test_all.py:166). Under
bf16 autocast the oracle rounds what autocast rounds around the block's GEMMs
(block_forward(autocast=True)), so the comparison measures the kernels, not
the operand precision the training configuration chooses.
Every case prints its name before touching the GPU.
"""
import random

import pytest
import torch

from helpers import rel, say, tiny_model
from oracle import fastmem as fm

pytestmark = pytest.mark.gpu

import ulm_native as nat  # noqa: E402
from ulm_native import call, ptr  # noqa: E402

NC_CASES = [
    # B, T, D, Kc
    (2, 37, 64, 4),       # the model's conv_size, ragged position tile
    (1, 5, 300, 4),       # T shorter than a tile, D not a multiple of 256
    (2, 200, 768, 4),     # 110M width
    (1, 3, 96, 1),        # a single tap: no halo
    (2, 70, 130, 8),      # the largest tap count
    (1, 33, 1024, 4),     # the widest channel-per-thread backward (16 waves)
    (1, 40, 2100, 4),     # wide rows: the backward's 8-position tile
]


def _nc_inputs(B, T, D, Kc, seed):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, D, generator=gen, dtype=torch.float64)
    nw = 1.0 + 0.3 * torch.randn(D, generator=gen, dtype=torch.float64)
    cw = 0.5 * torch.randn(D, 1, Kc, generator=gen, dtype=torch.float64)
    return x, nw, cw


@pytest.mark.parametrize("B,T,D,Kc", NC_CASES)
def test_norm_conv_fwd_matches_oracle(B, T, D, Kc):
    say(f"ulm_norm_conv_fwd B={B} T={T} D={D} Kc={Kc}")
    x, nw, cw = _nc_inputs(B, T, D, Kc, seed=T + D)
    xd, nwd, cwd = (t.float().cuda().contiguous() for t in (x, nw, cw.reshape(D, Kc)))
    h = torch.empty(B, T, D, device="cuda")
    u = torch.empty(B, T, D, device="cuda")
    hb = torch.empty(B, T, D, device="cuda", dtype=torch.bfloat16)
    ub = torch.empty(B, T, D, device="cuda", dtype=torch.bfloat16)
    rstd = torch.empty(B, T, device="cuda")
    s = nat.stream_of(xd)
    call("ulm_norm_conv_fwd", ptr(xd), nat.ULM_F32, ptr(nwd), ptr(cwd), Kc, 1e-5, ptr(h), nat.ULM_F32, ptr(u),
         nat.ULM_F32, ptr(rstd), B, T, D, s)
    call("ulm_norm_conv_fwd", ptr(xd), nat.ULM_F32, ptr(nwd), ptr(cwd), Kc, 1e-5, ptr(hb), nat.ULM_BF16, ptr(ub),
         nat.ULM_BF16, ptr(rstd), B, T, D, s)
    torch.cuda.synchronize()
    hr = fm.rmsnorm(x, nw, 1e-5)
    ur = fm.causal_conv(hr, cw)
    rr = torch.rsqrt(x.pow(2).mean(-1) + 1e-5)
    errs = {"h": rel(h, hr), "u": rel(u, ur), "rstd": rel(rstd, rr), "h16": rel(hb, hr), "u16": rel(ub, ur)}
    say(f"  rel errors {errs}")
    assert errs["h"] < 1e-6 and errs["u"] < 1e-6 and errs["rstd"] < 1e-6
    assert errs["h16"] < 1e-2 and errs["u16"] < 1e-2   # bf16 rounding of the outputs


@pytest.mark.parametrize("B,T,D,Kc", NC_CASES)
def test_norm_conv_bwd_matches_autograd(B, T, D, Kc):
    say(f"ulm_norm_conv_bwd B={B} T={T} D={D} Kc={Kc}")
    x, nw, cw = _nc_inputs(B, T, D, Kc, seed=3 * T + D)
    gen = torch.Generator().manual_seed(D)
    du, dhv, dres = (torch.randn(B, T, D, generator=gen, dtype=torch.float64) for _ in range(3))
    # float64 autograd of the oracle: L = <du, u> + <dhv, h>, dx gets dres on top
    xr, nwr, cwr = (t.clone().requires_grad_() for t in (x, nw, cw))
    hr = fm.rmsnorm(xr, nwr, 1e-5)
    ur = fm.causal_conv(hr, cwr)
    ((du * ur).sum() + (dhv * hr).sum()).backward()
    dx_ref = xr.grad + dres
    xd, nwd, cwd = (t.float().cuda().contiguous() for t in (x, nw, cw.reshape(D, Kc)))
    dud, dhvd, dresd = (t.float().cuda().contiguous() for t in (du, dhv, dres))
    s = nat.stream_of(xd)
    h = torch.empty(B, T, D, device="cuda")
    u = torch.empty(B, T, D, device="cuda")
    rstd = torch.empty(B, T, device="cuda")
    call("ulm_norm_conv_fwd", ptr(xd), nat.ULM_F32, ptr(nwd), ptr(cwd), Kc, 1e-5, ptr(h), nat.ULM_F32, ptr(u),
         nat.ULM_F32, ptr(rstd), B, T, D, s)
    dx = torch.empty(B, T, D, device="cuda")
    dnw = torch.empty(D, device="cuda")
    dcw = torch.empty(D, Kc, device="cuda")
    wsb = nat.lib().ulm_norm_conv_bwd_workspace_bytes(B, T, D, Kc)
    assert wsb > 0
    ws = torch.empty(wsb, device="cuda", dtype=torch.uint8)
    call("ulm_norm_conv_bwd", ptr(xd), nat.ULM_F32, ptr(rstd), ptr(nwd), ptr(cwd), Kc, ptr(dud), nat.ULM_F32,
         ptr(dhvd), nat.ULM_F32, ptr(dresd), ptr(dx), ptr(dnw), ptr(dcw), ptr(ws), wsb, B, T, D, s)
    # in place on the residual gradient, and without the value-GEMM term
    dx2 = dresd.clone()
    dnw2 = torch.empty(D, device="cuda")
    dcw2 = torch.empty(D, Kc, device="cuda")
    call("ulm_norm_conv_bwd", ptr(xd), nat.ULM_F32, ptr(rstd), ptr(nwd), ptr(cwd), Kc, ptr(dud), nat.ULM_F32,
         None, nat.ULM_F32, ptr(dx2), ptr(dx2), ptr(dnw2), ptr(dcw2), ptr(ws), wsb, B, T, D, s)
    torch.cuda.synchronize()
    errs = {"dx": rel(dx, dx_ref), "dnorm_w": rel(dnw, nwr.grad), "dconv_w": rel(dcw, cwr.grad.reshape(D, Kc))}
    say(f"  rel errors {errs}")
    assert max(errs.values()) < 1e-5, errs
    # the second call: L = <du, u> only
    xr2, nwr2, cwr2 = (t.clone().requires_grad_() for t in (x, nw, cw))
    (du * fm.causal_conv(fm.rmsnorm(xr2, nwr2, 1e-5), cwr2)).sum().backward()
    errs2 = {"dx": rel(dx2, xr2.grad + dres), "dnorm_w": rel(dnw2, nwr2.grad),
             "dconv_w": rel(dcw2, cwr2.grad.reshape(D, Kc))}
    say(f"  in place, no dhv: rel errors {errs2}")
    assert max(errs2.values()) < 1e-5, errs2


def _random_nc_cases(n, seed):
    """Seeded (B, T, D, Kc) draws: single and ragged position tiles, widths
    from one channel to 2100, every tap count up to the largest."""
    rng = random.Random(seed)
    return [(rng.choice([1, 2, 3]), rng.choice([1, 2, 5, 17, 64, 100, 257]),
             rng.choice([1, 5, 64, 100, 288, 768, 1024, 2100]), rng.choice([1, 2, 3, 4, 8])) for _ in range(n)]


@pytest.mark.parametrize("B,T,D,Kc", _random_nc_cases(10, 13))
def test_norm_conv_random_shapes(B, T, D, Kc):
    """The forward and backward checks above over seeded random draws."""
    test_norm_conv_fwd_matches_oracle(B, T, D, Kc)
    test_norm_conv_bwd_matches_autograd(B, T, D, Kc)


BLOCK_CASES = [
    # B, T, D, A, autocast
    (2, 200, 64, 140, False),     # the reference test's shape (test_all.py:140-154)
    (2, 200, 64, 140, True),
    (1, 70, 96, 320, False),      # A, D multiples of 32: the K-group products
    (2, 256, 128, 256, True),
    (1, 512, 768, 3072, True),    # 110M block shape
    (1, 1024, 768, 3072, False),  # 110M block shape, a whole 1024-position row, fp32
    (1, 1024, 512, 2048, True),   # 42M block shape, one row of 1024 positions
    (1, 1024, 512, 2048, False),
    (3, 1, 64, 64, False),        # a single position
    # D not a multiple of 32 (zero-padded features in the block-pair products), ragged chunk
    (2, 130, 100, 1600, False),
    (2, 130, 100, 1600, True),
    (2, 256, 288, 712, True),     # the reference's 15M model widths (docs/models.md:11), A off the 32 grid
    # A off the multiples of 4: the dr accumulation's element-wise path
    (2, 150, 64, 70, False),
    (2, 150, 64, 70, True),
]


def _head_loss(out, head, targets):
    """Cross-entropy of a fixed classifier over the block output: the upstream
    gradient has the structure of a training step (UnifiedLM.forward,
    model.py:149-162) rather than white noise, whose random signs the scalar
    gradients (log_eps, log_rate) would sum with heavy cancellation."""
    return torch.nn.functional.cross_entropy((out @ head.t()).reshape(-1, head.shape[0]), targets.reshape(-1))


def _block_run(B, T, D, A, autocast):
    """One block draw (seeded by T, A) forward and backward on the GPU under
    the head loss: (block, x, x on the GPU with its gradient, out, head, targets)."""
    say(f"UnifiedBlock fwd+bwd B={B} T={T} D={D} A={A} autocast={autocast}")
    model = tiny_model(seed=T + A, dim=D, hidden_dim=A, n_layers=1, vocab_size=97, max_seq_len=max(T, 64))
    blk = model.layers[0]
    gen = torch.Generator().manual_seed(A)
    with torch.no_grad():
        blk.norm.weight.copy_(1.0 + 0.2 * torch.randn(D, generator=gen))
    blk = blk.cuda().train()
    x = torch.randn(B, T, D, generator=gen)
    head = torch.randn(97, D, generator=gen, dtype=torch.float64) / D ** 0.5
    targets = torch.randint(0, 97, (B, T), generator=gen)
    xg = x.cuda().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        out = blk(xg)
    _head_loss(out, head.float().cuda(), targets.cuda()).backward()
    torch.cuda.synchronize()
    return blk, x, xg, out, head, targets


def _oracle_block(blk, x, head, targets, autocast, fast_memory=None):
    """The oracle's block in float64 with blk's parameters (its fast memory
    replaced by fast_memory when given): (out, dx, {name: gradient})."""
    p = {n: t.detach().double().cpu().requires_grad_() for n, t in blk.named_parameters()}
    xr = x.double().requires_grad_()
    orig = fm.fast_memory
    if fast_memory is not None:
        fm.fast_memory = fast_memory
    try:
        ref = fm.block_forward(p, "", xr, norm_eps=blk.norm.eps, autocast=autocast)
    finally:
        fm.fast_memory = orig
    _head_loss(ref, head, targets).backward()
    return ref.detach(), xr.grad, {n: t.grad for n, t in p.items()}


def _pair_floor(r, v, g, w, form="chunked", chunk=64):
    return fm.pair_form(r, v, g, w)


def _block_errors(B, T, D, A, autocast):
    """Relative errors of the block's output and every gradient against float64,
    with the run and the exact gradients for a closer look."""
    blk, x, xg, out, head, targets = _block_run(B, T, D, A, autocast)
    ref, dx, grads = _oracle_block(blk, x, head, targets, autocast)
    errs = {"out": rel(out, ref), "dx": rel(xg.grad, dx)}
    # With one position the memory holds nothing (k_0 = 0, so fast = 0 and
    # w q = r): the gradients of log_w, log_rate and the value weight are
    # exactly zero, a relative error is undefined, and ours are held to 1e-6 of
    # the input gradient's norm instead (fp32 rounding of terms that cancel).
    zero = {"log_w", "log_rate", "val.weight"} if T == 1 else set()
    for n, t in blk.named_parameters():
        errs[n] = (t.grad.norm() / xg.grad.norm()).item() if n in zero else rel(t.grad, grads[n])
        if n in zero:
            assert grads[n].abs().max().item() < 1e-12, (n, grads[n])
    say(f"  worst {max(errs.values()):.3e}: {errs}")
    return errs, (blk, x, head, targets), grads


@pytest.mark.parametrize("B,T,D,A,autocast", BLOCK_CASES)
def test_block_matches_oracle(B, T, D, A, autocast):
    errs = _block_errors(B, T, D, A, autocast)[0]
    # test_all.py:157-166 holds loss and every gradient to 1e-2
    assert all(e < 1e-2 for e in errs.values()), errs


_XFAIL_PAIR = "log_rate gradient {} of float64 on the block-pair form: the bf16 operand floor of this draw exceeds 1e-2"


@pytest.mark.parametrize("autocast,path", [
    pytest.param(False, "pair", marks=pytest.mark.xfail(strict=True, reason=_XFAIL_PAIR.format("2.1e-2"))),
    pytest.param(True, "pair", marks=pytest.mark.xfail(strict=True, reason=_XFAIL_PAIR.format("5.6e-2"))),
    (True, "generic"),
])
def test_ill_conditioned_block_draw(autocast, path, monkeypatch):
    """The D=40, A=70, T=150 draw, whose decay gradient bf16 operands alone move
    past 1e-2 (tests/test_conditioning.py), held to the parity bound. The
    block-pair form (the library's choice at this shape) misses it by as much
    as its roundings predict (test_ill_conditioned_draw_matches_its_rounding_floor):
    kept as strict expected failures. Under autocast the generic kernel, whose
    rounding profile differs, meets it."""
    monkeypatch.setenv("ULM_FM_PATH", path)
    test_block_matches_oracle(2, 150, 40, 70, autocast)


@pytest.mark.parametrize("autocast", [False, True])
def test_ill_conditioned_draw_matches_its_rounding_floor(autocast, monkeypatch):
    """The D=40, A=70, T=150 draw on the block-pair form: every gradient but log_rate within 1e-2 of
    float64, and log_rate as far from it as the block-pair products' own bf16
    roundings put it in otherwise exact arithmetic (oracle.fastmem.pair_form,
    within 15% of that distance, and on the same side of the exact value): the
    kernel's fp32 accumulations add nothing that matters beyond its operands'
    roundings."""
    B, T, D, A = 2, 150, 40, 70
    monkeypatch.setenv("ULM_FM_PATH", "pair")
    say("ill-conditioned block draw on the block-pair form")
    blk, x, _, _, head, targets = _block_run(B, T, D, A, autocast)
    exact = _oracle_block(blk, x, head, targets, autocast)[2]
    floor = _oracle_block(blk, x, head, targets, autocast, _pair_floor)[2]
    errs = {n: rel(t.grad, exact[n]) for n, t in blk.named_parameters()}
    want = rel(floor["log_rate"], exact["log_rate"])
    say(f"  kernel log_rate {errs['log_rate']:.3e}, bf16 rounding floor {want:.3e}; others {errs}")
    assert all(e < 1e-2 for n, e in errs.items() if n != "log_rate"), errs
    assert abs(errs["log_rate"] - want) < 0.15 * want
    got_dev = (blk.log_rate.grad.double().cpu() - exact["log_rate"]).item()
    want_dev = (floor["log_rate"] - exact["log_rate"]).item()
    assert got_dev * want_dev > 0


def _random_block_draws(n, seed):
    """n seeded (B, T, D, A, autocast) draws: single, ragged and whole-tile
    position counts, widths on and off the 32 grid, the reference's 15M widths."""
    rng = random.Random(seed)
    draws = []
    for _ in range(n):
        B = rng.choice([1, 2, 3])
        T = rng.choice([1, 33, 64, 100, 128, 200, 256, 300, 511])
        D = rng.choice([32, 48, 64, 96, 128, 160, 288])
        A = rng.choice([64, 70, 128, 140, 256, 320, 712, 1024])
        draws.append((B, T, D, A, rng.choice([False, True])))
    return draws


# Two draws that the library runs on the chunked state form (T <= 100 at
# these widths), each with one scalar gradient past 1e-2 of float64. The
# chunked form rounds its intra-chunk products at points of its own, which
# oracle.fastmem.pair_form does not restate, so no exact floor pins them; in
# float64, one class of bf16 operand roundings alone moves the same gradient
# as far (measured with pair_form's roundings one at a time, and with the
# decay gradient's positional identity of the chunked kernels over bf16 v,
# dfast, q, k and intra-chunk scores).
_CHUNKED_FLOOR = {
    (3, 100, 32, 256, False): "log_eps 1.07e-2 of float64 on the chunked form; rounding v alone to bf16 "
                              "moves it 1.42e-2, the intra-chunk dfast.v products alone 1.22e-2",
    (2, 64, 64, 320, True): "log_rate 1.69e-2 of float64 on the chunked form; the positional identity over "
                            "bf16 operands and intra-chunk products moves it 1.36e-2 (the generic kernel: 1.38e-2)",
}
RANDOM_BLOCK_DRAWS = [
    pytest.param(*d, marks=pytest.mark.xfail(strict=True, reason=_CHUNKED_FLOOR[d])) if d in _CHUNKED_FLOOR else d
    for d in _random_block_draws(40, 3)
]
SCALAR_GRADS = {"log_rate", "log_eps", "log_w"}
PATH_PAIR = 2


@pytest.mark.parametrize("B,T,D,A,autocast", RANDOM_BLOCK_DRAWS)
def test_block_random_draw(B, T, D, A, autocast):
    """Seeded block draws: output, input gradient and every weight gradient
    within 1e-2 of float64 (test_all.py:157-166). The three scalar gradients
    (log_rate, log_eps, log_w) each sum B T A terms that cancel, so bf16
    operands can move them past 1e-2 by themselves: one that lands past it on
    the block-pair form must sit where that form's own bf16 roundings put it
    in otherwise exact arithmetic (oracle.fastmem.pair_form: within 15% of
    that distance, and in the same direction)."""
    errs, (blk, x, head, targets), exact = _block_errors(B, T, D, A, autocast)
    over = {n for n, e in errs.items() if e >= 1e-2}
    assert over <= SCALAR_GRADS, errs
    if not over:
        return
    path = nat.lib().ulm_fm_path(B, T, A, D)
    assert path == PATH_PAIR, f"{sorted(over)} past 1e-2 on path {path}: {errs}"
    floor = _oracle_block(blk, x, head, targets, autocast, _pair_floor)[2]
    grads = dict(blk.named_parameters())
    for n in sorted(over):
        got = (grads[n].grad.double().cpu() - exact[n]).flatten()
        want = (floor[n] - exact[n]).flatten()
        cos = (got @ want / (got.norm() * want.norm())).item()
        say(f"  {n}: kernel {errs[n]:.3e}, bf16 rounding floor {rel(floor[n], exact[n]):.3e}, cos {cos:+.3f}")
        assert abs(got.norm() - want.norm()) < 0.15 * want.norm(), n
        assert cos > 0.9, n


WGRAD_CASES = [
    # K, N1, N2
    (1000, 200, 136),      # ragged K chunk and partial tiles on both sides
    (64, 8, 16),           # one k-step, tiny tiles
    (4096, 768, 768),      # value projection shape
    (16384, 768, 3072),    # mu weight gradient at the 110M shape
    (16384, 3072, 768),    # key weight gradient at the 110M shape
]


def test_block_params_match_autograd():
    """g = -exp(log_rate), w = exp(clamp(log_w, -7, 12)) and their chain rule
    (model.py:75, 84) against fp32 torch autograd, with log_w below, above and
    exactly at both clamp bounds (where torch's clamp passes the gradient)."""
    import kernel
    say("ulm_block_params / ulm_block_params_bwd A=300")
    A = 300
    gen = torch.Generator().manual_seed(7)
    lw = torch.randn(A, generator=gen) * 6.0
    lw[:6] = torch.tensor([-7.0, 12.0, -7.5, 12.5, -30.0, 30.0])
    lr = torch.tensor([-2.7])
    dg, dw = torch.randn(1, generator=gen), torch.randn(A, generator=gen)
    lrr, lwr = lr.clone().requires_grad_(), lw.clone().requires_grad_()
    g_ref, w_ref = -lrr.exp(), lwr.clamp(kernel.LOG_W_MIN, kernel.LOG_W_MAX).exp()
    ((g_ref * dg).sum() + (w_ref * dw).sum()).backward()
    lrd, lwd, dgd, dwd = (t.cuda() for t in (lr, lw, dg, dw))
    g, w = torch.empty(1, device="cuda"), torch.empty(A, device="cuda")
    dlr, dlw = torch.empty(1, device="cuda"), torch.empty(A, device="cuda")
    s = nat.stream_of(lrd)
    call("ulm_block_params", ptr(lrd), ptr(lwd), kernel.LOG_W_MIN, kernel.LOG_W_MAX, A, ptr(g), ptr(w), s)
    call("ulm_block_params_bwd", ptr(lrd), ptr(lwd), kernel.LOG_W_MIN, kernel.LOG_W_MAX, ptr(dgd), ptr(dwd), A,
         ptr(dlr), ptr(dlw), s)
    torch.cuda.synchronize()
    for got, ref in ((g, g_ref), (w, w_ref), (dlr, lrr.grad), (dlw, lwr.grad)):
        assert torch.allclose(got.cpu(), ref.detach(), rtol=1e-6, atol=0), (got, ref)
    assert (dlw.cpu()[2:6] == 0).all() and (dlw.cpu()[:2] != 0).all()


@pytest.mark.parametrize("K,N1,N2", WGRAD_CASES)
def test_wgrad_matches_fp32_product(K, N1, N2):
    """C = A^T B against the fp32 product of the same bf16 operands (float64
    on the CPU for the small cases)."""
    say(f"ulm_wgrad K={K} N1={N1} N2={N2}")
    gen = torch.Generator().manual_seed(K + N1)
    a = torch.randn(K, N1, generator=gen).to(torch.bfloat16)
    b = torch.randn(K, N2, generator=gen).to(torch.bfloat16)
    ad, bd = a.cuda(), b.cuda()
    c = torch.empty(N1, N2, device="cuda")
    wsb = nat.lib().ulm_wgrad_workspace_bytes(K, N1, N2)
    ws = torch.empty(max(wsb, 1), device="cuda", dtype=torch.uint8)
    call("ulm_wgrad", ptr(ad), ptr(bd), ptr(c), K, N1, N2, ptr(ws), wsb, nat.stream_of(ad))
    torch.cuda.synchronize()
    if K * N1 * N2 <= 1 << 28:
        ref = a.double().t() @ b.double()
    else:
        ref = (ad.double().t() @ bd.double()).cpu()
    err = rel(c, ref)
    say(f"  rel error {err:.2e}")
    assert err < 1e-5


def _random_wgrad_cases(n, seed):
    """Seeded (K, N1, N2) draws: contractions from one row to ragged
    thousands, widths multiples of 8 from 8 to 3200."""
    rng = random.Random(seed)
    return [(rng.choice([1, 7, 64, 100, 1000, 4096, 5000]), 8 * rng.randint(1, 400), 8 * rng.randint(1, 400))
            for _ in range(n)]


@pytest.mark.parametrize("K,N1,N2", _random_wgrad_cases(10, 17))
def test_wgrad_random_shapes(K, N1, N2):
    """The check of test_wgrad_matches_fp32_product over seeded random draws."""
    test_wgrad_matches_fp32_product(K, N1, N2)


@pytest.mark.parametrize("autocast", [False, True])
def test_fused_model_is_causal_and_finite(autocast):
    """test_all.py:119-137 on the native path: perturbing tokens from position
    25 on leaves the logits before 25 unchanged (every reduction on the path
    is within a row or over earlier positions, in a fixed order), and a
    training step's gradients are finite."""
    say(f"fused UnifiedLM causality and finite gradients, autocast={autocast}")
    model = tiny_model(dim=64, n_layers=2, hidden_dim=128, vocab_size=97, max_seq_len=100).cuda().train()
    gen = torch.Generator().manual_seed(12)
    x = torch.randint(0, 97, (2, 90), generator=gen)
    x2 = x.clone()
    x2[:, 25:] = torch.randint(0, 97, (2, 65), generator=gen)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        a = model(x.cuda(), x.cuda()).float()     # with targets: the logits of every position
        b = model(x2.cuda(), x2.cuda()).float()
    diff = (a[:, :25] - b[:, :25]).abs().max().item()
    say(f"  max |logit change| before position 25: {diff}; after: {(a[:, 25:] - b[:, 25:]).abs().max().item():.3f}")
    assert diff == 0.0
    assert (a[:, 25:] - b[:, 25:]).abs().max().item() > 0
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        model(x.cuda(), x.cuda())
    model.last_loss.backward()
    for name, p in model.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), name


@pytest.mark.parametrize("path", ["chunked", "pair", "generic"])
def test_native_reductions_are_deterministic(path, monkeypatch):
    """The fast-memory operator (every output and gradient), the split-K
    weight gradient and the norm/conv weight gradients sum in a fixed order:
    repeated calls agree bit for bit, on every evaluation of the products and
    at the reference test's widths (A=140, D=64)."""
    import kernel
    from helpers import fm_inputs
    say(f"determinism of ulm_fm_bwd ({path}), ulm_wgrad, ulm_norm_conv_bwd")
    monkeypatch.setenv("ULM_FM_PATH", path)
    gen = torch.Generator(device="cuda").manual_seed(5)
    shapes = [(2, 256, 256, 128)] + ([(2, 200, 140, 64)] if path != "chunked" else [])
    for B, T, A, D in shapes:
        r, v, g, w = fm_inputs(B, T, A, D, seed=5, device="cuda")
        r, v, g, w = (t.float().requires_grad_() for t in (r, v, g, w))
        dq, df = torch.randn(B, T, A, device="cuda", generator=gen), torch.randn(B, T, D, device="cuda", generator=gen)
        grads = []
        for _ in range(2):
            q, fast = kernel.unified_memory(r, v, g, w)
            grads.append((q, fast) + torch.autograd.grad((q, fast), (r, v, g, w), (dq, df)))
        for a_, b_ in zip(*grads):
            assert torch.equal(a_, b_), (B, T, A, D)
    a = torch.randn(4096, 256, device="cuda", generator=gen).to(torch.bfloat16)
    b = torch.randn(4096, 512, device="cuda", generator=gen).to(torch.bfloat16)
    c1, c2 = kernel._wgrad(a, b), kernel._wgrad(a, b)
    assert torch.equal(c1, c2)
    B, T, D, Kc = 2, 300, 256, 4
    x = torch.randn(B, T, D, device="cuda", generator=gen)
    nw, cw = torch.ones(D, device="cuda"), torch.randn(D, Kc, device="cuda", generator=gen)
    du = torch.randn(B, T, D, device="cuda", generator=gen)
    h, u = torch.empty_like(x), torch.empty_like(x)
    rstd = torch.empty(B, T, device="cuda")
    s = nat.stream_of(x)
    call("ulm_norm_conv_fwd", ptr(x), nat.ULM_F32, ptr(nw), ptr(cw), Kc, 1e-5, ptr(h), nat.ULM_F32, ptr(u),
         nat.ULM_F32, ptr(rstd), B, T, D, s)
    wsb = nat.lib().ulm_norm_conv_bwd_workspace_bytes(B, T, D, Kc)
    ws = torch.empty(wsb, device="cuda", dtype=torch.uint8)
    outs = []
    for _ in range(2):
        dx, dnw, dcw = torch.empty_like(x), torch.empty(D, device="cuda"), torch.empty(D, Kc, device="cuda")
        call("ulm_norm_conv_bwd", ptr(x), nat.ULM_F32, ptr(rstd), ptr(nw), ptr(cw), Kc, ptr(du), nat.ULM_F32, None,
             nat.ULM_F32, None, ptr(dx), ptr(dnw), ptr(dcw), ptr(ws), wsb, B, T, D, s)
        outs.append((dx, dnw, dcw))
    for a_, b_ in zip(*outs):
        assert torch.equal(a_, b_)
