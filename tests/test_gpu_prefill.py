"""Prefill (needs an MI355X): the forward of the fast memory plus the decode
state after the last position, against the float64 oracle, in both of its
forms: the chunked state form, and the block-pair products with the state as
one product over positions (ulm_fm_prefill_path; ULM_FM_PATH forces one).

Tolerances: q and c are fp32 scans (1e-5); fast and the state S come from bf16
MFMA products with fp32 accumulation, the training path's 1e-2 (test_all.py:166).
Every case prints its name before touching the GPU.
"""
import random

import pytest
import torch

from helpers import fm_inputs, oracle_params, rel, say, tiny_model
from oracle import fastmem as fm

pytestmark = pytest.mark.gpu

import kernel  # noqa: E402
import ulm_native as nat  # noqa: E402

PREFILL_CASES = [
    # B, T, A, D, lam, dtype of v
    (2, 200, 96, 64, 0.93, torch.float32),      # ragged last chunk, a wave without keys
    (1, 64, 128, 32, 0.93, torch.bfloat16),     # one whole chunk, a half-empty value tile
    (2, 1, 64, 64, 0.93, torch.float32),        # a single position
    (2, 300, 64, 128, 0.5, torch.float32),      # lam^64 below 2^-40
    (1, 600, 1600, 64, 0.93, torch.bfloat16),   # 3 key groups; the state scale renormalises
    (1, 512, 3072, 768, None, torch.bfloat16),  # 110M block shape
    # widths off the 32 grid (zero-padded tiles): the reference test's and 15M model's widths, both ragged
    (2, 200, 140, 64, 0.93, torch.float32),
    (1, 300, 712, 288, None, torch.bfloat16),
    (2, 130, 100, 36, 0.93, torch.float32),
]


@pytest.mark.parametrize("path", ["chunked", "pair"])
@pytest.mark.parametrize("B,T,A,D,lam,vdt", PREFILL_CASES)
def test_fm_prefill_matches_oracle_state(B, T, A, D, lam, vdt, path, monkeypatch):
    monkeypatch.setenv("ULM_FM_PATH", path)
    assert nat.lib().ulm_fm_prefill_path(B, T, A, D) == {"chunked": 1, "pair": 2}[path]
    say(f"fm_prefill B={B} T={T} A={A} D={D} lam={lam} v={vdt}, {path} form")
    r, v, g, w = fm_inputs(B, T, A, D, seed=T + A, device="cpu", lam=lam)
    q, fast, S, c = kernel.fm_prefill(r.float().cuda(), v.to(vdt).cuda(), g.float().cuda(), w.float().cuda())
    torch.cuda.synchronize()
    vr = v.to(vdt).double()
    qr, fr = fm.fast_memory(r, vr, g, w, "chunked")
    Sr, cr = fm.fast_memory_state(r, vr, g.exp(), w)
    errs = {"q": rel(q, qr), "fast": rel(fast, fr), "S": rel(S, Sr), "c": rel(c, cr)}
    say(f"  rel errors {errs}")
    assert S.shape == (B, D, A) and c.shape == (B, A)
    assert errs["q"] < 1e-5 and errs["c"] < 1e-5
    assert errs["fast"] < 1e-2 and errs["S"] < 1e-2


def _random_prefill_cases(n, seed):
    """Seeded (B, T, A, D, lam, dtype of v) draws: ragged and whole chunks,
    widths on and off the 32 grid, lam from fast to slow decay."""
    rng = random.Random(seed)
    return [(rng.choice([1, 2, 3]), rng.choice([1, 5, 63, 64, 65, 129, 256, 300, 517]),
             rng.choice([32, 64, 100, 140, 256, 320, 712, 1024]), rng.choice([16, 32, 36, 64, 96, 160, 288]),
             rng.choice([0.5, 0.8, 0.93, 0.99, None]), rng.choice([torch.float32, torch.bfloat16]))
            for _ in range(n)]


@pytest.mark.parametrize("path", ["chunked", "pair"])
@pytest.mark.parametrize("B,T,A,D,lam,vdt", _random_prefill_cases(12, 7))
def test_fm_prefill_random_shapes(B, T, A, D, lam, vdt, path, monkeypatch):
    """The checks of test_fm_prefill_matches_oracle_state over seeded random draws."""
    test_fm_prefill_matches_oracle_state(B, T, A, D, lam, vdt, path, monkeypatch)


def _oracle_states(p, tokens, n_layers):
    """The oracle's per-block decode states after every position of tokens."""
    B, T = tokens.shape
    states = [fm.init_state(p, f"layers.{i}.", B) for i in range(n_layers)]
    for t in range(T):
        h = p["tok_embeddings.weight"][tokens[:, t]]
        for i in range(n_layers):
            h = fm.block_step(p, f"layers.{i}.", h, states[i])
    return states


def _prefill_then_step(dim, hidden, n_layers, B, T0, T, seed):
    """UnifiedLM.prefill of T0 positions, then steps to T, against the
    oracle's forward_recurrent (logits within 1e-2), and the states right
    after the prompt against the oracle's (S = U - mu w, c, r_prev, the conv
    window; 1e-2)."""
    kw = dict(dim=dim, n_layers=n_layers, hidden_dim=hidden, vocab_size=97, max_seq_len=max(T, 64))
    model = tiny_model(seed=seed, **kw).cuda()
    x = torch.randint(0, 97, (B, T), generator=torch.Generator().manual_seed(seed + 2))
    logits0, states = model.prefill(x[:, :T0].cuda())
    cont = [model.step(x[:, t].cuda(), states) for t in range(T0, T)]
    torch.cuda.synchronize()
    p = oracle_params(model)
    ref = fm.forward_recurrent(p, x)
    assert rel(logits0, ref[:, T0 - 1]) < 1e-2
    if cont:
        assert rel(torch.stack(cont, 1), ref[:, T0:]) < 1e-2
    model2 = tiny_model(seed=seed, **kw).cuda()
    _, st = model2.prefill(x[:, :T0].cuda())
    so = _oracle_states(p, x[:, :T0], n_layers)
    for i, (a, o) in enumerate(zip(st, so)):
        w = fm.prior_mass(p[f"layers.{i}.log_w"])
        errs = {"S": rel(a["S"], o["U"] - p[f"layers.{i}.mu.weight"] * w), "c": rel(a["c"], o["c"]),
                "r_prev": rel(a["r_prev"], o["r_prev"]), "buf": rel(a["buf"], o["buf"])}
        if T0 == 1:
            # one position: its key r_{-1} is zero, so the state holds nothing:
            # S is exactly 0 (the oracle's U - mu w is float64 rounding of it)
            assert a["S"].abs().max().item() == 0.0
            errs["S"] = 0.0
        say(f"  block {i} rel errors {errs}")
        assert max(errs.values()) < 1e-2, errs


@pytest.mark.parametrize("path", ["chunked", "pair"])
@pytest.mark.parametrize("dim,hidden", [(32, 64), (64, 140)])
def test_model_prefill_then_step_matches_recurrent(dim, hidden, path, monkeypatch):
    monkeypatch.setenv("ULM_FM_PATH", path)
    say(f"UnifiedLM.prefill of 50 positions, then 20 steps, vs the oracle's forward_recurrent, dim={dim} A={hidden}, "
        f"{path} form")
    _prefill_then_step(dim, hidden, 3, 3, 50, 70, 0)


def _random_model_cases(n, seed):
    """Seeded (dim, hidden, n_layers, B, T0, T, form) draws: prompts of one to
    a hundred positions, 0 to 33 steps after them (two write-backs of the
    deferred state), slot counts that take the deferred state and one
    (A % 4 != 0) that takes the per-position kernel."""
    rng = random.Random(seed)
    cases = []
    for _ in range(n):
        T0 = rng.choice([1, 7, 50, 64, 100])
        cases.append((rng.choice([16, 32, 48, 64, 96]), rng.choice([24, 64, 70, 100, 140, 256]), rng.choice([1, 2, 3]),
                      rng.choice([1, 2, 4]), T0, T0 + rng.choice([0, 1, 17, 33]), rng.choice(["chunked", "pair"])))
    return cases


@pytest.mark.parametrize("dim,hidden,n_layers,B,T0,T,path", _random_model_cases(10, 23))
def test_model_prefill_then_step_random(dim, hidden, n_layers, B, T0, T, path, monkeypatch):
    monkeypatch.setenv("ULM_FM_PATH", path)
    say(f"UnifiedLM.prefill of {T0} positions, then {T - T0} steps, B={B} dim={dim} A={hidden} {n_layers} blocks, "
        f"{path} form")
    _prefill_then_step(dim, hidden, n_layers, B, T0, T, dim * 31 + hidden + T0)


def test_flushed_states_after_steps_match_oracle():
    """UnifiedLM.flush_states after 5 steps past a prefill (5 write terms
    pending in every block): each block's S, c and r_prev are the oracle's
    state after the same 55 tokens (S = U - mu w) within 1e-2 (S from bf16
    products in the prefill), and stepping on from the flushed states gives the
    oracle's logits."""
    say("UnifiedLM.flush_states after a prefill of 50 positions and 5 steps vs the oracle's states")
    kw = dict(dim=32, n_layers=2, hidden_dim=64, vocab_size=97, max_seq_len=80)
    model = tiny_model(**kw).cuda()
    x = torch.randint(0, 97, (3, 60), generator=torch.Generator().manual_seed(5))
    _, states = model.prefill(x[:, :50].cuda())
    for t in range(50, 55):
        model.step(x[:, t].cuda(), states)
    assert all(s["np"] == 5 for s in states)
    model.flush_states(states)
    p = oracle_params(model)
    so = _oracle_states(p, x[:, :55], kw["n_layers"])
    for i, (a, o) in enumerate(zip(states, so)):
        assert a["np"] == 0
        w = fm.prior_mass(p[f"layers.{i}.log_w"])
        errs = {"S": rel(a["S"], o["U"] - p[f"layers.{i}.mu.weight"] * w), "c": rel(a["c"], o["c"]),
                "r_prev": rel(a["r_prev"], o["r_prev"])}
        say(f"  block {i} rel errors {errs}")
        assert max(errs.values()) < 1e-2, errs
    cont = torch.stack([model.step(x[:, t].cuda(), states) for t in range(55, 60)], 1)
    ref = fm.forward_recurrent(p, x)
    assert rel(cont, ref[:, 55:]) < 1e-2


def test_model_prefill_short_prompt():
    """A prompt shorter than the conv window (T = 2 < 3): the window keeps its zeros."""
    say("UnifiedLM.prefill of 2 positions vs forward_recurrent")
    model = tiny_model(dim=32, n_layers=2, hidden_dim=64, vocab_size=97, max_seq_len=40).cuda()
    x = torch.randint(0, 97, (2, 6), generator=torch.Generator().manual_seed(4)).cuda()
    logits0, states = model.prefill(x[:, :2])
    cont = torch.stack([model.step(x[:, t], states) for t in range(2, 6)], 1)
    ref = model.forward_recurrent(x)
    assert rel(logits0, ref[:, 1]) < 1e-2
    assert rel(cont, ref[:, 2:]) < 1e-2


@pytest.mark.parametrize("path", ["chunked", "pair"])
def test_model_prefill_under_autocast(path, monkeypatch):
    """The fused prefill with bf16 GEMM operands (the bench's configuration)
    in both forms: logits and the decode states after the prompt against the
    oracle, 1e-2."""
    monkeypatch.setenv("ULM_FM_PATH", path)
    say(f"UnifiedLM.prefill under bf16 autocast, 100 positions, {path} form, vs the oracle's states and forward_recurrent")
    kw = dict(dim=64, n_layers=2, hidden_dim=128, vocab_size=97, max_seq_len=160)
    model = tiny_model(**kw).cuda()
    x = torch.randint(0, 97, (2, 120), generator=torch.Generator().manual_seed(6))
    T0 = 100
    with torch.autocast("cuda", dtype=torch.bfloat16):
        logits0, states = model.prefill(x[:, :T0].cuda())
    cont = torch.stack([model.step(x[:, t].cuda(), states) for t in range(T0, 120)], 1)
    torch.cuda.synchronize()
    p = oracle_params(model)
    ref = fm.forward_recurrent(p, x)
    errs = {"logits": rel(logits0.float(), ref[:, T0 - 1]), "continued": rel(cont, ref[:, T0:])}
    say(f"  rel errors {errs}")
    assert max(errs.values()) < 1e-2, errs
