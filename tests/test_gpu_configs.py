"""Parity at the widths of the 110M benchmark (needs an MI355X): the whole
12-block UnifiedLM, D=768, A=3072, vocab 32000, in its two uses.

- Decode (forward_recurrent, model.py:164-175) of N=3 sequences over 32
  positions in fp32 against the oracle's forward_recurrent in float64, held
  to 1e-5 relative (the decode tolerance of test_all.py:110-116 tightened to
  fp32's).
- One training step at T=1024 (test_all.py:140-166's protocol at the 110M
  shape, B=1): loss and every parameter gradient against the oracle's
  lm_forward in float64, within 1e-2; under bf16 autocast against the oracle
  with autocast's roundings (lm_forward(autocast=True)).

The oracle runs in float64 on the GPU with plain torch ops (the dense form of
the fast memory, pinned against brute force on the CPU); the weights are drawn
from the benchmark distribution, so every block's memory is populated.
"""
import pytest
import torch

from helpers import oracle_params, rel, say
from oracle import fastmem as fm

pytestmark = pytest.mark.gpu

from model import ModelArgs, UnifiedLM  # noqa: E402
from workloads import init_decode_model  # noqa: E402

WIDTH = dict(dim=768, n_layers=12, hidden_dim=3072, vocab_size=32000)


def _model(seed, max_seq_len):
    torch.manual_seed(seed)
    model = UnifiedLM(ModelArgs(**WIDTH, max_seq_len=max_seq_len))
    return init_decode_model(model, seed).cuda()


def test_decode_at_110m_width_matches_oracle():
    N, T = 3, 32
    say(f"decode at the 110M width: 12 blocks D=768 A=3072 V=32000, N={N}, {T} positions, fp32")
    model = _model(11, T).eval()
    x = torch.randint(0, WIDTH["vocab_size"], (N, T), generator=torch.Generator().manual_seed(11))
    with torch.no_grad():
        got = model.forward_recurrent(x.cuda())
        ref = fm.forward_recurrent(oracle_params(model, device="cuda"), x.cuda())
    torch.cuda.synchronize()
    err = rel(got, ref)
    worst = ((got.double() - ref).abs().max() / ref.abs().max()).item()
    say(f"  rel error {err:.3e}, max |diff| / max |logit| {worst:.3e}")
    assert err < 1e-5 and worst < 1e-5


@pytest.mark.parametrize("autocast", [False, True])
def test_training_step_at_110m_shape_matches_oracle(autocast):
    T = 1024
    say(f"training step at the 110M shape: 12 blocks D=768 A=3072 V=32000, B=1 T={T}, autocast={autocast}")
    model = _model(12, T).train()
    gen = torch.Generator().manual_seed(12)
    x = torch.randint(0, WIDTH["vocab_size"], (1, T), generator=gen)
    y = torch.randint(0, WIDTH["vocab_size"], (1, T), generator=gen)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        model(x.cuda(), y.cuda())
    model.last_loss.backward()
    torch.cuda.synchronize()
    params = oracle_params(model, device="cuda", requires_grad=True)
    _, loss = fm.lm_forward(params, x.cuda(), y.cuda(), form="dense", autocast=autocast)
    loss.backward()
    errs = {"loss": abs(model.last_loss.item() - loss.item()) / abs(loss.item())}
    for name, p in model.named_parameters():
        errs[name] = rel(p.grad, params[name].grad)
    worst = max(errs, key=errs.get)
    say(f"  loss {loss.item():.6f}; worst {worst} {errs[worst]:.3e}")
    assert max(errs.values()) < 1e-2, {k: e for k, e in errs.items() if e >= 1e-3}


def test_decode_at_its_benchmark_batch():
    """The decode workload at its own batch: N=256 sequences of a 512-token
    prompt through the chunked prefill (UnifiedLM.prefill, fp32 GEMMs), then 20
    decode steps (model.py:96-111, 164-175; one write-back of the deferred
    state at the 16th), the 29 GB of fp32 state resident. Rows 0, 137 and 255
    must equal (within 1e-5) the same prompts run alone at N=1, every row
    stays finite, and row 0's logits after the last step are within 1e-2 of
    the oracle's forward_recurrent over the same 532 tokens in float64 (the
    prefill's products take bf16 operands)."""
    N, T, steps = 256, 512, 20
    say(f"decode at the benchmark batch: N={N}, prefill {T} positions, {steps} steps, 12 blocks D=768 A=3072")
    model = _model(13, 1024).eval()
    gen = torch.Generator().manual_seed(13)
    prompt = torch.randint(0, WIDTH["vocab_size"], (N, T), generator=gen)
    nxt = torch.randint(0, WIDTH["vocab_size"], (steps, N), generator=gen)

    def run(rows):
        logits, states = model.prefill(prompt[rows].cuda())
        outs = [logits]
        for i in range(steps):
            outs.append(model.step(nxt[i, rows].cuda(), states))
        torch.cuda.synchronize()
        return torch.stack(outs, 1)          # (n, steps + 1, V)

    with torch.no_grad():
        full = run(slice(None))
        assert torch.isfinite(full).all()
        for row in (0, 137, 255):
            alone = run(slice(row, row + 1))
            err = rel(full[row], alone[0])
            say(f"  row {row}: N={N} vs N=1 rel {err:.3e}")
            assert err < 1e-5
        tokens = torch.cat([prompt[:1], nxt[:, :1].t()], 1).cuda()
        ref = fm.forward_recurrent(oracle_params(model, device="cuda"), tokens)[0, T - 1:]
    err = rel(full[0], ref)
    say(f"  row 0 vs the oracle's forward_recurrent: rel {err:.3e}")
    assert err < 1e-2
