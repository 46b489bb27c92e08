"""How far bf16 operands alone move the decay gradient of a block, in exact
arithmetic: the bound any bf16 evaluation of the fast memory meets (the
reference's Triton path rounds q and k to bf16 as well, kernel.py:205-213).

The block-parity cases (tests/test_gpu_block.py) hold every gradient to 1e-2
against float64. Their draws are ones where that bound sits well inside 1e-2;
this file pins it for two of them and for one draw where it does not (D=40,
A=70, T=150), which is why that draw is not a parity case: there q and k in
bf16, with every other operation exact, move the log_rate gradient by 9e-3.
"""
import pytest
import torch

from helpers import tiny_model
from oracle import fastmem as fm


def _block_grads(B, T, D, A, round_qk, monkeypatch):
    model = tiny_model(seed=T + A, dim=D, hidden_dim=A, n_layers=1, vocab_size=97, max_seq_len=max(T, 64))
    blk = model.layers[0]
    gen = torch.Generator().manual_seed(A)
    with torch.no_grad():
        blk.norm.weight.copy_(1.0 + 0.2 * torch.randn(D, generator=gen))
    x = torch.randn(B, T, D, generator=gen)
    head = torch.randn(97, D, generator=gen, dtype=torch.float64) / D ** 0.5
    targets = torch.randint(0, 97, (B, T), generator=gen)

    def dense(r, v, lam, w):
        # the quadratic form of the oracle, with q and k (optionally) in bf16
        k = fm.shift_keys(r)
        M = fm.decay_mask(r.shape[1], lam, r.dtype)
        q = r / (w + M @ k)
        qq, kk = (fm.round_bf16(q), fm.round_bf16(k)) if round_qk else (q, k)
        return q, ((qq @ kk.transpose(1, 2)) * M) @ v.to(r.dtype)

    monkeypatch.setattr(fm, "dense_fast_memory", dense)
    p = {n: t.detach().double().requires_grad_() for n, t in blk.named_parameters()}
    out = fm.block_forward(p, "", x.double(), norm_eps=blk.norm.eps, form="dense", autocast=True)
    torch.nn.functional.cross_entropy((out @ head.t()).reshape(-1, 97), targets.reshape(-1)).backward()
    return {n: t.grad for n, t in p.items()}


@pytest.mark.parametrize("B,T,D,A,lo,hi", [
    (2, 150, 64, 70, 0.0, 2e-3),      # parity cases of tests/test_gpu_block.py
    (2, 200, 64, 140, 0.0, 2e-3),
    (2, 150, 40, 70, 5e-3, 2e-2),     # the ill-conditioned draw
])
def test_bf16_qk_move_the_decay_gradient(B, T, D, A, lo, hi, monkeypatch):
    exact = _block_grads(B, T, D, A, False, monkeypatch)
    rounded = _block_grads(B, T, D, A, True, monkeypatch)
    moved = ((exact["log_rate"] - rounded["log_rate"]).norm() / exact["log_rate"].norm()).item()
    assert lo <= moved < hi, moved
