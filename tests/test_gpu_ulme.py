"""A ULMe v1 checkpoint loaded by the package and decoded on the GPU against the
reference's run.c (needs an MI355X). tests/golden/runc_greedy.npz holds the
checkpoint, a prompt, run.c's greedy sequence (run.c:542-571 at temperature 0)
and its logits at every position (tests/golden/make_golden.py).

Tolerances: the fp32 decode path 1e-5 (and the exact greedy tokens); the
chunked prefill, whose state comes from bf16 products, 1e-2.
"""
import os

import numpy as np
import pytest
import torch

from helpers import say

pytestmark = pytest.mark.gpu

import ulme  # noqa: E402

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "runc_greedy.npz")


def _load(tmp_path):
    z = np.load(GOLDEN)
    path = tmp_path / "model.bin"
    path.write_bytes(z["checkpoint"].tobytes())
    return z, ulme.load_ulme(str(path), device="cuda")


def test_greedy_decode_matches_runc(tmp_path):
    say("ULMe checkpoint -> GPU greedy decode (step) vs run.c")
    z, model = _load(tmp_path)
    steps = int(z["steps"])
    prompt = torch.from_numpy(z["prompt"])[None].cuda()
    seq = model.decode_greedy(prompt, steps, prefill=False)[0].cpu().numpy()
    assert np.array_equal(seq, z["tokens"]), (seq, z["tokens"])
    states = model.init_states(1, "cuda")
    got = torch.stack([model.step(torch.tensor([int(t)], device="cuda"), states)[0] for t in seq[:steps]]).cpu()
    ref = torch.from_numpy(z["logits"])
    assert (got - ref).abs().max() < 1e-5 * ref.abs().max()


def test_prefill_then_decode_matches_runc(tmp_path):
    say("ULMe checkpoint -> GPU chunked prefill of the prompt, then steps on run.c's sequence")
    z, model = _load(tmp_path)
    steps = int(z["steps"])
    seq = torch.from_numpy(z["tokens"]).cuda()
    T0 = len(z["prompt"])
    logits, states = model.prefill(seq[None, :T0])
    got = [logits[0]]
    for t in range(T0, steps):
        got.append(model.step(seq[t:t + 1], states)[0])
    got = torch.stack(got).cpu()
    ref = torch.from_numpy(z["logits"][T0 - 1:steps])
    err = ((got - ref).norm() / ref.norm()).item()
    say(f"  rel error {err:.2e}")
    assert err < 1e-2
