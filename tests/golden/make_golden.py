"""Writes two fixtures from the reference's own run.c:

tests/golden/runc_decode.npz: logits of run.c's forward() on a fixed token sequence;
tests/golden/runc_greedy.npz: a ULMe v1 checkpoint (bytes), a prompt, and the
greedy continuation run.c's generate loop (run.c:542-571) produces from it,
with the logits at every position.


The reference holds no numeric golden vectors, so this script makes one from
its C decoder: it compiles run.c unmodified (oracle/Makefile -> oracle/_ref),
writes seeded parameters as a ULMe v1 checkpoint, feeds a fixed token
sequence through run.c's forward() one position at a time (as its generate
loop does, run.c:542-571) and stores the parameters, the tokens and run.c's
fp32 logits. Needs the reference checkout; run from the repository root:

    python tests/golden/make_golden.py
"""
import os
import sys
import tempfile

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import fastmem, runc, ulme  # noqa: E402

OUT = os.path.join(ROOT, "tests", "golden", "runc_decode.npz")
OUT_GREEDY = os.path.join(ROOT, "tests", "golden", "runc_greedy.npz")
# slots and width multiples of 32, so the chunked prefill applies to this model
SHAPE_GREEDY = dict(dim=32, n_layers=2, hidden_dim=64, vocab_size=512, conv_size=4)
SEED_GREEDY, PROMPT, STEPS = 11, 9, 64


def greedy(ref, prompt, steps):
    """run.c's generate loop (run.c:542-571) with temperature 0: feed the prompt,
    then the argmax (first maximum, run.c:460-469); stop before emitting BOS = 1."""
    ref.reset()
    token, seq, logits = prompt[0], [prompt[0]], []
    for pos in range(steps):
        lg = ref.forward(token)
        logits.append(lg)
        nxt = prompt[pos + 1] if pos < len(prompt) - 1 else int(np.argmax(lg))
        if nxt == 1:
            break
        seq.append(nxt)
        token = nxt
    return np.array(seq, dtype=np.int64), np.stack(logits).astype(np.float32)


def main_greedy():
    p = fastmem.tiny_params(seed=SEED_GREEDY, **SHAPE_GREEDY, dtype=torch.float32)
    prompt = torch.randint(2, SHAPE_GREEDY["vocab_size"], (PROMPT,),
                           generator=torch.Generator().manual_seed(SEED_GREEDY + 1)).tolist()
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "model.bin")
        ulme.write_ulme_v1(p, path, max_seq_len=STEPS)
        ckpt = np.frombuffer(open(path, "rb").read(), dtype=np.uint8)
        seq, logits = greedy(runc.RuncReference(path), prompt, STEPS)
    np.savez_compressed(OUT_GREEDY, checkpoint=ckpt, prompt=np.array(prompt, dtype=np.int64), tokens=seq,
                        logits=logits, steps=np.int64(STEPS), seed=np.int64(SEED_GREEDY))
    print(f"wrote {OUT_GREEDY}: prompt {PROMPT}, sequence {len(seq)}, checkpoint {ckpt.size} bytes")
SHAPE = dict(dim=32, n_layers=3, hidden_dim=48, vocab_size=97, conv_size=4)
SEED, T = 7, 80


def main():
    runc.build()
    p = fastmem.tiny_params(seed=SEED, **SHAPE, dtype=torch.float32)
    tokens = torch.randint(0, SHAPE["vocab_size"], (T,), generator=torch.Generator().manual_seed(SEED + 1))
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "model.bin")
        ulme.write_ulme_v1(p, path, max_seq_len=T)
        logits = runc.RuncReference(path).logits(tokens.tolist())
    arrays = {"param/" + k: v.numpy() for k, v in p.items()}
    np.savez_compressed(OUT, tokens=tokens.numpy().astype(np.int64), logits=logits.astype(np.float32),
                        seed=np.int64(SEED), **arrays)
    print(f"wrote {OUT}: tokens {T}, logits {logits.shape}")


if __name__ == "__main__":
    main()
    main_greedy()
