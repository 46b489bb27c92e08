"""Writes tests/golden/runc_decode.npz: logits of the reference's own run.c.

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
