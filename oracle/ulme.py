"""Writer of the ULMe v1 fp32 checkpoint read by the reference's run.c
(ORACLE side, test infrastructure).

Layout (export.py:4-12, 37-82; run.c:140-186): a 256-byte header holding the
uint32 magic 0x554C4D65 ("ULMe"), int32 version 1 and seven int32 fields
(dim, n_layers, hidden_dim, vocab_size, max_seq_len, conv_size,
shared_classifier), zero padded; then fp32 arrays: the token embedding, per
block norm, conv taps (dim, conv_size) oldest -> newest, key weight, key bias,
mu, val, w = exp(clamp(log_w,-7,12)), lam = exp(-exp(log_rate)),
eps = exp(clamp(log_eps,-10,10)); then the final norm, and the classifier only
when it is not tied to the embedding.
"""
import struct

import numpy as np
import torch

MAGIC = 0x554C4D65
HEADER_BYTES = 256


def _f32(t):
    return torch.as_tensor(t).detach().cpu().to(torch.float32).reshape(-1).numpy().tobytes()


def write_ulme_v1(p, path, max_seq_len=256):
    """Write parameter dict ``p`` (state_dict names) as ULMe v1 to ``path``."""
    emb = p["tok_embeddings.weight"]
    out_w = p.get("output.weight", emb)
    shared = bool(out_w is emb or torch.equal(out_w, emb))
    n_layers = 1 + max(int(k.split(".")[1]) for k in p if k.startswith("layers."))
    key = p["layers.0.key.weight"]
    conv = p["layers.0.conv.weight"]
    vocab, dim = emb.shape
    header = struct.pack("<Ii7i", MAGIC, 1, dim, n_layers, key.shape[0], vocab, max_seq_len,
                         conv.shape[-1], int(shared))
    with open(path, "wb") as f:
        f.write(header + b"\0" * (HEADER_BYTES - len(header)))
        f.write(_f32(emb))
        for i in range(n_layers):
            g = lambda n: p[f"layers.{i}.{n}"]
            f.write(_f32(g("norm.weight")))
            f.write(_f32(g("conv.weight")[:, 0, :]))
            f.write(_f32(g("key.weight")))
            f.write(_f32(g("key.bias")))
            f.write(_f32(g("mu.weight")))
            f.write(_f32(g("val.weight")))
            f.write(_f32(g("log_w").clamp(-7.0, 12.0).exp()))
            f.write(_f32(torch.exp(-g("log_rate").exp())))
            f.write(_f32(g("log_eps").clamp(-10, 10).exp()))
        f.write(_f32(p["norm.weight"]))
        if not shared:
            f.write(_f32(out_w))


def read_header(path):
    with open(path, "rb") as f:
        raw = f.read(HEADER_BYTES)
    magic, version, *cfg = struct.unpack("<Ii7i", raw[:36])
    return magic, version, cfg
