"""ULMe v1: the fp32 checkpoint format of the reference's C decoder
(export.py:4-12, 37-82 writes it; run.c:140-186 reads it).

Layout: a 256-byte header holding the uint32 magic 0x554C4D65 ("ULMe"), the
int32 version 1 and seven int32 fields (dim, n_layers, hidden_dim, vocab_size,
max_seq_len, conv_size, shared_classifier), zero padded; then little-endian
fp32 arrays: the token embedding (vocab, dim); per block the norm weight
(dim), the conv taps (dim, conv_size) oldest first, the key weight
(hidden_dim, dim) and bias (hidden_dim), mu (dim, hidden_dim), val (dim, dim),
and the learned scalars in the form the decoder uses them:
w = exp(clamp(log_w, -7, 12)) (hidden_dim), lam = exp(-exp(log_rate)),
eps = exp(clamp(log_eps, -10, 10)); then the final norm (dim) and, when it is
not tied to the embedding, the classifier (vocab, dim).

load_ulme turns such a file back into this package's UnifiedLM: log_w, log_rate
and log_eps are the logarithms that give back the stored w, lam and eps, so
UnifiedLM.step / prefill decode what run.c decodes (the norm eps, fixed at
1e-5 in run.c:198, is ModelArgs' default).
"""
import struct

import numpy as np
import torch

MAGIC = 0x554C4D65
VERSION = 1
HEADER_BYTES = 256
_FIELDS = ("dim", "n_layers", "hidden_dim", "vocab_size", "max_seq_len", "conv_size", "shared_classifier")


def _f32(t):
    return t.detach().cpu().to(torch.float32).reshape(-1).numpy().astype("<f4").tobytes()


def export_ulme(model, path):
    """Write `model` (a UnifiedLM) as ULMe v1 (export.py:37-82)."""
    p = model.params
    shared = bool(torch.equal(model.tok_embeddings.weight, model.output.weight))
    header = struct.pack("<Ii7i", MAGIC, VERSION, p.dim, p.n_layers, p.hidden_dim, p.vocab_size, p.max_seq_len,
                         p.conv_size, int(shared))
    with open(path, "wb") as f:
        f.write(header + b"\0" * (HEADER_BYTES - len(header)))
        f.write(_f32(model.tok_embeddings.weight))
        for layer in model.layers:
            for t in (layer.norm.weight, layer.conv.weight[:, 0, :], layer.key.weight, layer.key.bias,
                      layer.mu.weight, layer.val.weight, layer._w(), torch.exp(-layer.log_rate.exp()),
                      layer.log_eps.clamp(-10, 10).exp()):
                f.write(_f32(t))
        f.write(_f32(model.norm.weight))
        if not shared:
            f.write(_f32(model.output.weight))


def read_header(data):
    """(config dict) from the first 256 bytes; raises ValueError as run.c exits
    on a bad magic or version (run.c:147-158)."""
    if len(data) < HEADER_BYTES:
        raise ValueError(f"ULMe header needs {HEADER_BYTES} bytes, got {len(data)}")
    magic, version, *vals = struct.unpack("<Ii7i", data[:36])
    if magic != MAGIC:
        raise ValueError(f"bad checkpoint magic for UnifiedLM: 0x{magic:08x}")
    if version != VERSION:
        raise ValueError(f"ULMe version {version}; this reader takes the fp32 version 1")
    cfg = dict(zip(_FIELDS, vals))
    if min(cfg[k] for k in _FIELDS[:6]) <= 0:
        raise ValueError(f"bad ULMe config {cfg}")
    return cfg


def load_ulme(path, device="cpu"):
    """A UnifiedLM (fp32, eval mode) holding the weights of a ULMe v1 file."""
    from model import ModelArgs, UnifiedLM
    data = open(path, "rb").read()
    cfg = read_header(data)
    d, L, m, V, Kc = cfg["dim"], cfg["n_layers"], cfg["hidden_dim"], cfg["vocab_size"], cfg["conv_size"]
    per_block = d + d * Kc + m * d + m + d * m + d * d + m + 1 + 1
    n = V * d + L * per_block + d + (0 if cfg["shared_classifier"] else V * d)
    body = np.frombuffer(data, dtype="<f4", offset=HEADER_BYTES)
    if body.size != n:
        raise ValueError(f"ULMe body holds {body.size} floats, the header implies {n}")
    pos = 0

    def take(*shape):
        nonlocal pos
        k = int(np.prod(shape))
        t = torch.from_numpy(body[pos:pos + k].copy()).reshape(*shape)
        pos += k
        return t

    model = UnifiedLM(ModelArgs(dim=d, n_layers=L, hidden_dim=m, vocab_size=V, max_seq_len=cfg["max_seq_len"],
                                conv_size=Kc))
    with torch.no_grad():
        model.tok_embeddings.weight.copy_(take(V, d))
        for layer in model.layers:
            layer.norm.weight.copy_(take(d))
            layer.conv.weight.copy_(take(d, Kc)[:, None, :])
            layer.key.weight.copy_(take(m, d))
            layer.key.bias.copy_(take(m))
            layer.mu.weight.copy_(take(d, m))
            layer.val.weight.copy_(take(d, d))
            layer.log_w.copy_(take(m).log())
            lam = take(1)[0]
            if not 0.0 < float(lam) < 1.0:
                raise ValueError(f"ULMe decay lam={float(lam)} outside (0, 1)")
            layer.log_rate.copy_(torch.log(-torch.log(lam)))
            layer.log_eps.copy_(take(1)[0].log())
        model.norm.weight.copy_(take(d))
        if cfg["shared_classifier"]:
            model.output.weight = model.tok_embeddings.weight
        else:
            model.output.weight = torch.nn.Parameter(take(V, d))
    return model.to(device).eval()
