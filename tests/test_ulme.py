"""ULMe v1 loader / exporter of the package (CPU), against the checkpoint the
oracle's writer made for the reference's run.c (tests/golden/runc_greedy.npz,
made by tests/golden/make_golden.py)."""
import os
import struct

import numpy as np
import pytest
import torch

from oracle import fastmem as fm

import ulme
from model import ModelArgs, UnifiedLM

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "runc_greedy.npz")
SHAPE = dict(dim=32, n_layers=2, hidden_dim=64, vocab_size=512, conv_size=4)


def _golden():
    z = np.load(GOLDEN)
    return z, z["checkpoint"].tobytes()


def _model_from_oracle_params(seed):
    p = fm.tiny_params(seed=seed, **SHAPE, dtype=torch.float32)
    model = UnifiedLM(ModelArgs(dim=SHAPE["dim"], n_layers=SHAPE["n_layers"], hidden_dim=SHAPE["hidden_dim"],
                                vocab_size=SHAPE["vocab_size"], conv_size=SHAPE["conv_size"], max_seq_len=64))
    model.load_state_dict({**p, "output.weight": p["tok_embeddings.weight"]})
    return model, p


def test_export_matches_the_golden_checkpoint(tmp_path):
    z, ckpt = _golden()
    model, _ = _model_from_oracle_params(int(z["seed"]))
    path = tmp_path / "m.bin"
    ulme.export_ulme(model, str(path))
    assert path.read_bytes() == ckpt


def test_load_gives_the_decoder_scalars_back(tmp_path):
    z, ckpt = _golden()
    path = tmp_path / "m.bin"
    path.write_bytes(ckpt)
    model = ulme.load_ulme(str(path))
    ref, p = _model_from_oracle_params(int(z["seed"]))
    assert model.params.dim == 32 and model.params.hidden_dim == 64 and model.params.max_seq_len == 64
    assert model.output.weight is model.tok_embeddings.weight
    for name, t in p.items():
        if name.endswith(("log_w", "log_rate", "log_eps")):
            continue
        assert torch.equal(model.state_dict()[name], t), name
    for a, b in zip(model.layers, ref.layers):
        assert torch.allclose(a._w(), b._w(), rtol=1e-6, atol=0)
        assert torch.allclose(torch.exp(-a.log_rate.exp()), torch.exp(-b.log_rate.exp()), rtol=1e-6, atol=0)
        assert torch.allclose(a.log_eps.exp(), b.log_eps.clamp(-10, 10).exp(), rtol=1e-6, atol=0)
    # and back: the same bytes
    again = tmp_path / "again.bin"
    ulme.export_ulme(model, str(again))
    assert again.read_bytes() == ckpt


def test_untied_classifier_round_trip(tmp_path):
    model, _ = _model_from_oracle_params(5)
    model.output.weight = torch.nn.Parameter(torch.randn_like(model.output.weight))
    path = tmp_path / "m.bin"
    ulme.export_ulme(model, str(path))
    header = ulme.read_header(path.read_bytes())
    assert header["shared_classifier"] == 0
    back = ulme.load_ulme(str(path))
    assert back.output.weight is not back.tok_embeddings.weight
    assert torch.equal(back.output.weight, model.output.weight)


@pytest.mark.parametrize("patch,match", [
    (lambda b: struct.pack("<I", 0x12345678) + b[4:], "magic"),
    (lambda b: b[:4] + struct.pack("<i", 2) + b[8:], "version"),
    (lambda b: b[:-4], "floats"),
    (lambda b: b[:100], "header"),
])
def test_malformed_checkpoints_are_rejected(tmp_path, patch, match):
    _, ckpt = _golden()
    path = tmp_path / "bad.bin"
    path.write_bytes(patch(ckpt))
    with pytest.raises(ValueError, match=match):
        ulme.load_ulme(str(path))
