"""Shared fixtures of the GPU parity tests."""
import ctypes
import math
import os
import sys

import torch

from model import ModelArgs, UnifiedLM


def say(msg):
    """Names the case about to run, flushed before any GPU work."""
    print(msg, flush=True)
    sys.stdout.flush()


def rel(got, ref):
    """Norm-wise relative error (test_all.py:153)."""
    got, ref = got.double().cpu(), ref.double().cpu()
    return ((got - ref).norm() / ref.norm().clamp(min=1e-30)).item()


def tiny_model(seed=0, **kw):
    """The reference's test fixture (test_all.py:78-90) on this package's model."""
    torch.manual_seed(seed)
    args = ModelArgs(**{**dict(dim=32, n_layers=3, hidden_dim=48, vocab_size=97, max_seq_len=40), **kw})
    model = UnifiedLM(args).eval()
    with torch.no_grad():
        for layer in model.layers:
            layer.conv.weight.normal_(std=0.5)
            layer.key.bias.normal_(std=0.5)
            layer.val.weight.normal_(std=0.2)
            layer.log_rate.fill_(math.log(0.05))
            layer.log_w.normal_(std=1.0)
    return model


def oracle_params(model, device="cpu", requires_grad=False):
    """The model's parameters as a float64 dict for the oracle."""
    out = {}
    for name, p in model.named_parameters():
        t = p.detach().to(device=device, dtype=torch.float64).clone()
        out[name] = t.requires_grad_(requires_grad)
    return out


def fm_inputs(B, T, A, D, seed=0, device="cuda", lam=None, zero_frac=0.5):
    """Seeded fast-memory inputs with the statistics of a real block: r from
    the relu^2 address of N(0,1) pre-activations (about half zero), v ~ N(0,1),
    w = 4 + noise, lam = sigmoid(N(3, .5)) unless given."""
    gen = torch.Generator().manual_seed(seed)
    pre = torch.randn(B, T, A, generator=gen, dtype=torch.float64)
    z = pre.clamp(min=0) ** 2
    r = z / (1.0 + z.sum(-1, keepdim=True))
    v = torch.randn(B, T, D, generator=gen, dtype=torch.float64)
    w = 4.0 * torch.exp(0.3 * torch.randn(A, generator=gen, dtype=torch.float64))
    if lam is None:
        lam = torch.sigmoid(3.0 + 0.5 * torch.randn((), generator=gen, dtype=torch.float64))
    g = torch.log(torch.as_tensor(lam, dtype=torch.float64))
    return [t.to(device) for t in (r, v, g, w)]


# ---- the test-only probe library (libulm_probe.so, include/ulm_probe.h)
_probe = None
PROBE_SIGNATURES = {
    "ulm_probe_mfma": (ctypes.c_int, [ctypes.c_void_p] * 4),
    "ulm_probe_lds_tr": (ctypes.c_int, [ctypes.c_void_p] * 3),
    "ulm_probe_lds_dma": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_void_p]),
    "ulm_last_error": (ctypes.c_char_p, []),
}


def probe_lib():
    """The layout-probe library built beside libulm_fm.so; raises if missing."""
    global _probe
    if _probe is None:
        import ulm_native as nat
        path = os.path.join(os.path.dirname(nat.LIB_PATH), "libulm_probe.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: build it with `python unifiedlm.c_amd/build.py`")
        lib = ctypes.CDLL(path)
        for name, (res, args) in PROBE_SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _probe = lib
    return _probe


def probe_call(name, *args):
    """Calls a probe and raises RuntimeError on a nonzero status."""
    st = getattr(probe_lib(), name)(*args)
    if st != 0:
        raise RuntimeError(f"{name} failed with status {st}: {probe_lib().ulm_last_error().decode(errors='replace')}")
