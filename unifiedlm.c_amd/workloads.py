"""Seeded synthetic workloads at the benchmark shapes of the fast-memory path.

Block inputs follow one distribution at every shape: h ~ N(0,1) as the block
input (RMSNorm weight 1 and the identity conv make u = h), key weight
K ~ N(0, 1/D), key bias 0, eps = 1 (log_eps = 0), value weight ~ N(0, 1/D),
prior w = 4, one decay lam = sigmoid(N(3, 0.5)) per block, mu ~ N(0, 0.02^2)
(0.02 read as a standard deviation). The relu^2 addresses then come out
about half zero with row sums below 1.
"""
import math

import torch

SHAPES = {
    "260K": dict(B=8, T=512, D=64, A=128, blocks=5),
    "15M": dict(B=32, T=256, D=288, A=1152, blocks=1),
    "42M": dict(B=16, T=1024, D=512, A=2048, blocks=1),
    "110M": dict(B=16, T=1024, D=768, A=3072, blocks=12),
    # the same widths and tokens per step in sequences of 8192 positions (the chunked state form's range)
    "110M-T8192": dict(B=2, T=8192, D=768, A=3072, blocks=12),
    # the reference's own published single-block timings (docs/kernel.md:57-62,
    # RTX 3090 Ti): 1.56 ms at D=288, A=712, B=32, T=256 and 3.18 ms at D=512,
    # A=1280, B=8, T=1024
    "ref-15M": dict(B=32, T=256, D=288, A=712, blocks=1, reference_ms=1.56),
    "ref-42M": dict(B=8, T=1024, D=512, A=1280, blocks=1, reference_ms=3.18),
}
DECODE_110M = dict(N=256, D=768, A=3072, blocks=12, vocab=32000, prefill=512, steps=256)


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def block_decay(seed):
    """lam = sigmoid(x), x ~ N(3, 0.5)."""
    return torch.sigmoid(3.0 + 0.5 * torch.randn((), generator=_gen(seed), dtype=torch.float64)).item()


def block_inputs(B, T, D, A, seed, device="cuda", v_dtype=torch.float32):
    """(r, v, g, w) of one block: r fp32 (B,T,A), v (B,T,D) in v_dtype, g 0-d fp32, w (A,) fp32."""
    gen = _gen(seed)
    h = torch.randn(B, T, D, generator=gen)
    K = torch.randn(A, D, generator=gen) / math.sqrt(D)
    Wv = torch.randn(D, D, generator=gen) / math.sqrt(D)
    h, K, Wv = h.to(device), K.to(device), Wv.to(device)
    z = torch.relu(h @ K.t()).square()
    r = z / (1.0 + z.sum(-1, keepdim=True))
    v = (h @ Wv.t()).to(v_dtype)
    lam = block_decay(seed + 7919)
    g = torch.tensor(math.log(lam), dtype=torch.float32, device=device)
    w = torch.full((A,), 4.0, dtype=torch.float32, device=device)
    return r.contiguous(), v.contiguous(), g, w


def init_decode_model(model, seed):
    """Re-draws every block of a UnifiedLM with the benchmark distribution
    (the default init zeroes the value weight, which would leave S = 0)."""
    gen = _gen(seed)
    D = model.params.dim
    with torch.no_grad():
        for i, layer in enumerate(model.layers):
            layer.key.weight.copy_(torch.randn(layer.key.weight.shape, generator=gen) / math.sqrt(D))
            layer.key.bias.zero_()
            layer.val.weight.copy_(torch.randn(layer.val.weight.shape, generator=gen) / math.sqrt(D))
            layer.mu.weight.copy_(torch.randn(layer.mu.weight.shape, generator=gen) * 0.02)
            layer.log_eps.zero_()
            layer.log_w.fill_(math.log(4.0))
            lam = block_decay(seed + 31 * i)
            layer.log_rate.fill_(math.log(-math.log(lam)))
    return model


def decode_bytes_per_step(N, L, A, D, V, conv_size=4, pending=1):
    """Algorithmic HBM bytes of one decode position for N sequences and L blocks, fp32:
    the state S, c and r_prev read+write, the conv window read+write, every block's
    weights once and the tied classifier. pending = 1: S read and written at
    every position. pending = J > 1 (the deferred write-back): S read at every
    position and written at one in J, the appended term (v and r_prev) written
    once, and the pending terms read, (J + 1) / 2 of them on average."""
    kw = conv_size - 1
    if pending <= 1:
        per_seq_block = 8 * A * D + 16 * A + 8 * kw * D
    else:
        per_seq_block = (4 * A * D * (pending + 1)) // pending + 16 * A + 8 * kw * D + 4 * (A + D) \
            + 2 * (A + D) * (pending + 1)
    # norm D, conv D*Kc, key A*D + bias A, mu D*A, val D*D, w A, lam, eps
    weights = 4 * (2 * A * D + D * D + 2 * A + (1 + conv_size) * D + 2)
    return N * L * per_seq_block + L * weights + 4 * V * D


def la_flops(B, T, K, V, chunk=64):
    """Algorithmic flops of one chunked product o = LA(a, b, c) with keys K and
    values V: state update 2KV, state read-out 2KV, intra scores 2CK and intra
    apply 2CV per token, intra tiles counted dense."""
    return B * T * (4 * K * V + 2 * chunk * (K + V))


def block_flops_per_token(T, A, D, chunk=64, path="chunked"):
    """Algorithmic flops of one UnifiedBlock per token, forward + backward: the
    key, value and mu GEMMs (2AD + 2D^2 + 2AD forward, twice that backward) and
    the fast memory, 16AD + 8C(A + D) in the chunked state form or
    3 (A + D) (T + 1) in the block-pair form (its average over a sequence)."""
    fm = 3 * (A + D) * (T + 1) if path == "pair" else 16 * A * D + 8 * chunk * (A + D)
    return 3 * (4 * A * D + 2 * D * D) + fm


def la_kernel_flops(B, T, K, V, chunk=64):
    """Algorithmic flops of one launch of the K-group chunked kernel: state
    update 2KV, read-out 2KV and intra apply 2CV per token. The intra scores
    (2CK per token) are computed once per chunk by the scores kernel."""
    return B * T * (4 * K * V + 2 * chunk * V)


PAIR_BLOCK = 128   # position block of the block-pair products


def pair_flops(B, T, A, D):
    """Algorithmic flops of the block-pair evaluation of one block's fast
    memory, forward + backward: every causal pair (t, s), s <= t, of a batch
    row costs 2A (scores) + 2D (apply) + 2D (dscores) + 2A (dq_f) + 2A (dk_f)
    + 2D (dv)."""
    return 3 * (A + D) * B * T * (T + 1)


def pair_tile_flops(B, T, A, D, G=PAIR_BLOCK):
    """The flops the six pair products execute: whole G x G tiles, the
    diagonal ones included (their upper halves are computed and masked)."""
    nb = -(-T // G)
    return B * nb * (nb + 1) * G * G * 3 * (A + D)


def chunked_flops_per_token(A, D, chunk=64):
    """Flops per token of the chunked state form of one block, fwd + bwd:
    16AD + 8C(A + D) (four chunked products)."""
    return 16 * A * D + 8 * chunk * (A + D)
