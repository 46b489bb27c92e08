"""Float64 CPU restatement of the UnifiedLM fast-memory path (ORACLE, test infrastructure).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, to check the product against. Nothing in the product imports it.

Every function works on plain tensors (or a dict of parameters named like the
reference's ``UnifiedLM.state_dict()``), so the oracle does not depend on the
product's ``model.py``. The maths restated here, for one batch row and time t:

    k_t    = r_{t-1},  k_0 = 0                         kernel.py:6, test_all.py:71
    c_t    = w + sum_{s<=t} lam^(t-s) k_s              kernel.py:7
    q_t    = r_t / c_t                                 kernel.py:8
    fast_t = sum_{s<=t} lam^(t-s) (q_t . k_s) v_s      kernel.py:9
    lam    = exp(g),  g = -exp(log_rate)               model.py:84

and the block around it (model.py:70-85): RMSNorm, causal depthwise conv,
relu^2 address normalised by eps + row sum, value projection, mu read-out.

How each function is pinned (tests/test_oracle.py):
  dense_fast_memory     closed form; brute-force double loop on tiny shapes;
                        special cases lam -> 0, lam = 1, T = 1, zero rows.
  chunked_fast_memory   equals dense for chunk 1, 7, 16, 64 (test_all.py:100-107).
  fast_memory_state     S q_{T-1} and r_{T-1} / c give the dense fast and q at the
                        last position; equals the block decode state of
                        forward_recurrent's own steps (U - mu w, c).
  address               row sums z/(eps+z) < 1, zero where pre <= 0,
                        gradcheck of its backward formula.
  fast_memory_grads     torch.autograd.gradcheck at tiny shapes and the
                        reference's dg identity (kernel.py:173-175).
  dg_bf16_floor         with rounding off equals autograd's dg (the identity
                        with the kernel's tau); rounding its operands to bf16
                        is the only difference.
  pair_form_grads       with no roundings equals float64 autograd of the dense
                        form (every output and gradient); each rounding moves
                        only the outputs that read its operand.
  block_forward         autocast=False is the reference block; with autocast=True
                        its forward and its scalar/bias gradients match torch's
                        CPU bf16 autocast of the block's products (30x closer
                        than the exact block), and a rounding left out (planted)
                        breaks the agreement.
  round_grad_bf16       equals the backward of torch's own bf16 round trip.
  lm_forward            parallel == forward_recurrent (test_all.py:110-116),
                        causality (test_all.py:119-128), finite grads.
  forward_recurrent     logits of the reference's own run.c (compiled under
                        oracle/_ref) and the committed run.c golden fixture.
"""
import math

import torch
import torch.nn.functional as F


# ---------------------------------------------------------------------------
# fast-memory operator (kernel.py:1-15, test_all.py:28-61)

def shift_keys(r):
    """Write addresses k_t = r_{t-1}, k_0 = 0 (test_all.py:71, kernel.py:126)."""
    return F.pad(r, (0, 0, 1, 0))[:, :-1]


def decay_mask(T, lam, dtype=torch.float64):
    """M[t, s] = lam^(t-s) for s <= t, else 0 (test_all.py:58)."""
    dev = lam.device if isinstance(lam, torch.Tensor) else None
    t = torch.arange(T, dtype=dtype, device=dev)
    lag = (t[:, None] - t[None, :])
    return (lag >= 0).to(dtype) * lam ** lag.clamp(min=0)


def dense_fast_memory(r, v, lam, w):
    """Quadratic form (test_all.py:54-61): returns (q, fast).

    r (B,T,A), v (B,T,D), lam 0-d tensor, w (A,)."""
    T = r.shape[1]
    k = shift_keys(r)
    M = decay_mask(T, lam, r.dtype)
    c = w + M @ k
    q = r / c
    fast = ((q @ k.transpose(1, 2)) * M) @ v.to(r.dtype)
    return q, fast


def chunked_fast_memory(r, v, lam, w, chunk=64):
    """Chunkwise form (test_all.py:28-51): quadratic inside chunks of length
    ``chunk``, the A x D state and the A-vector evidence carried between them."""
    B, T, A = r.shape
    D = v.shape[-1]
    k = shift_keys(r)
    v = v.to(r.dtype)
    state = r.new_zeros(B, A, D)          # sum_s lam^(t0-1-s) k_s v_s^T
    mass = r.new_zeros(B, 1, A)           # sum_s lam^(t0-1-s) k_s
    qs, fs = [], []
    for t0 in range(0, T, chunk):
        L = min(chunk, T - t0)
        i = torch.arange(L, dtype=r.dtype, device=r.device)
        M = decay_mask(L, lam, r.dtype)
        into = (lam ** (i + 1))[None, :, None]          # carried state -> row i
        tail = (lam ** (L - 1 - i))[None, :, None]      # row i -> chunk end
        kc, rc, vc = k[:, t0:t0 + L], r[:, t0:t0 + L], v[:, t0:t0 + L]
        q = rc / (w + into * mass + M @ kc)
        inter = (q * into) @ state
        intra = ((q @ kc.transpose(1, 2)) * M) @ vc
        fs.append(inter + intra)
        qs.append(q)
        state = lam ** L * state + (kc * tail).transpose(1, 2) @ vc
        mass = lam ** L * mass + (kc * tail).sum(1, keepdim=True)
    return torch.cat(qs, 1), torch.cat(fs, 1)


def fast_memory_state(r, v, lam, w):
    """The decode state after the last position, by the token recurrence of
    UnifiedBlock.step (model.py:96-111) without its constant prior term:
    S <- lam S + v_t k_t^T and c <- lam c + (1 - lam) w + k_t, k_t = r_{t-1},
    from S = 0, c = w. Returns S (B, D, A) and c (B, A)."""
    B, T, A = r.shape
    D = v.shape[-1]
    k = shift_keys(r)
    vv = v.to(r.dtype)
    S = r.new_zeros(B, D, A)
    c = w.expand(B, A).clone()
    for t in range(T):
        S = lam * S + vv[:, t, :, None] * k[:, t, None, :]
        c = lam * c + (1 - lam) * w + k[:, t]
    return S, c


def la_dense(a, b, c, lam, reverse=False):
    """The chunked kernel's building block in quadratic form (kernel.py:183-184):
    o_t = sum_{s<=t} lam^(t-s) (a_t . b_s) c_s, or s >= t when ``reverse``."""
    a, b, c = a.double(), b.double(), c.double()
    if reverse:
        a, b, c = a.flip(1), b.flip(1), c.flip(1)
    M = decay_mask(a.shape[1], torch.as_tensor(lam, dtype=torch.float64)).to(a.device)
    o = ((a @ b.transpose(1, 2)) * M) @ c
    return o.flip(1) if reverse else o


def fast_memory(r, v, g, w, form="chunked", chunk=64):
    """unified_memory(r, v, g, w) -> (q, fast) (kernel.py:236-238) in the
    dtype of r; lam = exp(g). Differentiable in r, v, g, w."""
    lam = torch.exp(g)
    if form == "dense":
        return dense_fast_memory(r, v, lam, w)
    return chunked_fast_memory(r, v, lam, w, chunk)


def fast_memory_grads(r, v, g, w, dq, dfast, form="chunked"):
    """Float64 gradients (dr, dv, dg, dw) of <q, dq> + <fast, dfast> by autograd."""
    r = r.detach().double().requires_grad_(True)
    v = v.detach().double().requires_grad_(True)
    g = g.detach().double().requires_grad_(True)
    w = w.detach().double().requires_grad_(True)
    q, fast = fast_memory(r, v, g, w, form)
    loss = (fast * dfast.double()).sum()
    if dq is not None:
        loss = loss + (q * dq.double()).sum()
    dr, dv, dg, dw = torch.autograd.grad(loss, (r, v, g, w))
    return dr, dv, dg, dw


def dg_identity(r, v, g, w, dq_out, dfast):
    """The reference's closed form of d loss / d g (kernel.py:155-175):

        dg = sum_t t [q.dq_f + dc.(c - w)]_t - sum_s s [k.(dk_f + dk_c)]_s

    computed here from float64 autograd pieces; used to pin that identity."""
    r, v, w, g = r.double(), v.double(), w.double(), g.double()
    lam = torch.exp(g)
    B, T, A = r.shape
    k = shift_keys(r)
    M = decay_mask(T, lam)
    c = w + M @ k
    q = r / c
    do = dfast.double()
    S = (do @ v.transpose(1, 2)) * M                 # (dfast_t . v_s) lam^(t-s)
    P = (q @ k.transpose(1, 2)) * M                  # (q_t . k_s) lam^(t-s)
    dq_f = S @ k
    dk_f = S.transpose(1, 2) @ q
    dq = dq_f + (dq_out.double() if dq_out is not None else 0.0)
    dc = -dq * q / c
    dk_c = M.transpose(0, 1) @ dc
    pos = torch.arange(T, dtype=torch.float64, device=r.device)[None, :, None]
    return ((pos * (q * dq_f + dc * (c - w))).sum() - (pos * k * (dk_f + dk_c)).sum()), P


def dg_bf16_floor(r, v, g, w, dq_out, dfast, round_bf16=True):
    """d loss / d g as a bf16-operand kernel of this path computes it, in exact
    arithmetic otherwise: the fast-read products take v, dfast, q and k rounded
    to bf16, and the positional identity (kernel.py:155-175, with tau =
    (T-1)/2) weights the dq_f and dk_f terms with the same rounded q and k.
    With round_bf16=False it is the exact dg (pinned against autograd in
    tests/test_oracle.py). Its distance from the exact dg is the error that
    bf16 operands alone leave in dg, before any accumulation error: the floor
    for a kernel with bf16 MFMA operands. dg is the small difference of two
    large positional sums, so for inputs without the structure of a training
    loss (white-noise upstream gradients, long T) this floor can exceed 1e-2."""
    r, v, w, g = r.double(), v.double(), w.double(), g.double()
    rnd = (lambda x: x.to(torch.bfloat16).double()) if round_bf16 else (lambda x: x)
    lam = torch.exp(g)
    B, T, A = r.shape
    k = shift_keys(r)
    M = decay_mask(T, lam)
    c = w + M @ k
    q = r / c
    V, DO, K, Q = rnd(v), rnd(dfast.double()), rnd(k), rnd(q)
    S = (DO @ V.transpose(1, 2)) * M
    dq_f = S @ K
    dk_f = S.transpose(1, 2) @ Q
    dq = dq_f + (dq_out.double() if dq_out is not None else 0.0)
    dc = -dq * q / c
    dk_c = M.transpose(0, 1) @ dc
    pos = torch.arange(T, dtype=torch.float64, device=r.device)[None, :, None] - 0.5 * (T - 1)
    return (pos * (Q * dq_f + dc * (c - w))).sum() - (pos * (K * dk_f + k * dk_c)).sum()


# ---------------------------------------------------------------------------
# relu^2 slot address (model.py:70-72) and the block (model.py:31-42, 77-85)

def address(pre, log_eps):
    """r = z / (exp(clamp(log_eps, -10, 10)) + sum_a z), z = relu(pre)^2 where
    ``pre`` already includes the key bias (model.py:70-72)."""
    z = F.relu(pre).square()
    return z / (log_eps.clamp(-10, 10).exp() + z.sum(-1, keepdim=True))


def rmsnorm(x, weight, eps):
    """x * rsqrt(mean(x^2) + eps) * weight (model.py:37-42)."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * weight


def causal_conv(h, weight):
    """Depthwise causal conv: weight (D, 1, K), taps oldest -> newest (model.py:61, 79)."""
    Kc = weight.shape[-1]
    T = h.shape[1]
    return F.conv1d(h.transpose(1, 2), weight, padding=Kc - 1, groups=h.shape[-1])[..., :T].transpose(1, 2)


def prior_mass(log_w):
    """w = exp(clamp(log_w, -7, 12)) (model.py:74-75)."""
    return log_w.clamp(-7.0, 12.0).exp()


def decay_log(log_rate):
    """g = -exp(log_rate), so lam = exp(g) (model.py:84, 104)."""
    return -log_rate.exp()


def round_bf16(x):
    """x rounded to bf16 in the forward, the identity in the backward: the
    value of a bf16 operand with an exact gradient."""
    return x + (x.to(torch.bfloat16).to(x.dtype) - x).detach()


class _RoundGradBf16(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        return x.view_as(x)

    @staticmethod
    def backward(ctx, g):
        return g.to(torch.bfloat16).to(g.dtype)


def round_grad_bf16(x):
    """The identity in the forward; the gradient arriving at x is rounded to
    bf16 on its way back: the gradient of a tensor stored in bf16."""
    return _RoundGradBf16.apply(x)


def block_forward(p, prefix, x, norm_eps=1e-5, form="chunked", chunk=64, autocast=False):
    """UnifiedBlock.forward with the fast read replaced by a reference form
    (model.py:77-85, test_all.py:64-72). ``p`` maps state_dict names to tensors.

    autocast=True keeps the arithmetic exact but rounds to bf16 what bf16
    autocast rounds around the block's GEMMs (train.py trains under
    torch.autocast(bfloat16)). In the forward: the conv output u, both
    operands of the key, value and mu products, and the key and value
    outputs; the key bias is added after the rounding and the mu product's
    output stays unrounded, as the fused block computes them. In the
    backward, the gradients of the tensors held in bf16: of the key and value
    outputs, of the mu product's operand w q, and the block's upstream
    gradient as the mu product and the fast memory receive it (the residual
    path keeps it exact). Every other gradient passes the roundings
    unchanged."""
    g = lambda n: p[prefix + n]
    rnd = round_bf16 if autocast else (lambda t: t)
    rgr = round_grad_bf16 if autocast else (lambda t: t)
    h = rmsnorm(x, g("norm.weight"), norm_eps)
    u = rnd(causal_conv(h, g("conv.weight")))
    pre = rgr(rnd(F.linear(rnd(u), rnd(g("key.weight")))))
    r = address(pre + g("key.bias"), g("log_eps"))
    v = rgr(rnd(F.linear(rnd(h), rnd(g("val.weight")))))
    w = prior_mass(g("log_w"))
    q, fast = fast_memory(r, v, decay_log(g("log_rate")), w, form, chunk)
    return x + rgr(F.linear(rgr(rnd(q * w)), rnd(g("mu.weight"))) + fast)


def n_layers_of(p):
    return 1 + max(int(k.split(".")[1]) for k in p if k.startswith("layers."))


def lm_forward(p, tokens, targets=None, norm_eps=1e-5, form="chunked", chunk=64, autocast=False):
    """UnifiedLM.forward in a reference form (test_all.py:64-75, model.py:149-162).
    Returns (logits, loss); the classifier is tied to the embedding (model.py:127).
    autocast: the blocks' bf16 roundings as in block_forward."""
    emb = p["tok_embeddings.weight"]
    h = emb[tokens]
    for i in range(n_layers_of(p)):
        h = block_forward(p, f"layers.{i}.", h, norm_eps, form, chunk, autocast)
    logits = F.linear(rmsnorm(h, p["norm.weight"], norm_eps), p.get("output.weight", emb))
    loss = None
    if targets is not None:
        loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]), targets.reshape(-1), ignore_index=-1)
    return logits, loss


# ---------------------------------------------------------------------------
# the block-pair evaluation's bf16 roundings, in otherwise exact arithmetic

PAIR_ROUNDINGS = frozenset({"qk", "P", "v", "dfast", "dS", "qk_bwd"})


def _rb(x, on):
    return x.to(torch.bfloat16).to(x.dtype) if on else x


def pair_form_grads(r, v, g, w, dq_out, dfast, roundings=PAIR_ROUNDINGS):
    """(q, fast, dr, dv, dg, dw) of <q, dq_out> + <fast, dfast> as the block-pair
    products evaluate them, each operand the products read in bf16 rounded to
    bf16 (the ones named in ``roundings``) and every other step exact:

      "qk"      q and k in the scores P = lam^(t-s) (q_t . k_s)
      "P"       P in the apply and dv products; the decay gradient's pair sum
                weights with P + bf16(P - bf16(P)) (16 significant bits)
      "v"       v in the apply and dscores products
      "dfast"   dfast in the dscores and dv products
      "dS"      dS = lam^(t-s) (dfast_t . v_s) in the dq_f and dk_f products
      "qk_bwd"  k and q in the dq_f and dk_f products

    The gradients are the closed forms of the definition (kernel.py:139-180,
    summed directly over pairs for the decay): dq_f = dS k, dk_f = dS^T q,
    dv = P^T dfast, dc = -dq q / c, dk_c = M^T dc, dr_t = dq_t / c_t +
    (dk_f + dk_c)_{t+1}, dw = sum dc, dg = sum (t-s) P[t][s] (dfast_t . v_s) +
    sum dc (sum_s (t-s) lam^(t-s) k_s). With no roundings they equal float64
    autograd of dense_fast_memory (tests/test_oracle.py)."""
    r, v, g, w, dfast = (x.detach().double() for x in (r, v, g, w, dfast))
    R = set(roundings)
    lam = torch.exp(g)
    T = r.shape[1]
    k = shift_keys(r)
    M = decay_mask(T, lam).to(r.device)
    t = torch.arange(T, dtype=torch.float64, device=r.device)
    lagM = (t[:, None] - t[None, :]).clamp(min=0) * M
    c = w + M @ k
    q = r / c
    P = (_rb(q, "qk" in R) @ _rb(k, "qk" in R).transpose(1, 2)) * M
    P_hi = _rb(P, "P" in R)
    P_dg = P_hi + _rb(P - P_hi, "P" in R) if "P" in R else P
    V, DO = _rb(v, "v" in R), _rb(dfast, "dfast" in R)
    fast = P_hi @ V
    dots = DO @ V.transpose(1, 2)                    # dfast_t . v_s
    dS = _rb(dots * M, "dS" in R)
    dq_f = dS @ _rb(k, "qk_bwd" in R)
    dk_f = dS.transpose(1, 2) @ _rb(q, "qk_bwd" in R)
    dv = P_hi.transpose(1, 2) @ DO
    dq = dq_f + (dq_out.detach().double() if dq_out is not None else 0.0)
    dc = -dq * q / c
    dk = dk_f + M.transpose(0, 1) @ dc
    dr = dq / c
    dr[:, :-1] += dk[:, 1:]
    dg = ((t[:, None] - t[None, :]) * P_dg * dots).sum() + (dc * (lagM @ k)).sum()
    return q, fast, dr, dv, dg, dc.sum((0, 1))


class _PairForm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, r, v, g, w, roundings):
        ctx.save_for_backward(r, v, g, w)
        ctx.roundings = roundings
        q, fast = pair_form_grads(r, v, g, w, None, torch.zeros_like(v), roundings)[:2]
        return q.to(r.dtype), fast.to(r.dtype)

    @staticmethod
    def backward(ctx, dq, dfast):
        r, v, g, w = ctx.saved_tensors
        if dfast is None:
            dfast = torch.zeros_like(v)
        _, _, dr, dv, dg, dw = pair_form_grads(r, v, g, w, dq, dfast, ctx.roundings)
        return dr.to(r.dtype), dv.to(v.dtype), dg.to(g.dtype).reshape(g.shape), dw.to(w.dtype), None


def pair_form(r, v, g, w, roundings=PAIR_ROUNDINGS):
    """unified_memory(r, v, g, w) -> (q, fast) as the block-pair products
    evaluate it (pair_form_grads), differentiable in r, v, g, w."""
    return _PairForm.apply(r, v, g, w, frozenset(roundings))


# ---------------------------------------------------------------------------
# token-by-token decode (model.py:87-111, 164-175; run.c:193-265)

def init_state(p, prefix, batch):
    """Decode state at the prior (model.py:88-94, run.c:121-138):
    U = mu * w, c = w, r_prev = 0, empty conv buffer."""
    mu = p[prefix + "mu.weight"]
    w = prior_mass(p[prefix + "log_w"])
    D, A = mu.shape
    Kc = p[prefix + "conv.weight"].shape[-1]
    return {"buf": mu.new_zeros(batch, D, Kc - 1),
            "U": (mu * w).expand(batch, D, A).clone(),
            "c": w.expand(batch, A).clone(),
            "r_prev": mu.new_zeros(batch, A)}


def block_step(p, prefix, x, s, norm_eps=1e-5):
    """One position of UnifiedBlock.step (model.py:96-111): write under the
    previous address with decay toward the prior, then read with q = r / c."""
    g = lambda n: p[prefix + n]
    h = rmsnorm(x, g("norm.weight"), norm_eps)
    win = torch.cat([s["buf"], h[:, :, None]], dim=-1)
    u = (win * g("conv.weight")[:, 0, :]).sum(-1)
    s["buf"] = win[:, :, 1:]
    r = address(F.linear(u, g("key.weight"), g("key.bias")), g("log_eps"))
    lam = torch.exp(decay_log(g("log_rate")))
    v = F.linear(h, g("val.weight"))
    w = prior_mass(g("log_w"))
    mu = g("mu.weight")
    s["U"] = lam * s["U"] + (1 - lam) * mu * w + v[:, :, None] * s["r_prev"][:, None, :]
    s["c"] = lam * s["c"] + (1 - lam) * w + s["r_prev"]
    y = (s["U"] @ (r / s["c"])[:, :, None]).squeeze(-1)
    s["r_prev"] = r
    return x + y


def forward_recurrent(p, tokens, norm_eps=1e-5):
    """UnifiedLM.forward_recurrent (model.py:164-175): logits (B, T, V)."""
    B, T = tokens.shape
    L = n_layers_of(p)
    emb = p["tok_embeddings.weight"]
    states = [init_state(p, f"layers.{i}.", B) for i in range(L)]
    out = []
    for t in range(T):
        h = emb[tokens[:, t]]
        for i in range(L):
            h = block_step(p, f"layers.{i}.", h, states[i], norm_eps)
        out.append(F.linear(rmsnorm(h, p["norm.weight"], norm_eps), p.get("output.weight", emb)))
    return torch.stack(out, 1)


# ---------------------------------------------------------------------------
# seeded parameters

def tiny_params(seed=0, dim=32, n_layers=3, hidden_dim=48, vocab_size=97, max_seq_len=40,
                conv_size=4, prior=4.0, dtype=torch.float64):
    """Parameters with every path non-trivial, distributed like the reference's
    ``tiny_model`` fixture (test_all.py:78-90) on top of the UnifiedLM init
    (model.py:129-147): conv ~ N(0, .5^2), key bias ~ N(0, .5^2), val ~ N(0, .2^2),
    log_rate = log 0.05, log_w ~ N(0, 1). Values are this generator's own draws."""
    gen = torch.Generator().manual_seed(seed)
    n = lambda *shape, std=1.0: torch.randn(*shape, generator=gen, dtype=dtype) * std
    p = {"tok_embeddings.weight": n(vocab_size, dim, std=0.02)}
    for i in range(n_layers):
        pre = f"layers.{i}."
        p[pre + "norm.weight"] = torch.ones(dim, dtype=dtype)
        p[pre + "conv.weight"] = n(dim, 1, conv_size, std=0.5)
        p[pre + "key.weight"] = n(hidden_dim, dim, std=0.02)
        p[pre + "key.bias"] = n(hidden_dim, std=0.5)
        p[pre + "mu.weight"] = n(dim, hidden_dim, std=0.02 / math.sqrt(n_layers))
        p[pre + "log_eps"] = torch.zeros((), dtype=dtype)
        p[pre + "val.weight"] = n(dim, dim, std=0.2)
        p[pre + "log_rate"] = torch.tensor(math.log(0.05), dtype=dtype)
        p[pre + "log_w"] = n(hidden_dim, std=1.0)
    p["norm.weight"] = torch.ones(dim, dtype=dtype)
    return p
