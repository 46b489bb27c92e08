"""UnifiedLM on the MI355X fast-memory kernels.

What is kept from the reference (model.py:13-175) is its interface only: the
class names, ModelArgs' fields and defaults, the module tree and parameter
names (state dicts interchange), the initial values, and the order in which
construction draws from the default RNG (a seeded construction yields the same
weights). Every body here is this package's own:

  * UnifiedBlock.forward is one fused block (kernel.unified_block): RMSNorm and
    the causal conv, the relu^2 address, the fast memory, w q and the residual
    in native kernels around the library GEMMs (model.py:77-85);
  * step / forward_recurrent run the batched decode kernels (model.py:96-111,
    164-175) on a state that holds the slot contents as S = U - mu w (so
    S_t = lam S_{t-1} + v_t r_{t-1}^T), the evidence c = w + n, the previous
    address and the conv window;
  * prefill runs a prompt in one chunked pass and leaves the decode state.

The reference's training-loop and sampling helpers keep their signatures
(configure_optimizers, estimate_mfu, generate: train.py:172, 295, sample.py:61)
with bodies of this package's own; generate samples on the decode kernels.
"""
import inspect
import math
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from kernel import (CHUNK, LOG_W_MAX, LOG_W_MIN, block_prefill, decode_addr, decode_addr_deferred, decode_deferred,
                    decode_pre, decode_state,
                    fm_prefill,
                    relu2_address, unified_block, unified_memory)


@dataclass
class ModelArgs:
    """Hyperparameters under the reference's field names (model.py:13-23):
    residual width `dim`, `n_layers` blocks of `hidden_dim` memory slots each,
    `conv_size` taps of the address path's causal depthwise conv, and `prior`,
    every slot's initial prior mass w in tokens."""
    dim: int = 288
    n_layers: int = 12
    hidden_dim: int = 712
    vocab_size: int = 32000
    max_seq_len: int = 256
    norm_eps: float = 1e-5
    dropout: float = 0.0
    conv_size: int = 4
    prior: float = 4.0


def _compute_dtype():
    """The GEMM operand dtype of the fused block: autocast's when it is on."""
    return torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else torch.float32


class RMSNorm(nn.Module):
    """x / sqrt(mean(x^2) + eps) * weight over the last dimension
    (model.py:31-42), evaluated in fp32 for any input dtype and returned in it."""

    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x):
        x32 = x.float()
        scaled = x32 * torch.rsqrt(x32.square().mean(dim=-1, keepdim=True) + self.eps)
        return scaled.to(x.dtype) * self.weight


# write terms a decode state holds before it writes S back (at most
# ulm_decode_max_pending(), 16)
DECODE_PENDING = 16


class UnifiedBlock(nn.Module):
    """An associative memory with posterior-mean slots:

        address  r_t = relu(K u_t + b)^2 / (eps + sum relu(.)^2),  u_t = conv(RMSNorm(x_t))
        write    under key r_{t-1} the value v_t = W_v h_t, decaying by lam = exp(-exp(log_rate))
        read     y_t = sum_a r_t,a (w_a mu_a + S_t,a) / (w_a + n_t,a),  w = exp(clamp(log_w))
    """

    def __init__(self, args: ModelArgs):
        super().__init__()
        width, slots, taps = args.dim, args.hidden_dim, args.conv_size
        # registered in the reference's order (model.py:59-68): the submodules'
        # default initialisations draw from the RNG in this order, and
        # parameters() / state_dict() list the same names in the same order
        # (a module's own parameters before its submodules'), so optimizer
        # states keyed by position carry over. The memory's own parameters are
        # the implicit null slot (log eps), the forgetting rate
        # (1 / (4 max_seq_len)) and the prior mass.
        self.norm = RMSNorm(width, eps=args.norm_eps)
        self.conv = nn.Conv1d(width, width, taps, padding=taps - 1, groups=width, bias=False)
        self.key = nn.Linear(width, slots)
        self.mu = nn.Linear(slots, width, bias=False)
        self.log_eps = nn.Parameter(torch.zeros(()))
        self.val = nn.Linear(width, width, bias=False)
        self.log_rate = nn.Parameter(torch.tensor(-math.log(4.0 * args.max_seq_len)))
        self.log_w = nn.Parameter(torch.full((slots,), math.log(args.prior)))
        self.dropout = nn.Dropout(args.dropout)

    def code(self, u):
        """The relu^2 address of u (model.py:70-72); the key bias is added in
        fp32 inside the address kernel."""
        return relu2_address(F.linear(u, self.key.weight), self.key.bias, self.log_eps)

    def _w(self):
        return torch.exp(torch.clamp(self.log_w, LOG_W_MIN, LOG_W_MAX))

    def _decay_log(self):
        return -torch.exp(self.log_rate)

    def forward(self, x):
        """One fused block for an fp32 residual stream; its GEMM operands take
        the autocast dtype, as the reference's bf16-autocast training step runs
        them (train.py). Dropout in training and other residual dtypes take the
        composed path."""
        if x.dtype != torch.float32 or (self.training and self.dropout.p > 0):
            return self.forward_composed(x)
        cdt = _compute_dtype()
        with torch.autocast("cuda", enabled=False):
            return unified_block(x, self.norm.weight, self.conv.weight, self.key.weight, self.key.bias,
                                 self.log_eps, self.val.weight, self.mu.weight, self.log_rate, self.log_w,
                                 self.norm.eps, cdt)

    def _address_and_value(self, x):
        """h = RMSNorm(x), its causal depthwise conv u, the address r of u and
        the value v of h."""
        h = self.norm(x)
        T = x.shape[1]
        u = F.conv1d(h.transpose(1, 2), self.conv.weight, padding=self.conv.padding, groups=self.conv.groups)
        u = u[..., :T].transpose(1, 2)
        return h, self.code(u), self.val(h)

    def forward_composed(self, x):
        """The block op by op around the native fast memory and address."""
        _, r, v = self._address_and_value(x)
        w = self._w()
        q, fast = unified_memory(r, v, self._decay_log(), w)
        read = self.mu((q * w).to(x.dtype)) + fast.to(x.dtype)
        return x + self.dropout(read)

    # ---- one position at a time (model.py:87-111)

    @torch.no_grad()
    def _step_params(self, device):
        """fp32 copies of what every step reads, in the layouts of the decode
        kernels (taken once per decode session: weights do not change while it
        decodes)."""
        def f32(t):
            return t.detach().to(device=device, dtype=torch.float32).contiguous()
        return {"norm_w": f32(self.norm.weight), "conv_w": f32(self.conv.weight[:, 0, :]),
                "key_wt": f32(self.key.weight.t()), "key_b": f32(self.key.bias),
                "log_eps": f32(self.log_eps).reshape(1), "val_wt": f32(self.val.weight.t()),
                "mu_wt": f32(self.mu.weight.t()), "w": f32(self._w()), "g": f32(self._decay_log()).reshape(1)}

    @torch.no_grad()
    def init_state(self, batch: int, device):
        """The decode state before the first position (S = 0, c = w, no
        previous address, an empty conv window) with the parameter copies."""
        width, slots = self.mu.out_features, self.mu.in_features
        params = self._step_params(device)
        zeros = lambda *shape: torch.zeros(*shape, device=device, dtype=torch.float32)
        return {"buf": zeros(batch, width, self.conv.kernel_size[0] - 1),
                "S": zeros(batch, width, slots),
                "c": params["w"].repeat(batch, 1),   # its own storage: the step updates it in place
                "r_prev": zeros(batch, slots),
                "params": params}

    @torch.no_grad()
    def prefill(self, x):
        """`forward` over a prompt x (B, T, d) in one chunked pass, returning
        with it the decode state after position T-1, the state T calls of
        `step` would leave (S and c from bf16 MFMA products with fp32
        accumulation instead of T fp32 updates). An fp32 x runs the fused
        block prefill, its GEMMs in the autocast dtype."""
        B, T, width = x.shape
        if x.dtype == torch.float32:
            cdt = _compute_dtype()
            with torch.autocast("cuda", enabled=False):
                out, S, c, r_prev, h = block_prefill(x, self.norm.weight, self.conv.weight, self.key.weight,
                                                     self.key.bias, self.log_eps, self.val.weight, self.mu.weight,
                                                     self.log_rate, self.log_w, self.norm.eps, cdt)
        else:
            h, r, v = self._address_and_value(x)
            w = self._w()
            q, fast, S, c = fm_prefill(r, v, self._decay_log(), w)
            out = x + self.mu((q * w).to(x.dtype)) + fast.to(x.dtype)
            r_prev = r[:, -1, :].float().contiguous()
        # the conv window: the last (up to) taps - 1 normalised inputs, oldest first
        kw = self.conv.kernel_size[0] - 1
        buf = torch.zeros(B, width, kw, device=x.device, dtype=torch.float32)
        n = min(kw, T)
        if n > 0:
            buf[:, :, kw - n:] = h[:, T - n:, :].float().transpose(1, 2)
        return out, {"buf": buf, "S": S, "c": c, "r_prev": r_prev, "params": self._step_params(x.device)}

    @torch.no_grad()
    def step(self, x, s):
        """One position x (B, d) for a batch of sequences: write (key r_{t-1},
        value v_t), then read with the new address.

        With slots a multiple of 4 (at most 4096) the write is deferred: the
        state holds S (its last written value) and up to DECODE_PENDING
        pending write terms (s["pv"], s["pr"], s["np"] of them); a position
        appends its term and reads S with the terms added, and the position
        that fills the last term writes S back with all of them. The maths of
        model.py:107-109 in another order: S moves one write per
        DECODE_PENDING positions instead of one per position."""
        p = s["params"]
        x32 = x.float().contiguous()
        h, u = decode_pre(x32, p["norm_w"], p["conv_w"], s["buf"], self.norm.eps)
        N, width, slots = s["S"].shape
        if slots % 4 or slots > 4096:
            r, q, wq = decode_addr(u @ p["key_wt"], p["key_b"], p["log_eps"], p["w"], p["g"], s["r_prev"], s["c"])
            out = decode_state(s["S"], h @ p["val_wt"], s["r_prev"], q, p["g"], x32, wq @ p["mu_wt"])
        else:
            if "pv" not in s:
                s["pv"] = torch.empty(DECODE_PENDING, N, width, device=x.device, dtype=torch.float32)
                s["pr"] = torch.empty(DECODE_PENDING, N, slots, device=x.device, dtype=torch.float32)
                s["np"] = 0
            m = s["np"]
            flush = m + 1 == DECODE_PENDING
            # appends r_prev as pending key m (and the terms' read-out weights unless this position writes back)
            r, q, wq, cj = decode_addr_deferred(u @ p["key_wt"], p["key_b"], p["log_eps"], p["w"], p["g"],
                                                s["r_prev"], s["c"], s["pr"], m, not flush)
            torch.mm(h, p["val_wt"], out=s["pv"][m])
            out = decode_deferred(s["S"], s["pv"], s["pr"], m + 1, flush, q, p["g"], x32, wq @ p["mu_wt"], cj)
            s["np"] = 0 if flush else m + 1
        s["r_prev"] = r
        return out.to(x.dtype)

    @torch.no_grad()
    def flush_state(self, s):
        """Writes a deferred decode state's pending terms into s["S"] (S <- S_t,
        no pending terms left), so that s["S"] is the state after the last
        position `step` took; a no-op when nothing is pending."""
        m = s.get("np", 0)
        if not m:
            return s
        p = s["params"]
        N, width, slots = s["S"].shape
        zeros = torch.zeros(N, slots, device=s["S"].device, dtype=torch.float32)
        x0 = torch.zeros(N, width, device=s["S"].device, dtype=torch.float32)
        decode_deferred(s["S"], s["pv"], s["pr"], m, True, zeros, p["g"], x0, x0)   # the read-out is discarded
        s["np"] = 0
        return s


class UnifiedLM(nn.Module):
    """Token embedding, `n_layers` UnifiedBlocks, a final RMSNorm and a
    classifier tied to the embedding (model.py:114-162)."""
    last_loss: Optional[torch.Tensor]

    def __init__(self, params: ModelArgs):
        super().__init__()
        self.params = params
        self.tok_embeddings = nn.Embedding(params.vocab_size, params.dim)
        self.dropout = nn.Dropout(params.dropout)
        self.layers = nn.ModuleList(UnifiedBlock(params) for _ in range(params.n_layers))
        self.norm = RMSNorm(params.dim, eps=params.norm_eps)
        self.output = nn.Linear(params.dim, params.vocab_size, bias=False)
        self.tok_embeddings.weight = self.output.weight   # one (vocab, dim) matrix for both
        self._initialise(params.n_layers)
        self.last_loss = None

    @torch.no_grad()
    def _initialise(self, n_layers):
        """The reference's initial values and RNG draw order (model.py:129-147):
        every linear and embedding weight N(0, 0.02^2) in module order (the
        tied matrix twice) and linear biases zero; then each block's mu weight
        N(0, (0.02 / sqrt(n_layers))^2), its value weight zero (an empty fast
        store) and its conv the identity (u_t = h_t)."""
        for mod in self.modules():
            if isinstance(mod, (nn.Linear, nn.Embedding)):
                mod.weight.normal_(0.0, 0.02)
                if getattr(mod, "bias", None) is not None:
                    mod.bias.zero_()
        for layer in self.layers:
            layer.mu.weight.normal_(0.0, 0.02 / math.sqrt(n_layers))
            layer.val.weight.zero_()
            layer.conv.weight.zero_()
            layer.conv.weight[:, 0, -1] = 1.0

    def forward(self, tokens: torch.Tensor, targets: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Logits (B, T, V) and the cross-entropy in last_loss (targets -1
        ignored) with targets; without them the last position's logits
        (B, 1, V) and last_loss None."""
        h = self.dropout(self.tok_embeddings(tokens))
        for layer in self.layers:
            h = layer(h)
        h = self.norm(h)
        if targets is None:
            self.last_loss = None
            return self.output(h[:, -1:, :])
        logits = self.output(h)
        self.last_loss = F.cross_entropy(logits.flatten(0, 1), targets.flatten(), ignore_index=-1)
        return logits

    def init_states(self, batch: int, device):
        return [layer.init_state(batch, device) for layer in self.layers]

    def flush_states(self, states):
        """Every block's decode state written back (UnifiedBlock.flush_state)."""
        for layer, s in zip(self.layers, states):
            layer.flush_state(s)
        return states

    @torch.no_grad()
    def prefill(self, tokens: torch.Tensor):
        """A prompt (B, T) in one chunked pass: the logits of its last position
        (B, V) and the per-block decode states, from which `step` continues
        exactly as after T calls of `step`."""
        h = self.tok_embeddings(tokens)
        states = []
        for layer in self.layers:
            h, s = layer.prefill(h)
            states.append(s)
        return self.output(self.norm(h[:, -1, :])), states

    @torch.no_grad()
    def step(self, tokens: torch.Tensor, states) -> torch.Tensor:
        """One position for a batch of sequences: tokens (B,) -> logits (B, V)."""
        h = self.tok_embeddings(tokens)
        for layer, s in zip(self.layers, states):
            h = layer.step(h, s)
        return self.output(self.norm(h))

    @torch.no_grad()
    def decode_greedy(self, prompt: torch.Tensor, steps: int, prefill: bool = True) -> torch.Tensor:
        """The generate loop of the reference's C decoder at temperature 0
        (run.c:542-571, without its BOS stop): positions 0 .. steps-1 are run,
        the prompt (B, T0) is forced and every later token is the argmax of the
        previous position's logits (first maximum on ties, run.c:460-469).
        Returns (B, steps + 1) tokens. With `prefill` the prompt goes through
        one chunked pass (`prefill`) instead of T0 calls of `step`."""
        B, T0 = prompt.shape
        if steps < T0:
            raise ValueError(f"steps={steps} is shorter than the prompt ({T0})")
        if prefill:
            logits, states = self.prefill(prompt)
        else:
            states = self.init_states(B, prompt.device)
            for t in range(T0):
                logits = self.step(prompt[:, t], states)
        out = [prompt]
        for pos in range(T0 - 1, steps):
            nxt = logits.argmax(-1)
            out.append(nxt[:, None])
            if pos + 1 < steps:
                logits = self.step(nxt, states)
        return torch.cat(out, 1)

    @torch.no_grad()
    def forward_recurrent(self, tokens: torch.Tensor) -> torch.Tensor:
        """Logits (B, T, V) position by position on the decode kernels, with a
        constant-size state per block: what run.c computes (model.py:164-175)."""
        states = self.init_states(tokens.shape[0], tokens.device)
        return torch.stack([self.step(tokens[:, t], states) for t in range(tokens.shape[1])], dim=1)

    # ---- the training loop's and the sampler's helpers (train.py:172, 295; sample.py:61)

    def configure_optimizers(self, weight_decay, learning_rate, betas, device_type):
        """AdamW over two groups: weight decay on the matrices (every parameter
        of two or more dimensions: embedding, key, mu, value and conv weights),
        none on the vectors and scalars (norm weights, key biases, log_eps,
        log_rate, log_w), in parameters() order (model.py:177-194). The fused
        AdamW kernel is used on a GPU when this torch provides it."""
        params = [p for p in self.parameters() if p.requires_grad]
        matrices = [p for p in params if p.dim() >= 2]
        vectors = [p for p in params if p.dim() < 2]
        print(f"num decayed parameter tensors: {len(matrices)}, with {sum(p.numel() for p in matrices):,} "
              "parameters")
        print(f"num non-decayed parameter tensors: {len(vectors)}, with {sum(p.numel() for p in vectors):,} "
              "parameters")
        fused = device_type == "cuda" and "fused" in inspect.signature(torch.optim.AdamW).parameters
        groups = [{"params": matrices, "weight_decay": weight_decay}, {"params": vectors, "weight_decay": 0.0}]
        optimizer = torch.optim.AdamW(groups, lr=learning_rate, betas=betas, **({"fused": True} if fused else {}))
        print(f"using fused AdamW: {fused}")
        return optimizer

    def estimate_mfu(self, fwdbwd_per_iter, dt, peak_flops=2516.6e12):
        """Model flops utilisation of one iteration of fwdbwd_per_iter sequences
        of max_seq_len tokens taking dt seconds. The model flops per token are
        the reference's count (model.py:196-203): 6 per parameter, plus per
        block 6 (min(CHUNK, T) (2 A + D) + 2 A D) for the chunk-local mixing
        and the carried state. The reference divides by the A100's bf16 peak
        (312 TFLOP/s); here the default is the MI355X's dense bf16 peak."""
        n_params = sum(p.numel() for p in self.parameters())
        cfg = self.params
        T, A, D = cfg.max_seq_len, cfg.hidden_dim, cfg.dim
        mixing = min(CHUNK, T) * (2 * A + D) + 2 * A * D
        per_token = 6 * n_params + 6 * cfg.n_layers * mixing
        return per_token * T * fwdbwd_per_iter / dt / peak_flops

    @torch.inference_mode()
    def generate(self, idx, max_new_tokens, temperature=1.0, top_k=None):
        """Appends max_new_tokens sampled tokens to idx (B, T0) (model.py:205-222):
        each is drawn from the last position's logits over at most max_seq_len
        preceding tokens, divided by temperature and cut to the top_k largest
        (temperature 0: the argmax). While the context fits max_seq_len the
        sequences are decoded recurrently (one chunked prefill, then one
        decode step per token), which gives the logits of a full forward over
        the same context; once it slides, each token re-reads the window of
        the last max_seq_len tokens in one chunked pass."""
        window = self.params.max_seq_len
        states = None
        for _ in range(max_new_tokens):
            if states is None or idx.size(1) > window:
                logits, states = self.prefill(idx[:, -window:])
            nxt = self._sample(logits.float(), temperature, top_k)
            idx = torch.cat((idx, nxt), dim=1)
            if idx.size(1) <= window:
                logits = self.step(nxt[:, 0], states)
        return idx

    @staticmethod
    def _sample(logits, temperature, top_k):
        if temperature == 0.0:
            return logits.argmax(-1, keepdim=True)
        logits = logits / temperature
        if top_k is not None:
            kth = torch.topk(logits, min(top_k, logits.size(-1))).values[:, -1:]
            logits = logits.masked_fill(logits < kth, -float("inf"))
        return torch.multinomial(torch.softmax(logits, dim=-1), num_samples=1)
