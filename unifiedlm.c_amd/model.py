"""UnifiedLM with the fast-memory path on MI355X HIP kernels.

Same call surface, module tree and parameter names as the reference's
model.py (model.py:13-222), so state dicts and checkpoints are interchangeable
and seeded construction draws the same initial weights. What changes:

  * UnifiedBlock.code runs the fused relu^2 address kernel on the key GEMM
    output (model.py:70-72);
  * UnifiedBlock.forward calls kernel.unified_memory, backed by libulm_fm.so
    (model.py:84);
  * UnifiedBlock.step / UnifiedLM.forward_recurrent run the batched decode
    kernels (model.py:96-111, 164-175). The per-block state holds the slot
    contents as S = U - mu*w (so S_t = lam S_{t-1} + v_t r_{t-1}^T) with the
    evidence mass c = w + n, the previous address and the conv window.
"""
import inspect
import math
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from kernel import (CHUNK, LOG_W_MAX, LOG_W_MIN, block_prefill, decode_addr, decode_pre, decode_state, fm_prefill,
                    relu2_address, unified_block, unified_memory)


@dataclass
class ModelArgs:
    dim: int = 288
    n_layers: int = 12          # number of UnifiedBlocks
    hidden_dim: int = 712       # memory slots per block
    vocab_size: int = 32000
    max_seq_len: int = 256
    norm_eps: float = 1e-5
    dropout: float = 0.0
    conv_size: int = 4          # causal depthwise conv on the address path
    prior: float = 4.0          # initial prior mass w of every slot, in tokens


def _hi(x):
    """Slot statistics stay in fp32 even under bf16/fp16 autocast (model.py:26-28)."""
    return x.float() if x.dtype in (torch.float16, torch.bfloat16) else x


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def _norm(self, x):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps)

    def forward(self, x):
        return self._norm(_hi(x)).type_as(x) * self.weight


class UnifiedBlock(nn.Module):
    """One associative memory whose slots hold running posterior means:

        address  r_t = normalize(relu(K u_t + b)^2),  u_t = causal depthwise conv(RMSNorm(x_t))
        write    key r_{t-1}, value v_t = W_v h_t
        read     y_t = sum_a r_t,a (w_a mu_a + S_t,a) / (w_a + n_t,a)
    """

    def __init__(self, args: ModelArgs):
        super().__init__()
        d, m = args.dim, args.hidden_dim
        self.norm = RMSNorm(d, eps=args.norm_eps)
        self.conv = nn.Conv1d(d, d, args.conv_size, groups=d, padding=args.conv_size - 1, bias=False)
        self.key = nn.Linear(d, m, bias=True)
        self.mu = nn.Linear(m, d, bias=False)
        self.log_eps = nn.Parameter(torch.zeros(()))
        self.val = nn.Linear(d, d, bias=False)
        self.log_rate = nn.Parameter(torch.tensor(math.log(1.0 / (4 * args.max_seq_len))))
        self.log_w = nn.Parameter(torch.full((m,), math.log(args.prior)))
        self.dropout = nn.Dropout(args.dropout)

    def code(self, u):
        """relu^2 address; the key bias is added in fp32 inside the kernel."""
        return relu2_address(F.linear(u, self.key.weight), self.key.bias, self.log_eps)

    def _w(self):
        return self.log_w.clamp(LOG_W_MIN, LOG_W_MAX).exp()

    def forward(self, x):
        """model.py:77-85. One fused block (fast memory, RMSNorm + conv, address,
        w q and the residual in native kernels around the library GEMMs) for an
        fp32 residual stream; GEMM operands take the autocast dtype, as the
        reference's bf16-autocast training step runs them (train.py)."""
        if x.dtype != torch.float32 or (self.training and self.dropout.p > 0):
            return self.forward_composed(x)
        cdt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else torch.float32
        with torch.autocast("cuda", enabled=False):
            return unified_block(x, self.norm.weight, self.conv.weight, self.key.weight, self.key.bias,
                                 self.log_eps, self.val.weight, self.mu.weight, self.log_rate, self.log_w,
                                 self.norm.eps, cdt)

    def forward_composed(self, x):
        """The same block op by op (model.py:77-85): the fast memory and the
        address in native kernels, the rest in torch; the path for dropout and
        for a non-fp32 residual stream."""
        h = self.norm(x)
        u = self.conv(h.transpose(1, 2))[..., : h.size(1)].transpose(1, 2)
        r = self.code(u)
        v = self.val(h)
        w = self._w()
        q, fast = unified_memory(r, v, -self.log_rate.exp(), w)
        return x + self.dropout(self.mu((q * w).type_as(x)) + fast.type_as(x))

    # ---- token-by-token form (model.py:87-111)
    @torch.no_grad()
    def _step_params(self, device):
        """The fp32 views of the parameters that every step uses (taken once per
        decode session: the weights do not change while a session decodes)."""
        f = lambda t: t.detach().to(device=device, dtype=torch.float32).contiguous()
        return {"norm_w": f(self.norm.weight), "conv_w": f(self.conv.weight[:, 0, :]), "key_wt": f(self.key.weight.t()),
                "key_b": f(self.key.bias), "log_eps": f(self.log_eps).reshape(1), "val_wt": f(self.val.weight.t()),
                "mu_wt": f(self.mu.weight.t()), "w": f(self._w()), "g": f(-self.log_rate.exp()).reshape(1)}

    @torch.no_grad()
    def init_state(self, batch: int, device):
        """Decode state of one block before any position, plus its parameter views."""
        d, m = self.mu.out_features, self.mu.in_features
        kw = self.conv.kernel_size[0] - 1
        params = self._step_params(device)
        return {"buf": torch.zeros(batch, d, kw, device=device, dtype=torch.float32),
                "S": torch.zeros(batch, d, m, device=device, dtype=torch.float32),
                "c": params["w"].expand(batch, m).clone(),   # updated in place: never a view of w
                "r_prev": torch.zeros(batch, m, device=device, dtype=torch.float32),
                "params": params}

    @torch.no_grad()
    def prefill(self, x):
        """`forward` over a whole prompt x (B, T, d) in one chunked pass, also
        returning the decode state after position T-1: the state that T calls of
        `step` would leave (model.py:88-111), with S and c from the chunked
        kernels (bf16 operands, fp32 accumulation) instead of T fp32 updates.
        With an fp32 x the block runs fused (kernel.block_prefill), its GEMMs in
        the autocast dtype."""
        B, T, d = x.shape
        A = self.mu.in_features
        if x.dtype == torch.float32:
            cdt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else torch.float32
            with torch.autocast("cuda", enabled=False):
                out, S, c, r_prev, h = block_prefill(x, self.norm.weight, self.conv.weight, self.key.weight,
                                                     self.key.bias, self.log_eps, self.val.weight, self.mu.weight,
                                                     self.log_rate, self.log_w, self.norm.eps, cdt)
        else:
            w = self._w()
            g = -self.log_rate.exp()
            h = self.norm(x)
            u = self.conv(h.transpose(1, 2))[..., : h.size(1)].transpose(1, 2)
            r = self.code(u)
            v = self.val(h)
            q, fast, S, c = fm_prefill(r, v, g, w)
            out = x + self.mu((q * w).type_as(x)) + fast.type_as(x)
            r_prev = r[:, -1, :].float().contiguous()
        kw = self.conv.kernel_size[0] - 1
        buf = torch.zeros(B, d, kw, device=x.device, dtype=torch.float32)
        if kw > 0:
            tail = h[:, max(0, T - kw):, :].float().transpose(1, 2)   # the last (up to) kw positions, oldest first
            buf[:, :, kw - tail.size(-1):] = tail
        state = {"buf": buf, "S": S, "c": c, "r_prev": r_prev, "params": self._step_params(x.device)}
        return out, state

    @torch.no_grad()
    def step(self, x, s):
        """x: (B, d), one position. Write (key r_{t-1}, value v_t), then read."""
        p = s["params"]
        x32 = x.float().contiguous()
        h, u = decode_pre(x32, p["norm_w"], p["conv_w"], s["buf"], self.norm.eps)
        pre = u @ p["key_wt"]
        v = h @ p["val_wt"]
        r, q, wq = decode_addr(pre, p["key_b"], p["log_eps"], p["w"], p["g"], s["r_prev"], s["c"])
        ymu = wq @ p["mu_wt"]
        out = decode_state(s["S"], v, s["r_prev"], q, p["g"], x32, ymu)
        s["r_prev"] = r
        return out.to(x.dtype)


class UnifiedLM(nn.Module):
    last_loss: Optional[torch.Tensor]

    def __init__(self, params: ModelArgs):
        super().__init__()
        self.params = params
        self.tok_embeddings = nn.Embedding(params.vocab_size, params.dim)
        self.dropout = nn.Dropout(params.dropout)
        self.layers = nn.ModuleList([UnifiedBlock(params) for _ in range(params.n_layers)])
        self.norm = RMSNorm(params.dim, eps=params.norm_eps)
        self.output = nn.Linear(params.dim, params.vocab_size, bias=False)
        self.tok_embeddings.weight = self.output.weight

        self.apply(self._init_weights)
        for pn, p in self.named_parameters():
            if pn.endswith("mu.weight"):
                nn.init.normal_(p, mean=0.0, std=0.02 / math.sqrt(params.n_layers))
            elif pn.endswith("val.weight"):
                nn.init.zeros_(p)
            elif pn.endswith("conv.weight"):
                with torch.no_grad():
                    p.zero_()
                    p[:, 0, -1] = 1.0
        self.last_loss = None

    def _init_weights(self, module):
        if isinstance(module, nn.Linear):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def forward(self, tokens: torch.Tensor, targets: Optional[torch.Tensor] = None) -> torch.Tensor:
        h = self.dropout(self.tok_embeddings(tokens))
        for layer in self.layers:
            h = layer(h)
        h = self.norm(h)
        if targets is not None:
            logits = self.output(h)
            self.last_loss = F.cross_entropy(logits.view(-1, logits.size(-1)), targets.view(-1), ignore_index=-1)
        else:
            logits = self.output(h[:, [-1], :])
            self.last_loss = None
        return logits

    def init_states(self, batch: int, device):
        return [layer.init_state(batch, device) for layer in self.layers]

    @torch.no_grad()
    def prefill(self, tokens: torch.Tensor):
        """A prompt (B, T) in one chunked pass: returns the logits of its last
        position (B, V) and the per-block decode states, from which `step`
        continues exactly as after T calls of `step`."""
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
        one chunked pass (`prefill`) instead of
        T0 calls of `step`."""
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
        """Token-by-token inference with constant state per block, exactly what run.c computes."""
        B, T = tokens.shape
        states = self.init_states(B, tokens.device)
        return torch.stack([self.step(tokens[:, t], states) for t in range(T)], dim=1)

    def configure_optimizers(self, weight_decay, learning_rate, betas, device_type):
        param_dict = {pn: p for pn, p in self.named_parameters() if p.requires_grad}
        decay_params = [p for n, p in param_dict.items() if p.dim() >= 2]
        nodecay_params = [p for n, p in param_dict.items() if p.dim() < 2]
        optim_groups = [
            {"params": decay_params, "weight_decay": weight_decay},
            {"params": nodecay_params, "weight_decay": 0.0},
        ]
        fused_available = "fused" in inspect.signature(torch.optim.AdamW).parameters
        extra_args = dict(fused=True) if fused_available and device_type == "cuda" else dict()
        return torch.optim.AdamW(optim_groups, lr=learning_rate, betas=betas, **extra_args)

    def estimate_mfu(self, fwdbwd_per_iter, dt):
        """Model flops utilisation in units of A100 bf16 peak (model.py:196-204)."""
        N = sum(p.numel() for p in self.parameters())
        cfg = self.params
        T, m, d = cfg.max_seq_len, cfg.hidden_dim, cfg.dim
        mix = min(CHUNK, T) * (2 * m + d) + 2 * m * d
        flops_per_token = 6 * N + 6 * cfg.n_layers * mix
        return flops_per_token * T * fwdbwd_per_iter * (1.0 / dt) / 312e12

    @torch.inference_mode()
    def generate(self, idx, max_new_tokens, temperature=1.0, top_k=None):
        for _ in range(max_new_tokens):
            idx_cond = idx if idx.size(1) <= self.params.max_seq_len else idx[:, -self.params.max_seq_len:]
            logits = self(idx_cond)[:, -1, :]
            if temperature == 0.0:
                _, idx_next = torch.topk(logits, k=1, dim=-1)
            else:
                logits = logits / temperature
                if top_k is not None:
                    v, _ = torch.topk(logits, min(top_k, logits.size(-1)))
                    logits[logits < v[:, [-1]]] = -float("Inf")
                idx_next = torch.multinomial(F.softmax(logits, dim=-1), num_samples=1)
            idx = torch.cat((idx, idx_next), dim=1)
        return idx
