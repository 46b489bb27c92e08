"""UnifiedBlock's fast memory on MI355X: the operator surface of the reference's
kernel.py (kernel.py:1-15, 199-238), computed by hand-written gfx950 HIP
kernels in libulm_fm.so.

unified_memory(r, v, g, w) -> (q, fast), for every batch row and position t:

    k_t    = r_{t-1}                                     (k_0 = 0, write address)
    c_t    = w + sum_{s<=t} lam^(t-s) k_s                (slot evidence mass, lam = exp(g))
    q_t    = r_t / c_t
    fast_t = sum_{s<=t} lam^(t-s) (q_t . k_s) v_s

Matmul operands are bf16 with fp32 accumulation and an fp32 chunk state kept
on chip; c, q and all their gradients are fp32, as in the reference.

Besides the operator this module exposes the relu^2 slot address
(model.py:70-72) as an autograd Function and the three per-token decode
kernels used by UnifiedBlock.step.
"""
from typing import Optional

import torch

import ulm_native as nat
from ulm_native import call, ptr

CHUNK = 64          # kernel.py:20


def _check_float(name, t):
    if not torch.is_floating_point(t):
        raise TypeError(f"{name} must be a floating tensor, got {t.dtype}")


def _check_fm(r, v, g, w):
    for name, t in (("r", r), ("v", v), ("g", g), ("w", w)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a tensor")
        _check_float(name, t)
    if r.dim() != 3 or v.dim() != 3:
        raise ValueError(f"r and v must be (B, T, A) and (B, T, D); got {tuple(r.shape)} and {tuple(v.shape)}")
    B, T, A = r.shape
    if v.shape[:2] != r.shape[:2]:
        raise ValueError(f"r {tuple(r.shape)} and v {tuple(v.shape)} disagree on (B, T)")
    if B == 0 or T == 0 or A == 0 or v.shape[2] == 0:
        raise ValueError(f"empty input: r {tuple(r.shape)}, v {tuple(v.shape)}")
    if w.shape != (A,):
        raise ValueError(f"w must have shape ({A},), got {tuple(w.shape)}")
    if g.numel() != 1:
        raise ValueError(f"g must hold one scalar, got shape {tuple(g.shape)}")
    nat.dtype_code(v.dtype)
    nat.require_device(r, v, g, w)


# The operators below are registered torch ops (torch.library.custom_op) with
# fake (meta) implementations and registered autograd, so torch.compile traces
# models that use them without graph breaks: each op is one opaque node whose
# output shapes the fake implementation gives. Their real implementations
# launch the native kernels on the current stream. Outputs never alias inputs;
# what a backward needs of an input's cast is recomputed from the input.

Tensor = torch.Tensor


def _fm_fwd_impl(r: Tensor, v: Tensor, g: Tensor, w: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """(q fp32, fast in v's dtype, saved uint8): ulm_fm_fwd."""
    B, T, A = r.shape
    D = v.shape[-1]
    r32 = r.float().contiguous()
    vc = v.contiguous()
    g1 = g.float().reshape(1).contiguous()
    w32 = w.float().contiguous()
    q = torch.empty(B, T, A, device=r.device, dtype=torch.float32)
    fast = torch.empty(B, T, D, device=r.device, dtype=v.dtype)
    vdt = nat.dtype_code(v.dtype)
    saved_bytes = nat.lib().ulm_fm_saved_bytes(B, T, A, D, vdt)
    saved = torch.empty(saved_bytes, device=r.device, dtype=torch.uint8)
    ws_bytes = nat.lib().ulm_fm_fwd_workspace_bytes(B, T, A, D, vdt)
    ws = torch.empty(max(ws_bytes, 1), device=r.device, dtype=torch.uint8)
    call("ulm_fm_fwd", ptr(r32), ptr(vc), vdt, ptr(g1), ptr(w32), ptr(q), ptr(fast), vdt, ptr(saved), saved_bytes,
         ptr(ws), ws_bytes, B, T, A, D, nat.stream_of(r))
    return q, fast, saved


fm_fwd = torch.library.custom_op("ulm::fm_fwd", mutates_args=())(_fm_fwd_impl)


@fm_fwd.register_fake
def _fm_fwd_fake(r, v, g, w):
    B, T, A = r.shape
    D = v.shape[-1]
    saved_bytes = nat.lib().ulm_fm_saved_bytes(B, T, A, D, nat.dtype_code(v.dtype))
    return (r.new_empty(B, T, A, dtype=torch.float32), v.new_empty(B, T, D),
            r.new_empty(saved_bytes, dtype=torch.uint8))


def _fm_bwd_impl(r: Tensor, g: Tensor, w: Tensor, saved: Tensor, v_dtype: torch.dtype, dq_out: Optional[Tensor],
                 dfast: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(dr fp32, dv in dfast's dtype, dg (1,), dw (A,)): ulm_fm_bwd."""
    B, T, A = r.shape
    D = dfast.shape[-1]
    r32 = r.float().contiguous()
    g1 = g.float().reshape(1).contiguous()
    w32 = w.float().contiguous()
    ddt = nat.dtype_code(dfast.dtype)
    dfast = dfast.contiguous()
    dqo = dq_out.float().contiguous() if dq_out is not None else None
    dr = torch.empty(B, T, A, device=r.device, dtype=torch.float32)
    dv = torch.empty(B, T, D, device=r.device, dtype=dfast.dtype)
    dg = torch.empty(1, device=r.device, dtype=torch.float32)
    dw = torch.empty(A, device=r.device, dtype=torch.float32)
    # the saved buffer's size names the form its forward used; the backward follows it
    ws_bytes = nat.lib().ulm_fm_bwd_workspace_bytes(B, T, A, D, ddt, saved.numel(), nat.dtype_code(v_dtype))
    ws = torch.empty(max(ws_bytes, 1), device=r.device, dtype=torch.uint8)
    call("ulm_fm_bwd", ptr(r32), ptr(g1), ptr(w32), ptr(saved), saved.numel(), nat.dtype_code(v_dtype), ptr(dfast),
         ddt, ptr(dqo), ptr(dr), ptr(dv), ddt, ptr(dg), ptr(dw), ptr(ws), ws_bytes, B, T, A, D, nat.stream_of(r))
    return dr, dv, dg, dw


fm_bwd = torch.library.custom_op("ulm::fm_bwd", mutates_args=())(_fm_bwd_impl)


@fm_bwd.register_fake
def _fm_bwd_fake(r, g, w, saved, v_dtype, dq_out, dfast):
    B, T, A = r.shape
    D = dfast.shape[-1]
    return (r.new_empty(B, T, A, dtype=torch.float32), dfast.new_empty(B, T, D),
            r.new_empty(1, dtype=torch.float32), r.new_empty(A, dtype=torch.float32))


def _fm_setup(ctx, inputs, output):
    r, v, g, w = inputs
    _, _, saved = output
    ctx.save_for_backward(r, g, w, saved)
    ctx.v_dtype, ctx.D = v.dtype, v.shape[-1]
    ctx.mark_non_differentiable(saved)
    # no zero-filled stand-ins for absent gradients (the saved buffer's above all)
    ctx.set_materialize_grads(False)


def _fm_backward_with(bwd, ctx, dq_out, dfast):
    r, g, w, saved = ctx.saved_tensors
    if dq_out is None and dfast is None:
        return None, None, None, None
    if dfast is None:
        dfast = r.new_zeros(*r.shape[:2], ctx.D, dtype=torch.float32)
    dr, dv, dg, dw = bwd(r, g, w, saved, ctx.v_dtype, dq_out, dfast)
    return dr, dv, dg.reshape(g.shape), dw


def _fm_backward(ctx, dq_out, dfast, _dsaved):
    return _fm_backward_with(fm_bwd, ctx, dq_out, dfast)


torch.library.register_autograd("ulm::fm_fwd", _fm_backward, setup_context=_fm_setup)


# the number of active torch dispatch modes (one assumed where torch does not say)
_dispatch_modes = getattr(torch._C, "_len_torch_dispatch_stack", lambda: 1)


def _plain_eager(*tensors):
    """True when the call runs eagerly on plain tensors: no torch.compile
    trace, no dispatch mode (fake tensors, functionalization) and no tensor
    subclass, so the native kernels can be called without the registered
    op's dispatch."""
    if torch.compiler.is_compiling() or _dispatch_modes() > 0:
        return False
    return all(type(t) is torch.Tensor for t in tensors)


class _FMEager(torch.autograd.Function):
    """The registered op pair ulm::fm_fwd / ulm::fm_bwd as a plain autograd
    Function over the same implementations: the eager path, without the
    registered ops' dispatch (about 20 us of host time per call, which
    small shapes feel). torch.compile traces the registered ops instead."""

    @staticmethod
    def forward(ctx, r, v, g, w):
        out = _fm_fwd_impl(r, v, g, w)
        _fm_setup(ctx, (r, v, g, w), out)
        return out

    @staticmethod
    def backward(ctx, dq_out, dfast, _dsaved):
        return _fm_backward_with(_fm_bwd_impl, ctx, dq_out, dfast)


def unified_memory(r, v, g, w):
    """r: (B,T,M) read addresses, v: (B,T,D) values, g: scalar log decay, w: (M,) prior mass.
    Returns (q fp32, fast in v's dtype) (kernel.py:236-238)."""
    _check_fm(r, v, g, w)
    if _plain_eager(r, v, g, w):
        q, fast, _ = _FMEager.apply(r, v, g, w)
    else:
        q, fast, _ = fm_fwd(r, v, g, w)
    return q, fast


class UnifiedMemory:
    """The reference's autograd Function (kernel.py:199-233) as a call
    surface: apply(r, v, g, w) is unified_memory, whose backward is the
    registered ulm::fm_bwd. The forward keeps one opaque buffer of what the
    backward needs (bf16 operand tiles of q, k and v, score tiles and the
    per-chunk evidence checkpoints that stand in for the full c tensor); v is
    passed in its own dtype and cast to bf16 for the products inside
    (kernel.py:205)."""

    @staticmethod
    def apply(r, v, g, w):
        return unified_memory(r, v, g, w)


def la(a, b, c, g, reverse=False, split=False):
    """o_t = sum_{s<=t} lam^(t-s) (a_t . b_s) c_s (s>=t when reverse), fp32 output.
    The chunked building block (kernel.py:183-196); a, b (B,T,K), c (B,T,V).
    split carries the decayed state-update operand as a bf16 hi + lo pair."""
    nat.require_device(a, b, c, g)
    a16, b16, c16 = (x.to(torch.bfloat16).contiguous() for x in (a, b, c))
    B, T, K = a16.shape
    V = c16.shape[-1]
    if b16.shape != a16.shape or c16.shape[:2] != a16.shape[:2]:
        raise ValueError("la: a, b must be (B,T,K) and c (B,T,V)")
    g1 = g.float().reshape(1).contiguous()
    out = torch.empty(B, T, V, device=a.device, dtype=torch.float32)
    ws_bytes = nat.lib().ulm_la_workspace_bytes(B, T, K, V)
    ws = torch.empty(max(ws_bytes, 1), device=a.device, dtype=torch.uint8)
    call("ulm_la", ptr(a16), ptr(b16), ptr(c16), ptr(g1), ptr(out), B, T, K, V, int(reverse), int(split), ptr(ws),
         ws_bytes, nat.stream_of(a))
    return out


# ---------------------------------------------------------------------------
# relu^2 slot address (model.py:70-72)

@torch.library.custom_op("ulm::addr_fwd", mutates_args=())
def addr_fwd(pre: Tensor, bias: Optional[Tensor], log_eps: Tensor) -> tuple[Tensor, Tensor]:
    """(r fp32 shaped like pre, denom (M,) fp32): ulm_addr_fwd."""
    A = pre.shape[-1]
    pre_c = pre.contiguous()
    b32 = bias.float().contiguous() if bias is not None else None
    le = log_eps.float().reshape(1).contiguous()
    M = pre_c.numel() // A
    r = torch.empty(pre.shape, device=pre.device, dtype=torch.float32)
    denom = torch.empty(M, device=pre.device, dtype=torch.float32)
    call("ulm_addr_fwd", ptr(pre_c), nat.dtype_code(pre.dtype), ptr(b32), ptr(le), ptr(r), ptr(denom), M, A,
         nat.stream_of(pre))
    return r, denom


@addr_fwd.register_fake
def _addr_fwd_fake(pre, bias, log_eps):
    return pre.new_empty(pre.shape, dtype=torch.float32), pre.new_empty(pre.numel() // pre.shape[-1],
                                                                        dtype=torch.float32)


@torch.library.custom_op("ulm::addr_bwd", mutates_args=())
def addr_bwd(pre: Tensor, bias: Optional[Tensor], log_eps: Tensor, r: Tensor, denom: Tensor,
             dr: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """(dpre in pre's dtype, dbias (A,) fp32 or (0,) without a bias, dlog_eps (1,)): ulm_addr_bwd."""
    A = pre.shape[-1]
    pre_c = pre.contiguous()
    M = pre_c.numel() // A
    b32 = bias.float().contiguous() if bias is not None else None
    le = log_eps.float().reshape(1).contiguous()
    dr = dr.float().contiguous()
    dpre = torch.empty_like(pre_c)
    dbias = torch.empty(A if bias is not None else 0, device=pre.device, dtype=torch.float32)
    dle = torch.empty(1, device=pre.device, dtype=torch.float32)
    ws_bytes = nat.lib().ulm_addr_bwd_workspace_bytes(M, A)
    ws = torch.empty(ws_bytes, device=pre.device, dtype=torch.uint8)
    call("ulm_addr_bwd", ptr(pre_c), nat.dtype_code(pre.dtype), ptr(b32), ptr(le), ptr(r.contiguous()),
         ptr(denom), ptr(dr), ptr(dpre), ptr(dbias if bias is not None else None), ptr(dle), ptr(ws), ws_bytes,
         M, A, nat.stream_of(pre))
    return dpre, dbias, dle


@addr_bwd.register_fake
def _addr_bwd_fake(pre, bias, log_eps, r, denom, dr):
    A = pre.shape[-1]
    return (torch.empty_like(pre, memory_format=torch.contiguous_format),
            pre.new_empty(A if bias is not None else 0, dtype=torch.float32), pre.new_empty(1, dtype=torch.float32))


def _addr_setup(ctx, inputs, output):
    pre, bias, log_eps = inputs
    r, denom = output
    ctx.save_for_backward(pre, bias, log_eps, r, denom)
    ctx.mark_non_differentiable(denom)
    ctx.set_materialize_grads(False)


def _addr_backward(ctx, dr, _ddenom):
    if dr is None:
        return None, None, None
    pre, bias, log_eps, r, denom = ctx.saved_tensors
    dpre, dbias, dle = addr_bwd(pre, bias, log_eps, r, denom, dr)
    return dpre, (dbias if bias is not None else None), dle.reshape(log_eps.shape)


torch.library.register_autograd("ulm::addr_fwd", _addr_backward, setup_context=_addr_setup)


def relu2_address(pre, bias, log_eps):
    """The slot address of model.py:70-72 from pre = K u (the bias added in fp32
    inside): r = z / (exp(clamp(log_eps,-10,10)) + sum_a z), z = relu(pre + bias)^2."""
    _check_float("pre", pre)
    if pre.dim() < 1 or pre.numel() == 0:
        raise ValueError(f"pre must be non-empty (..., A), got {tuple(pre.shape)}")
    A = pre.shape[-1]
    if bias is not None and bias.shape != (A,):
        raise ValueError(f"bias must have shape ({A},), got {tuple(bias.shape)}")
    if log_eps.numel() != 1:
        raise ValueError("log_eps must hold one scalar")
    nat.dtype_code(pre.dtype)
    nat.require_device(pre, bias, log_eps)
    return addr_fwd(pre, bias, log_eps)[0]


# ---------------------------------------------------------------------------
# UnifiedBlock.forward (model.py:77-85) with the fast memory and its
# elementwise ends fused; the GEMMs are plain library GEMMs (hipBLASLt through
# torch.mm) with fp32 accumulation

# clamp range of a block's log prior mass, w = exp(clamp(log_w, -7, 12)) (model.py:75)
LOG_W_MIN, LOG_W_MAX = -7.0, 12.0


def _mm(a, b, out_dtype):
    """a @ b, written in out_dtype straight from the fp32 accumulator."""
    return torch.mm(a, b) if a.dtype == out_dtype else torch.mm(a, b, out_dtype=out_dtype)


def _wgrad(a, b):
    """a^T b in fp32 for a (K, N1), b (K, N2) with K the token dimension: the
    split-K MFMA kernel for bf16 operands whose widths are multiples of 8,
    the library GEMM otherwise."""
    K, N1 = a.shape
    N2 = b.shape[1]
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16 or N1 % 8 or N2 % 8:
        return _mm(a.t(), b, torch.float32)
    a, b = a.contiguous(), b.contiguous()
    c = torch.empty(N1, N2, device=a.device, dtype=torch.float32)
    ws_bytes = nat.lib().ulm_wgrad_workspace_bytes(K, N1, N2)
    ws = torch.empty(max(ws_bytes, 1), device=a.device, dtype=torch.uint8)
    call("ulm_wgrad", ptr(a), ptr(b), ptr(c), K, N1, N2, ptr(ws), ws_bytes, nat.stream_of(a))
    return c


def _addmm_(c, a, b):
    """c += a @ b in place, c fp32, accumulated in the GEMM's epilogue."""
    if a.dtype == c.dtype:
        return torch.addmm(c, a, b, out=c)
    return torch.addmm(c, a, b, out_dtype=c.dtype, out=c)


# One UnifiedBlock (model.py:77-85) as two registered ops:
#
#     h, u   = RMSNorm(x), causal conv(h)               ulm_norm_conv_fwd
#     pre, v = u K^T, h W_v^T                            GEMMs in cdt
#     denom  = the relu^2 address's row sums of pre + b  ulm_addr_fwd (r not written)
#     g, w   = -exp(log_rate), exp(clamp(log_w))         ulm_block_params
#     wq, y  = w q, x + fast                             ulm_block_fm_fwd (r formed from pre)
#     out    = y + wq mu^T                               GEMM accumulating into y
#
# cdt is the GEMM operand dtype: bf16 under bf16 autocast (the reference's
# training configuration, train.py), fp32 otherwise. x is the fp32 residual
# stream; every gradient is returned in fp32. The forward's extra outputs are
# what the backward reads (the normalised input, the conv output, the key
# GEMM's output, the address denominators, g and w, the fast memory's saved
# buffer and w q).

_BLOCK_SAVED = 9   # outputs of block_fwd past `out`


@torch.library.custom_op("ulm::block_fwd", mutates_args=())
def block_fwd(x: Tensor, norm_w: Tensor, conv_w: Tensor, key_w: Tensor, key_b: Optional[Tensor], log_eps: Tensor,
              val_w: Tensor, mu_w: Tensor, log_rate: Tensor, log_w: Tensor, norm_eps: float,
              cdt: torch.dtype) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(out, rstd, h, u, pre, denom, g, w, saved, wq)."""
    # the GEMM dtypes are explicit: autocast must not re-cast them
    with torch.autocast("cuda", enabled=False):
        return _block_fwd_impl(x, norm_w, conv_w, key_w, key_b, log_eps, val_w, mu_w, log_rate, log_w, norm_eps, cdt)


def _block_fwd_impl(x, norm_w, conv_w, key_w, key_b, log_eps, val_w, mu_w, log_rate, log_w, norm_eps, cdt):
    B, T, D = x.shape
    A = key_w.shape[0]
    Kc = conv_w.shape[-1]
    M = B * T
    dev = x.device
    s = nat.stream_of(x)
    cd = nat.dtype_code(cdt)
    f32 = torch.float32
    x32 = x.contiguous()
    nw = norm_w.float().contiguous()
    cw = conv_w.float().reshape(D, Kc).contiguous()
    h = torch.empty(B, T, D, device=dev, dtype=cdt)
    u = torch.empty(B, T, D, device=dev, dtype=cdt)
    rstd = torch.empty(B, T, device=dev, dtype=f32)
    call("ulm_norm_conv_fwd", ptr(x32), nat.ULM_F32, ptr(nw), ptr(cw), Kc, float(norm_eps), ptr(h), cd, ptr(u), cd,
         ptr(rstd), B, T, D, s)
    kw, vw, mw = (t.to(cdt).contiguous() for t in (key_w, val_w, mu_w))
    pre = torch.mm(u.view(M, D), kw.t())
    v = torch.mm(h.view(M, D), vw.t())
    b32 = key_b.float().contiguous() if key_b is not None else None
    le = log_eps.float().reshape(1).contiguous()
    denom = torch.empty(M, device=dev, dtype=f32)
    # r itself is never written: the fast memory forms it from pre, bias and denom
    call("ulm_addr_fwd", ptr(pre), cd, ptr(b32), ptr(le), None, ptr(denom), M, A, s)
    lr = log_rate.float().reshape(1).contiguous()
    lw = log_w.float().contiguous()
    g1 = torch.empty(1, device=dev, dtype=f32)
    w32 = torch.empty(A, device=dev, dtype=f32)
    call("ulm_block_params", ptr(lr), ptr(lw), LOG_W_MIN, LOG_W_MAX, A, ptr(g1), ptr(w32), s)
    saved_bytes = nat.lib().ulm_fm_saved_bytes(B, T, A, D, cd)
    saved = torch.empty(saved_bytes, device=dev, dtype=torch.uint8)
    ws_bytes = nat.lib().ulm_block_fm_fwd_workspace_bytes(B, T, A, D)
    ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    qw = torch.empty(M, A, device=dev, dtype=cdt)
    y = torch.empty(M, D, device=dev, dtype=f32)
    call("ulm_block_fm_fwd", ptr(pre), cd, ptr(b32), ptr(denom), ptr(v), cd, ptr(g1), ptr(w32), ptr(qw), cd,
         ptr(x32), ptr(y), ptr(saved), saved_bytes, ptr(ws), ws_bytes, B, T, A, D, s)
    del ws, v
    out = _addmm_(y, qw, mw.t())
    return out.view(B, T, D), rstd, h, u, pre, denom, g1, w32, saved, qw


@block_fwd.register_fake
def _block_fwd_fake(x, norm_w, conv_w, key_w, key_b, log_eps, val_w, mu_w, log_rate, log_w, norm_eps, cdt):
    B, T, D = x.shape
    A = key_w.shape[0]
    M = B * T
    f32 = torch.float32
    saved_bytes = nat.lib().ulm_fm_saved_bytes(B, T, A, D, nat.dtype_code(cdt))
    e = x.new_empty
    return (e(B, T, D, dtype=f32), e(B, T, dtype=f32), e(B, T, D, dtype=cdt), e(B, T, D, dtype=cdt),
            e(M, A, dtype=cdt), e(M, dtype=f32), e(1, dtype=f32), e(A, dtype=f32), e(saved_bytes, dtype=torch.uint8),
            e(M, A, dtype=cdt))


@torch.library.custom_op("ulm::block_bwd", mutates_args=())
def block_bwd(dout: Tensor, x: Tensor, norm_w: Tensor, conv_w: Tensor, key_w: Tensor, key_b: Optional[Tensor],
              log_eps: Tensor, val_w: Tensor, mu_w: Tensor, log_rate: Tensor, log_w: Tensor, rstd: Tensor, h: Tensor,
              u: Tensor, pre: Tensor, denom: Tensor, g1: Tensor, w32: Tensor, saved: Tensor, qw: Tensor,
              cdt: torch.dtype) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                                         Tensor]:
    """(dx, dnorm_w, dconv_w, dkey_w, dkey_b ((0,) without a bias), dlog_eps,
    dval_w, dmu_w, dlog_rate, dlog_w), all fp32."""
    with torch.autocast("cuda", enabled=False):
        return _block_bwd_impl(dout, x, norm_w, conv_w, key_w, key_b, log_eps, val_w, mu_w, log_rate, log_w, rstd, h,
                               u, pre, denom, g1, w32, saved, qw, cdt)


def _block_bwd_impl(dout, x, norm_w, conv_w, key_w, key_b, log_eps, val_w, mu_w, log_rate, log_w, rstd, h, u, pre,
                    denom, g1, w32, saved, qw, cdt):
    B, T, D = x.shape
    A = key_w.shape[0]
    Kc = conv_w.shape[-1]
    M = B * T
    dev = x.device
    s = nat.stream_of(x)
    cd = nat.dtype_code(cdt)
    f32 = torch.float32
    x32 = x.contiguous()
    nw = norm_w.float().contiguous()
    cw = conv_w.float().reshape(D, Kc).contiguous()
    kw, vw, mw = (t.to(cdt).contiguous() for t in (key_w, val_w, mu_w))
    b32 = key_b.float().contiguous() if key_b is not None else None
    le = log_eps.float().reshape(1).contiguous()
    lr = log_rate.float().reshape(1).contiguous()
    lw = log_w.float().contiguous()
    dout = dout.float().contiguous()
    if cdt == f32:
        d16 = dout
    else:
        d16 = torch.empty(B, T, D, device=dev, dtype=cdt)
        call("ulm_cast", ptr(dout), nat.ULM_F32, ptr(d16), cd, M * D, s)
    d2 = d16.view(M, D)
    dqw = torch.mm(d2, mw)                       # d(w q) = dout mu
    dmu = _wgrad(d2, qw)
    dr = torch.empty(M, A, device=dev, dtype=f32)
    dv = torch.empty(M, D, device=dev, dtype=cdt)
    dg = torch.empty(1, device=dev, dtype=f32)
    dw = torch.empty(A, device=dev, dtype=f32)
    ws_bytes = nat.lib().ulm_fm_bwd_workspace_bytes(B, T, A, D, cd, saved.numel(), cd)
    ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    call("ulm_block_fm_bwd", ptr(pre), cd, ptr(b32), ptr(denom), ptr(g1), ptr(w32), ptr(saved), saved.numel(), cd,
         ptr(d16), cd, ptr(dqw), cd, ptr(dr), ptr(dv), cd, ptr(dg), ptr(dw), ptr(ws), ws_bytes, B, T, A, D, s)
    del ws, dqw
    dlr = torch.empty(1, device=dev, dtype=f32)
    dlw = torch.empty(A, device=dev, dtype=f32)
    call("ulm_block_params_bwd", ptr(lr), ptr(lw), LOG_W_MIN, LOG_W_MAX, ptr(dg), ptr(dw), A, ptr(dlr), ptr(dlw), s)
    dpre = torch.empty_like(pre)
    dbias = torch.empty(A if key_b is not None else 0, device=dev, dtype=f32)
    dle = torch.empty(1, device=dev, dtype=f32)
    ws_bytes = nat.lib().ulm_addr_bwd_workspace_bytes(M, A)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    call("ulm_addr_bwd", ptr(pre), cd, ptr(b32), ptr(le), None, ptr(denom), ptr(dr), ptr(dpre),
         ptr(dbias if key_b is not None else None), ptr(dle), ptr(ws), ws_bytes, M, A, s)
    del ws, dr
    du = _mm(dpre, kw, f32)
    dkey = _wgrad(dpre, u.view(M, D))
    dhv = _mm(dv, vw, f32)
    dval = _wgrad(dv, h.view(M, D))
    dx = torch.empty(B, T, D, device=dev, dtype=f32)
    dnw = torch.empty(D, device=dev, dtype=f32)
    dcw = torch.empty(D, Kc, device=dev, dtype=f32)
    ws_bytes = nat.lib().ulm_norm_conv_bwd_workspace_bytes(B, T, D, Kc)
    if ws_bytes == 0:
        raise ValueError(f"ulm_norm_conv_bwd: unsupported D={D}")
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    call("ulm_norm_conv_bwd", ptr(x32), nat.ULM_F32, ptr(rstd), ptr(nw), ptr(cw), Kc, ptr(du), nat.ULM_F32, ptr(dhv),
         nat.ULM_F32, ptr(dout), ptr(dx), ptr(dnw), ptr(dcw), ptr(ws), ws_bytes, B, T, D, s)
    return (dx, dnw, dcw.view(conv_w.shape), dkey, dbias, dle.reshape(log_eps.shape), dval, dmu,
            dlr.reshape(log_rate.shape), dlw)


@block_bwd.register_fake
def _block_bwd_fake(dout, x, norm_w, conv_w, key_w, key_b, log_eps, val_w, mu_w, log_rate, log_w, rstd, h, u, pre,
                    denom, g1, w32, saved, qw, cdt):
    f32 = torch.float32
    A = key_w.shape[0]
    e = x.new_empty
    return (e(x.shape, dtype=f32), e(norm_w.shape, dtype=f32), e(conv_w.shape, dtype=f32), e(key_w.shape, dtype=f32),
            e(A if key_b is not None else 0, dtype=f32), e(log_eps.shape, dtype=f32), e(val_w.shape, dtype=f32),
            e(mu_w.shape, dtype=f32), e(log_rate.shape, dtype=f32), e(log_w.shape, dtype=f32))


def _block_setup(ctx, inputs, output):
    x, norm_w, conv_w, key_w, key_b, log_eps, val_w, mu_w, log_rate, log_w, norm_eps, cdt = inputs
    ctx.save_for_backward(x, norm_w, conv_w, key_w, key_b, log_eps, val_w, mu_w, log_rate, log_w, *output[1:])
    ctx.cdt = cdt
    ctx.mark_non_differentiable(*output[1:])
    # the extra outputs never get gradients: no zero-filled stand-ins for them
    ctx.set_materialize_grads(False)


def _block_backward(ctx, dout, *_unused):
    if dout is None:
        return (None,) * 12
    saved = ctx.saved_tensors
    key_b = saved[4]
    dx, dnw, dcw, dkey, dbias, dle, dval, dmu, dlr, dlw = block_bwd(dout, *saved, ctx.cdt)
    return dx, dnw, dcw, dkey, (dbias if key_b is not None else None), dle, dval, dmu, dlr, dlw, None, None


torch.library.register_autograd("ulm::block_fwd", _block_backward, setup_context=_block_setup)


def unified_block(x, norm_w, conv_w, key_w, key_b, log_eps, val_w, mu_w, log_rate, log_w, norm_eps,
                  cdt=torch.float32):
    """x + mu(w q) + fast of one UnifiedBlock (model.py:77-85) in one fused
    forward and backward. x (B, T, D) fp32; key_w (A, D), mu_w (D, A),
    val_w (D, D), conv_w (D, 1, Kc); log_rate (a scalar) and log_w (A,) are the
    block's parameters: g = -exp(log_rate), w = exp(clamp(log_w, LOG_W_MIN,
    LOG_W_MAX)) (model.py:75, 84) are formed, and differentiated, natively."""
    if x.dim() != 3 or x.dtype != torch.float32:
        raise ValueError(f"x must be (B, T, D) fp32, got {tuple(x.shape)} {x.dtype}")
    B, T, D = x.shape
    A = key_w.shape[0]
    if B == 0 or T == 0 or D == 0:
        raise ValueError(f"empty input {tuple(x.shape)}")
    if key_w.shape != (A, D) or mu_w.shape != (D, A) or val_w.shape != (D, D) or log_w.shape != (A,):
        raise ValueError("block weights disagree with x: key (A, D), mu (D, A), val (D, D), log_w (A,)")
    if log_rate.numel() != 1:
        raise ValueError(f"log_rate must hold one value, got {tuple(log_rate.shape)}")
    if conv_w.numel() % D or not 1 <= conv_w.shape[-1] <= 8:
        raise ValueError(f"conv_w must be (D, 1, Kc) with 1 <= Kc <= 8, got {tuple(conv_w.shape)}")
    if cdt not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError(f"unsupported GEMM dtype {cdt}")
    nat.require_device(x, norm_w, conv_w, key_w, key_b, log_eps, val_w, mu_w, log_rate, log_w)
    return block_fwd(x, norm_w, conv_w, key_w, key_b, log_eps, val_w, mu_w, log_rate, log_w, float(norm_eps), cdt)[0]


# ---------------------------------------------------------------------------
# per-token decode (model.py:96-111), N sequences at once, fp32

@torch.no_grad()
def block_prefill(x, norm_w, conv_w, key_w, key_b, log_eps, val_w, mu_w, log_rate, log_w, norm_eps,
                  cdt=torch.float32):
    """UnifiedBlock.forward over a prompt (no autograd), fused as in
    block_fwd, plus what decoding continues from: returns (out, S, c,
    r_prev, h) with S (B, D, A) and c (B, A) the fast-memory state after the
    last position (as fm_prefill), r_prev (B, A) fp32 the address at that
    position and h (B, T, D) the normalised input in cdt (its last positions
    fill the conv window). log_rate and log_w are the block's parameters, as
    for unified_block."""
    if x.dim() != 3 or x.dtype != torch.float32:
        raise ValueError(f"x must be (B, T, D) fp32, got {tuple(x.shape)} {x.dtype}")
    B, T, D = x.shape
    A = key_w.shape[0]
    Kc = conv_w.shape[-1]
    M = B * T
    nat.require_device(x, norm_w, conv_w, key_w, key_b, log_eps, val_w, mu_w, log_rate, log_w)
    cd = nat.dtype_code(cdt)
    ws_bytes = nat.lib().ulm_block_fm_prefill_workspace_bytes(B, T, A, D, cd)
    if ws_bytes == 0:
        raise ValueError(f"block_prefill: unsupported sizes B={B} T={T} A={A} D={D}")
    dev = x.device
    s = nat.stream_of(x)
    f32 = torch.float32
    x32 = x.contiguous()
    nw = norm_w.float().contiguous()
    cw = conv_w.float().reshape(D, Kc).contiguous()
    h = torch.empty(B, T, D, device=dev, dtype=cdt)
    u = torch.empty(B, T, D, device=dev, dtype=cdt)
    rstd = torch.empty(B, T, device=dev, dtype=f32)
    call("ulm_norm_conv_fwd", ptr(x32), nat.ULM_F32, ptr(nw), ptr(cw), Kc, float(norm_eps), ptr(h), cd, ptr(u), cd,
         ptr(rstd), B, T, D, s)
    kw, vw, mw = (t.to(cdt).contiguous() for t in (key_w, val_w, mu_w))
    pre = torch.mm(u.view(M, D), kw.t())
    v = torch.mm(h.view(M, D), vw.t())
    del u
    b32 = key_b.float().contiguous() if key_b is not None else None
    le = log_eps.float().reshape(1).contiguous()
    denom = torch.empty(M, device=dev, dtype=f32)
    call("ulm_addr_fwd", ptr(pre), cd, ptr(b32), ptr(le), None, ptr(denom), M, A, s)
    lr = log_rate.float().reshape(1).contiguous()
    lw = log_w.float().contiguous()
    g1 = torch.empty(1, device=dev, dtype=f32)
    w32 = torch.empty(A, device=dev, dtype=f32)
    call("ulm_block_params", ptr(lr), ptr(lw), LOG_W_MIN, LOG_W_MAX, A, ptr(g1), ptr(w32), s)
    qw = torch.empty(M, A, device=dev, dtype=cdt)
    y = torch.empty(M, D, device=dev, dtype=f32)
    S = torch.empty(B, D, A, device=dev, dtype=f32)
    c = torch.empty(B, A, device=dev, dtype=f32)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    call("ulm_block_fm_prefill", ptr(pre), cd, ptr(b32), ptr(denom), ptr(v), cd, ptr(g1), ptr(w32), ptr(qw), cd,
         ptr(x32), ptr(y), ptr(S), ptr(c), ptr(ws), ws_bytes, B, T, A, D, s)
    del ws, v
    out = _addmm_(y, qw, mw.t())
    # the address at the last position, the decode state's r_prev
    pre_last = pre.view(B, T, A)[:, -1].contiguous()
    r_prev = torch.empty(B, A, device=dev, dtype=f32)
    dn_last = torch.empty(B, device=dev, dtype=f32)
    call("ulm_addr_fwd", ptr(pre_last), cd, ptr(b32), ptr(le), ptr(r_prev), ptr(dn_last), B, A, s)
    return out.view(B, T, D), S, c, r_prev, h


def fm_prefill(r, v, g, w):
    """The forward of unified_memory (no autograd) plus the decode state after
    the last position: returns (q, fast, S, c) with S (B, D, A) fp32 =
    sum_s lam^(T-1-s) v_s k_s^T and c (B, A) fp32 = w + sum_s lam^(T-1-s) k_s,
    the state UnifiedBlock.step carries (model.py:88-111)."""
    _check_fm(r, v, g, w)
    B, T, A = r.shape
    D = v.shape[-1]
    r32 = r.float().contiguous()
    vc = v.contiguous()
    g1 = g.float().reshape(1).contiguous()
    w32 = w.float().contiguous()
    vdt = nat.dtype_code(v.dtype)
    ws_bytes = nat.lib().ulm_fm_prefill_workspace_bytes(B, T, A, D, vdt, vdt)
    if ws_bytes == 0:
        raise RuntimeError(f"fm_prefill: unsupported sizes B={B} T={T} A={A} D={D}")
    q = torch.empty_like(r32)
    fast = torch.empty(B, T, D, device=r.device, dtype=v.dtype)
    S = torch.empty(B, D, A, device=r.device, dtype=torch.float32)
    c = torch.empty(B, A, device=r.device, dtype=torch.float32)
    ws = torch.empty(ws_bytes, device=r.device, dtype=torch.uint8)
    call("ulm_fm_prefill", ptr(r32), ptr(vc), vdt, ptr(g1), ptr(w32), ptr(q), ptr(fast), vdt, ptr(S), ptr(c), ptr(ws),
         ws_bytes, B, T, A, D, nat.stream_of(r))
    return q, fast, S, c


def _f32c(t):
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise ValueError("decode tensors must be contiguous float32")
    return t


def decode_pre(x, norm_w, conv_w, conv_buf, norm_eps):
    """h = RMSNorm(x), u = causal conv over [conv_buf, h]; conv_buf shifted in place."""
    N, D = x.shape
    Kc = conv_w.shape[-1]
    nat.require_device(x, norm_w, conv_w, conv_buf)
    h = torch.empty_like(x)
    u = torch.empty_like(x)
    call("ulm_decode_pre", ptr(_f32c(x)), ptr(_f32c(norm_w)), ptr(_f32c(conv_w)), ptr(_f32c(conv_buf)), ptr(h), ptr(u),
         N, D, Kc, float(norm_eps), nat.stream_of(x))
    return h, u


def decode_addr(pre, bias, log_eps, w, g, r_prev, c):
    """r = relu^2 address, c <- lam c + (1-lam) w + r_prev (in place), q = r / c.
    Returns (r, q, w*q)."""
    N, A = pre.shape
    nat.require_device(pre, bias, log_eps, w, g, r_prev, c)
    r = torch.empty_like(pre)
    q = torch.empty_like(pre)
    wq = torch.empty_like(pre)
    call("ulm_decode_addr", ptr(_f32c(pre)), ptr(None if bias is None else _f32c(bias)), ptr(_f32c(log_eps)),
         ptr(_f32c(w)), ptr(_f32c(g)), ptr(_f32c(r_prev)), ptr(_f32c(c)), ptr(r), ptr(q), ptr(wq), N, A,
         nat.stream_of(pre))
    return r, q, wq


def decode_state(S, v, r_prev, q, g, x, ymu, out=None):
    """S <- lam S + v r_prev^T (in place); returns x + S q + ymu."""
    N, D, A = S.shape
    nat.require_device(S, v, r_prev, q, g, x, ymu)
    out = torch.empty_like(x) if out is None else out
    call("ulm_decode_state", ptr(_f32c(S)), ptr(_f32c(v)), ptr(_f32c(r_prev)), ptr(_f32c(q)), ptr(_f32c(g)),
         ptr(_f32c(x)), ptr(_f32c(ymu)), ptr(out), N, D, A, nat.stream_of(S))
    return out


def decode_addr_deferred(pre, bias, log_eps, w, g, r_prev, c, pr, slot, dots):
    """decode_addr for a deferred state: also appends r_prev as pending key
    `slot` of pr (J,N,A) and, with dots, returns the read-out weights
    cj (slot+1, N) of the terms 0 .. slot. Returns (r, q, w*q, cj or None)."""
    N, A = pre.shape
    nat.require_device(pre, bias, log_eps, w, g, r_prev, c, pr)
    r = torch.empty_like(pre)
    q = torch.empty_like(pre)
    wq = torch.empty_like(pre)
    cj = torch.empty(slot + 1, N, device=pre.device, dtype=torch.float32) if dots else None
    call("ulm_decode_addr_deferred", ptr(_f32c(pre)), ptr(None if bias is None else _f32c(bias)), ptr(_f32c(log_eps)),
         ptr(_f32c(w)), ptr(_f32c(g)), ptr(_f32c(r_prev)), ptr(_f32c(c)), ptr(r), ptr(q), ptr(wq), ptr(_f32c(pr)),
         slot, ptr(cj), N, A, nat.stream_of(pre))
    return r, q, wq, cj


def decode_deferred(S, pv, pr, m, flush, q, g, x, ymu, cj=None):
    """One position on a deferred state (S_base, the first m of the pending
    write terms pv (J,N,D), pr (J,N,A), the newest term already appended):
    with flush, S_base <- S_t in place; else S_base is only read, with the
    terms' read-out weights cj (m,N) (formed here by ulm_decode_dots when not
    given). Returns x + S_t q + ymu."""
    N, D, A = S.shape
    nat.require_device(S, pv, pr, q, g, x, ymu)
    out = torch.empty_like(x)
    st = nat.stream_of(S)
    if flush:
        call("ulm_decode_flush", ptr(_f32c(S)), ptr(_f32c(pv)), ptr(_f32c(pr)), m, ptr(_f32c(q)), ptr(_f32c(g)),
             ptr(_f32c(x)), ptr(_f32c(ymu)), ptr(out), N, D, A, st)
    else:
        if cj is None:
            cj = torch.empty(m, N, device=S.device, dtype=torch.float32)
            call("ulm_decode_dots", ptr(_f32c(pr)), ptr(_f32c(q)), ptr(cj), m, N, A, st)
        call("ulm_decode_read", ptr(_f32c(S)), ptr(_f32c(pv)), ptr(_f32c(cj)), m, ptr(_f32c(q)), ptr(_f32c(g)),
             ptr(_f32c(x)), ptr(_f32c(ymu)), ptr(out), N, D, A, st)
    return out
