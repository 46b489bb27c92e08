"""The drop-in under torch.compile (the reference trains a compiled model,
train.py:177-180): the native operators are registered torch ops
(torch.library.custom_op) with fake implementations and registered autograd.

CPU part: under FakeTensorMode with fake ROCm tensors the ops (the block in
fp32 and bf16 GEMM dtypes) and a whole UnifiedLM forward produce the shapes
and dtypes of the real ones without touching a GPU. GPU part (marked gpu): torch.compile of the model with
fullgraph=True (so any graph break fails) runs forward and backward and
matches eager at 1e-5, fp32 and under bf16 autocast. The compile uses the
aot_eager backend: dynamo and AOTAutograd trace through the registered ops and
their fake implementations; no code is generated for the ops around them."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import kernel
from model import ModelArgs, UnifiedLM


def test_ops_are_registered():
    for name in ("fm_fwd", "fm_bwd", "addr_fwd", "addr_bwd", "block_fwd", "block_bwd"):
        assert hasattr(torch.ops.ulm, name), name


@pytest.mark.parametrize("A", [128, 140])
def test_fake_shapes_match_the_operators(A):
    B, T, D = 2, 70, 64
    with FakeTensorMode(), torch.device("cuda"):
        r = torch.rand(B, T, A)
        v = torch.randn(B, T, D, dtype=torch.bfloat16)
        q, fast = kernel.unified_memory(r, v, torch.tensor(-0.05), torch.full((A,), 4.0))
        assert q.shape == (B, T, A) and q.dtype == torch.float32
        assert fast.shape == (B, T, D) and fast.dtype == torch.bfloat16
        pre = torch.randn(B, T, A, dtype=torch.bfloat16)
        addr = kernel.relu2_address(pre, torch.zeros(A), torch.zeros(()))
        assert addr.shape == (B, T, A) and addr.dtype == torch.float32
        model = UnifiedLM(ModelArgs(dim=D, n_layers=2, hidden_dim=A, vocab_size=97, max_seq_len=T))
        blk = model.layers[0]
        xb = torch.randn(B, T, D)
        for cdt in (torch.float32, torch.bfloat16):   # the block's GEMM dtype under autocast
            out = kernel.unified_block(xb, blk.norm.weight, blk.conv.weight, blk.key.weight, blk.key.bias,
                                       blk.log_eps, blk.val.weight, blk.mu.weight, blk.log_rate, blk.log_w, 1e-5, cdt)
            assert out.shape == (B, T, D) and out.dtype == torch.float32
        x = torch.randint(0, 97, (B, T))
        logits = model(x, x)
        assert logits.shape == (B, T, 97) and logits.dtype == torch.float32 and model.last_loss.shape == ()


def _grads(model):
    return {n: p.grad.detach().clone() for n, p in model.named_parameters()}


@pytest.mark.gpu
@pytest.mark.parametrize("autocast", [False, True])
def test_compiled_model_matches_eager(autocast):
    from helpers import rel, say, tiny_model
    say(f"torch.compile(UnifiedLM, fullgraph=True) fwd+bwd vs eager, autocast={autocast}")
    torch._dynamo.reset()
    model = tiny_model(dim=64, n_layers=2, hidden_dim=140, vocab_size=97, max_seq_len=128).cuda().train()
    x = torch.randint(0, 97, (2, 128), generator=torch.Generator().manual_seed(3)).cuda()
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        eager = model(x, x).float()
    model.last_loss.backward()
    loss_e, g_e = model.last_loss.item(), _grads(model)
    model.zero_grad(set_to_none=True)
    compiled = torch.compile(model, backend="aot_eager", fullgraph=True)
    for _ in range(2):   # the second call runs the cached graph
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            out = compiled(x, x).float()
        model.last_loss.backward()
    torch.cuda.synchronize()
    errs = {"logits": rel(out, eager), "loss": abs(model.last_loss.item() - loss_e) / abs(loss_e)}
    errs.update({n: rel(p.grad, g_e[n]) for n, p in model.named_parameters()})
    say(f"  worst {max(errs.values()):.3e}")
    assert max(errs.values()) < 1e-5, errs


@pytest.mark.gpu
def test_eager_function_matches_registered_op():
    """unified_memory on plain tensors calls the native kernels through a plain
    autograd Function; the registered op pair (what torch.compile traces) must
    give the same outputs and gradients bit for bit."""
    from helpers import say
    import workloads
    B, T, D, A = 2, 200, 64, 140
    say(f"eager Function vs registered op, B={B} T={T} D={D} A={A}")
    r, v, g, w = workloads.block_inputs(B, T, D, A, seed=7, device=torch.device("cuda"), v_dtype=torch.bfloat16)
    gen = torch.Generator(device="cuda").manual_seed(8)
    dq = torch.randn(B, T, A, device="cuda", generator=gen) * 0.01
    df = torch.randn(B, T, D, device="cuda", generator=gen).to(torch.bfloat16)
    res = []
    for eager in (True, False):
        leaves = [t.detach().clone().requires_grad_(True) for t in (r, v, g, w)]
        if eager:
            assert kernel._plain_eager(*leaves)
            q, fast = kernel.unified_memory(*leaves)
        else:
            q, fast, _ = kernel.fm_fwd(*leaves)
        grads = torch.autograd.grad((q, fast), leaves, (dq, df))
        res.append([q, fast, *grads])
    for a, b in zip(*res):
        assert a.dtype == b.dtype and torch.equal(a, b)
