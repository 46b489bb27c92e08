"""The C-ABI boundary and the host-side checks (CPU only: no compute call
reaches the GPU; invalid calls must fail before any HIP call)."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ulm_fm.h")

import ulm_native as nat  # noqa: E402


def header_functions(header=HEADER):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ulm_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = nat.lib()
    declared = header_functions()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(nat.SIGNATURES) == declared
    assert lib.ulm_abi_version() == 3


def test_integration_notes_name_every_entry_point():
    """Every function include/ulm_fm.h declares has its row in the
    integration notes' table of entry points."""
    notes = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    missing = [name for name in header_functions() if f"`{name}`" not in notes]
    assert not missing, missing


def test_probes_live_in_the_test_library_only():
    """The layout probes (include/ulm_probe.h) are exported by the test-only
    libulm_probe.so and not by the product library."""
    from helpers import PROBE_SIGNATURES, probe_lib
    declared = header_functions(os.path.join(ROOT, "include", "ulm_probe.h"))
    assert declared == sorted(n for n in PROBE_SIGNATURES if n.startswith("ulm_probe_"))
    plib = probe_lib()
    lib = nat.lib()
    for name in declared:
        assert hasattr(plib, name), name
        assert not hasattr(lib, name), name
    st = plib.ulm_probe_mfma(None, None, None, None)
    assert st == nat.ULM_ERR_INVALID and b"null pointer" in plib.ulm_last_error()


def test_c_side_rejects_bad_sizes_without_touching_the_gpu():
    lib = nat.lib()
    st = lib.ulm_la(None, None, None, None, None, 0, 10, 8, 8, 0, 0, None, 0, None)
    assert st == nat.ULM_ERR_INVALID
    assert b"bad sizes" in lib.ulm_last_error()
    st = lib.ulm_fm_fwd(None, None, 0, *([None] * 4), 0, None, 0, None, 0, 2, 64, 8, 8, None)
    assert st == nat.ULM_ERR_INVALID and b"null pointer" in lib.ulm_last_error()
    st = lib.ulm_decode_state(*([None] * 8), 4, 8, 100000, None)
    assert st == nat.ULM_ERR_INVALID and b"LDS" in lib.ulm_last_error()


def test_timer_product_query_checks_its_tag():
    """ulm_la_timer_product: tags outside ULM_PRODUCT_* and null outputs are
    rejected (no HIP call); the Python tag table equals the header's enum."""
    lib = nat.lib()
    ms, n = ctypes.c_double(), ctypes.c_int()
    for tag in (0, -1, 8):
        assert lib.ulm_la_timer_product(tag, ctypes.byref(ms), ctypes.byref(n)) == nat.ULM_ERR_INVALID
        assert b"bad product tag" in lib.ulm_last_error()
    assert lib.ulm_la_timer_product(1, None, ctypes.byref(n)) == nat.ULM_ERR_INVALID
    assert lib.ulm_la_timer_product(nat.PRODUCTS["scores"], ctypes.byref(ms), ctypes.byref(n)) == nat.ULM_OK
    assert n.value >= 0 and ms.value >= 0.0
    enum = {k.lower(): int(v) for k, v in re.findall(r"ULM_PRODUCT_(\w+) = (\d+)", open(HEADER).read())}
    names = {"scores": "scores", "apply": "apply", "dscores": "dscores", "dv": "dv", "dqstats": "dq_f",
             "dkdr": "dk_f", "state": "state"}
    assert {names[k]: v for k, v in enum.items()} == nat.PRODUCTS


def test_nonzero_status_surfaces_as_runtime_error():
    with pytest.raises(RuntimeError, match="status 1"):
        nat.call("ulm_la", None, None, None, None, None, 1, 0, 8, 8, 0, 0, None, 0, None)


def test_workspace_sizes(monkeypatch):
    lib = nat.lib()
    B, T, A, D = 16, 1024, 3072, 768
    NT = (T + 63) // 64
    # at the 110M shape the block-pair form needs fewer flops than the chunked state form
    assert lib.ulm_fm_path(B, T, A, D) == 2
    assert lib.ulm_fm_path(B, 8192, A, D) == 1            # past 4096 positions: the state form
    assert lib.ulm_fm_path(2, 200, 140, 64) == 2          # widths off the 32 grid: padded pair tiles
    assert lib.ulm_fm_path(2, 5000, 12, 8) == 0           # ... past 4096 positions: the generic kernel
    # ... and where the pair form would need more than twice the state form's
    # flops: at the reference's 15M widths from about 2400 positions on
    assert lib.ulm_fm_path(32, 2048, 712, 288) == 2
    assert lib.ulm_fm_path(32, 2560, 712, 288) == 0
    assert lib.ulm_fm_path(32, 4096, 712, 288) == 0
    # pair form, saved: bf16 q, k (Q layout), v (R layout), the scores P, their
    # transpose and their bf16 residual (Tq x Tq per row), n checkpoints
    Tq = (T + 127) // 128 * 128
    for dt in (nat.ULM_BF16, nat.ULM_F32):
        assert lib.ulm_fm_saved_bytes(B, T, A, D, dt) >= B * T * (4 * A + 2 * D) + 3 * B * Tq * Tq * 2 + B * NT * A * 4
    # backward: two tiled dfast copies, dS and its transpose, the per-tile statistics;
    # dq_f and dk_f stay in the products' epilogues (no fp32 (B, T, A) copies)
    # forward: q, k in the R layout for the scores, v in the Q layout for the apply
    nfw = lib.ulm_fm_fwd_workspace_bytes(B, T, A, D, nat.ULM_F32)
    assert nfw == 2 * B * NT * 64 * A * 2 + B * NT * 64 * D * 2
    nbw = lib.ulm_fm_bwd_workspace_bytes(B, T, A, D, nat.ULM_F32, 0, 0)
    assert B * T * 4 * D + 2 * B * Tq * Tq * 2 <= nbw < B * T * 4 * D + 2 * B * Tq * Tq * 2 + B * T * 4 * A
    assert (lib.ulm_fm_bwd_workspace_bytes(B, T, A, D, nat.ULM_F32, 0, 0)
            == lib.ulm_fm_bwd_workspace_bytes(B, T, A, D, nat.ULM_BF16, 0, 0))
    monkeypatch.setenv("ULM_FM_PATH", "chunked")
    assert lib.ulm_fm_path(B, T, A, D) == 1
    # 4 key groups of 768 slots: fp32 partial outputs, plus the forward score tiles
    assert lib.ulm_fm_fwd_workspace_bytes(B, T, A, D, nat.ULM_F32) >= 4 * B * T * D * 4 + B * NT * 64 * 64 * 2
    assert lib.ulm_fm_fwd_workspace_bytes(B, T, A, D, nat.ULM_BF16) >= B * T * D * 4
    assert lib.ulm_fm_bwd_workspace_bytes(B, T, A, D, nat.ULM_BF16, 0, 0) >= B * T * (2 * A * 4 + D * 4)
    # an fp32 dfast adds the bf16 remainder tiles of its two tiled copies
    assert (lib.ulm_fm_bwd_workspace_bytes(B, T, A, D, nat.ULM_F32, 0, 0)
            - lib.ulm_fm_bwd_workspace_bytes(B, T, A, D, nat.ULM_BF16, 0, 0)) == 2 * B * T * D * 2
    # saved: bf16 q, k in both tiled layouts, two v copies, n checkpoints
    assert lib.ulm_fm_saved_bytes(B, T, A, D, nat.ULM_BF16) >= B * T * (8 * A + 4 * D) + B * NT * A * 4
    assert (lib.ulm_fm_saved_bytes(B, T, A, D, nat.ULM_F32)
            - lib.ulm_fm_saved_bytes(B, T, A, D, nat.ULM_BF16)) == 2 * B * T * D * 2   # both multiples of 4 KB
    # the generic kernel keeps natural bf16 copies of q, k, v and the checkpoints
    assert lib.ulm_fm_saved_bytes(2, 5000, 12, 8, nat.ULM_F32) >= 2 * 5000 * (12 * 4 + 8 * 2) + 2 * 79 * 12 * 4
    # its bare product needs partial planes only past one 128-key tile
    assert lib.ulm_la_workspace_bytes(2, 70, 12, 8) == 0
    assert lib.ulm_la_workspace_bytes(2, 70, 300, 8) == 3 * 2 * 70 * 8 * 4
    assert lib.ulm_la_workspace_bytes(B, T, A, D) >= 3 * B * NT * A * 64 * 2 + 4 * B * T * D * 4
    assert lib.ulm_addr_bwd_workspace_bytes(B * T, A) >= A * 4
    assert lib.ulm_fm_bwd_workspace_bytes(0, T, A, D, nat.ULM_F32, 0, 0) == 0


def test_saved_buffer_names_its_form(monkeypatch):
    """The saved buffer's size records the form that filled it: ulm_fm_bwd and
    its workspace sizer follow that form whatever ULM_FM_PATH says later, and a
    size that names no form is rejected before any HIP call."""
    lib = nat.lib()
    B, T, A, D = 16, 1024, 3072, 768
    sizes = {}
    for name, code in (("pair", 2), ("chunked", 1), ("generic", 0)):
        monkeypatch.setenv("ULM_FM_PATH", name)
        n = lib.ulm_fm_saved_bytes(B, T, A, D, nat.ULM_BF16)
        assert lib.ulm_fm_saved_path(n, B, T, A, D, nat.ULM_BF16) == code
        # the size also pins the shape and the dtype of v
        assert lib.ulm_fm_saved_path(n, B, T + 64, A, D, nat.ULM_BF16) == -1
        assert lib.ulm_fm_saved_path(n, B, T, A, D, nat.ULM_F32) in (-1, code) and n % 4096 == 256 * (code + 1)
        assert lib.ulm_fm_saved_path(n + 4096, B, T, A, D, nat.ULM_BF16) == -1
        sizes[name] = (n, lib.ulm_fm_bwd_workspace_bytes(B, T, A, D, nat.ULM_BF16, 0, 0))
    assert len({n for n, _ in sizes.values()}) == 3
    # under another setting, the workspace sizer still answers for the saved form
    monkeypatch.setenv("ULM_FM_PATH", "pair")
    for name, (n, ws) in sizes.items():
        assert lib.ulm_fm_bwd_workspace_bytes(B, T, A, D, nat.ULM_BF16, n, nat.ULM_BF16) == ws, name
    assert lib.ulm_fm_bwd_workspace_bytes(B, T, A, D, nat.ULM_BF16, 12345, nat.ULM_BF16) == 0
    # a form the shape does not allow: the chunked form needs A, D multiples of 32
    monkeypatch.setenv("ULM_FM_PATH", "chunked")
    n_unaligned = lib.ulm_fm_saved_bytes(2, 200, 140, 64, nat.ULM_BF16)
    assert lib.ulm_fm_saved_path(n_unaligned, 2, 200, 140, 64, nat.ULM_BF16) == 2
    # the entry points reject a saved size that names no form, or a workspace
    # sized for another form, before touching the GPU
    x = ctypes.c_void_p(256)
    n_pair, ws_pair = sizes["pair"]
    n_chunked, ws_chunked = sizes["chunked"]
    assert ws_chunked > ws_pair
    st = lib.ulm_fm_bwd(x, x, x, x, n_pair + 1, nat.ULM_BF16, x, nat.ULM_BF16, None, x, x, nat.ULM_BF16, x, x, x,
                        1 << 40, B, T, A, D, None)
    assert st == nat.ULM_ERR_INVALID and b"names no form" in lib.ulm_last_error()
    st = lib.ulm_fm_bwd(x, x, x, x, n_chunked, nat.ULM_BF16, x, nat.ULM_BF16, None, x, x, nat.ULM_BF16, x, x, x,
                        ws_pair, B, T, A, D, None)
    assert st == nat.ULM_ERR_INVALID and b"workspace" in lib.ulm_last_error()
    st = lib.ulm_fm_fwd(x, x, nat.ULM_BF16, x, x, x, x, nat.ULM_BF16, x, n_pair - 256, x, 1 << 40, B, T, A, D, None)
    assert st == nat.ULM_ERR_INVALID and b"names no form" in lib.ulm_last_error()
    st = lib.ulm_block_fm_bwd(x, nat.ULM_BF16, None, x, x, x, x, n_pair + 4096, nat.ULM_BF16, x, nat.ULM_BF16, x,
                              nat.ULM_BF16, x, x, nat.ULM_BF16, x, x, x, 1 << 40, B, T, A, D, None)
    assert st == nat.ULM_ERR_INVALID and b"names no form" in lib.ulm_last_error()


def _fm_args(B=2, T=70, A=12, D=8, dtype=torch.float32):
    return (torch.rand(B, T, A, dtype=dtype), torch.randn(B, T, D, dtype=dtype),
            torch.tensor(-0.05), torch.full((A,), 4.0))


def test_unified_memory_input_checks():
    from kernel import unified_memory
    r, v, g, w = _fm_args()
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        unified_memory(r, v, g, w)                       # CPU tensors: no fallback
    with pytest.raises(ValueError, match="disagree"):
        unified_memory(r, v[:, :5], g, w)
    with pytest.raises(ValueError, match="w must have shape"):
        unified_memory(r, v, g, w[:5])
    with pytest.raises(ValueError, match="empty"):
        unified_memory(r[:0], v[:0], g, w)
    with pytest.raises(ValueError, match="one scalar"):
        unified_memory(r, v, torch.zeros(2), w)
    with pytest.raises(TypeError, match="floating"):
        unified_memory(r.long(), v, g, w)
    with pytest.raises(ValueError, match=r"\(B, T, A\)"):
        unified_memory(r[0], v[0], g, w)


def test_address_input_checks():
    from kernel import relu2_address
    pre = torch.randn(4, 10)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        relu2_address(pre, torch.zeros(10), torch.zeros(()))
    with pytest.raises(ValueError, match="bias"):
        relu2_address(pre, torch.zeros(9), torch.zeros(()))
    with pytest.raises(TypeError, match="floating"):
        relu2_address(pre.int(), None, torch.zeros(()))


def test_decode_rejects_non_fp32():
    from kernel import decode_state
    S = torch.zeros(2, 4, 8, dtype=torch.float64)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        decode_state(S, torch.zeros(2, 4), torch.zeros(2, 8), torch.zeros(2, 8), torch.zeros(1), torch.zeros(2, 4),
                     torch.zeros(2, 4))


def test_model_parameters_match_reference_layout():
    """The module tree and parameter names of the reference (model.py:45-147)."""
    from model import ModelArgs, UnifiedLM
    m = UnifiedLM(ModelArgs(dim=16, n_layers=2, hidden_dim=24, vocab_size=50, max_seq_len=32))
    names = [n for n, _ in m.named_parameters()]
    expect = ["tok_embeddings.weight"]
    for i in range(2):
        # a module's own parameters come before its submodules' in named_parameters()
        expect += [f"layers.{i}.{n}" for n in ("log_eps", "log_rate", "log_w", "norm.weight", "conv.weight",
                                               "key.weight", "key.bias", "mu.weight", "val.weight")]
    expect += ["norm.weight"]
    assert names == expect
    # the state dict lists the same tensors in the same order (the tied output matrix last)
    assert list(m.state_dict()) == expect + ["output.weight"]
    # registration order inside a block (model.py:59-68): norm, conv, key, mu,
    # log_eps, val, log_rate, log_w, dropout
    blk = m.layers[0]
    assert list(blk._modules) == ["norm", "conv", "key", "mu", "val", "dropout"]
    assert list(blk._parameters) == ["log_eps", "log_rate", "log_w"]
    assert m.output.weight is m.tok_embeddings.weight
    assert torch.all(m.layers[0].val.weight == 0) and torch.all(m.layers[0].conv.weight[:, 0, -1] == 1)


def test_training_helpers_of_the_reference_interface():
    """configure_optimizers and estimate_mfu, called as train.py:172 and :295 call them."""
    from model import ModelArgs, UnifiedLM
    args = ModelArgs(dim=16, n_layers=2, hidden_dim=24, vocab_size=50, max_seq_len=32)
    m = UnifiedLM(args)
    opt = m.configure_optimizers(0.1, 3e-4, (0.9, 0.95), "cpu")
    assert isinstance(opt, torch.optim.AdamW)
    decay, nodecay = opt.param_groups
    assert decay["weight_decay"] == 0.1 and nodecay["weight_decay"] == 0.0
    assert opt.defaults["lr"] == 3e-4 and opt.defaults["betas"] == (0.9, 0.95)
    named = dict(m.named_parameters())
    ids = lambda group: [id(p) for p in group["params"]]
    # matrices decay (the tied embedding once), vectors and scalars do not, in parameters() order
    assert ids(decay) == [id(p) for n, p in named.items() if p.dim() >= 2]
    assert ids(nodecay) == [id(p) for n, p in named.items() if p.dim() < 2]
    assert {n for n, p in named.items() if p.dim() < 2} == {
        f"layers.{i}.{n}" for i in range(2) for n in ("log_eps", "log_rate", "log_w", "norm.weight", "key.bias")
    } | {"norm.weight"}
    # the MFU of an iteration that runs at exactly the peak rate is 1
    n_params = sum(p.numel() for p in m.parameters())
    mixing = min(64, 32) * (2 * 24 + 16) + 2 * 24 * 16
    flops = (6 * n_params + 6 * 2 * mixing) * 32 * 8
    assert abs(m.estimate_mfu(8, flops / 2516.6e12) - 1.0) < 1e-12
    assert abs(m.estimate_mfu(8, flops / 312e12, peak_flops=312e12) - 1.0) < 1e-12


def test_block_entry_points_reject_bad_arguments_without_touching_the_gpu():
    lib = nat.lib()
    P = None
    # norm/conv: taps outside 1..8, h and u in different dtypes, D too wide for the backward
    st = lib.ulm_norm_conv_fwd(P, nat.ULM_F32, P, P, 9, 1e-5, P, nat.ULM_F32, P, nat.ULM_F32, P, 2, 8, 16, P)
    assert st == nat.ULM_ERR_INVALID and b"Kc=9" in lib.ulm_last_error()
    st = lib.ulm_norm_conv_fwd(P, nat.ULM_F32, P, P, 4, 1e-5, P, nat.ULM_BF16, P, nat.ULM_F32, P, 2, 8, 16, P)
    assert st == nat.ULM_ERR_INVALID and b"share one" in lib.ulm_last_error()
    st = lib.ulm_norm_conv_bwd(P, nat.ULM_F32, P, P, P, 4, P, nat.ULM_F32, P, nat.ULM_F32, P, P, P, P, P, 0, 2, 8,
                               1 << 20, P)
    assert st == nat.ULM_ERR_INVALID and b"too large" in lib.ulm_last_error()
    assert lib.ulm_norm_conv_bwd_workspace_bytes(2, 8, 1 << 20, 4) == 0
    # the block's fast memory: address inputs missing, y aliasing x
    st = lib.ulm_block_fm_fwd(P, nat.ULM_BF16, P, P, P, nat.ULM_BF16, P, P, P, nat.ULM_BF16, P, P, P, 0, P, 0,
                              2, 64, 32, 32, P)
    assert st == nat.ULM_ERR_INVALID and b"null pointer" in lib.ulm_last_error()
    x = ctypes.c_void_p(16)
    st = lib.ulm_block_fm_fwd(x, nat.ULM_BF16, P, x, x, nat.ULM_BF16, x, x, x, nat.ULM_BF16, x, x, x, 1 << 40, x,
                              1 << 40, 2, 64, 32, 32, P)
    assert st == nat.ULM_ERR_INVALID and b"alias" in lib.ulm_last_error()
    st = lib.ulm_block_fm_bwd(P, 7, P, P, P, P, P, 0, nat.ULM_BF16, P, nat.ULM_BF16, P, nat.ULM_BF16, P, P,
                              nat.ULM_BF16, P, P, P, 0, 2, 64, 32, 32, P)
    assert st == nat.ULM_ERR_INVALID and b"bad dtype" in lib.ulm_last_error()
    # weight gradient: widths must be multiples of 8
    st = lib.ulm_wgrad(x, x, x, 64, 12, 16, P, 0, P)
    assert st == nat.ULM_ERR_INVALID and b"multiples of 8" in lib.ulm_last_error()
    st = lib.ulm_cast(P, 5, P, nat.ULM_F32, 4, P)
    assert st == nat.ULM_ERR_INVALID and b"bad dtype" in lib.ulm_last_error()
    # block parameters: sizes, pointers, the clamp range
    st = lib.ulm_block_params(P, P, -7.0, 12.0, 0, P, P, P)
    assert st == nat.ULM_ERR_INVALID and b"A=0" in lib.ulm_last_error()
    st = lib.ulm_block_params(P, None, -7.0, 12.0, 16, P, P, P)
    assert st == nat.ULM_ERR_INVALID and b"null pointer" in lib.ulm_last_error()
    st = lib.ulm_block_params_bwd(x, x, 12.0, -7.0, x, x, 16, x, x, P)
    assert st == nat.ULM_ERR_INVALID and b"empty clamp range" in lib.ulm_last_error()


def test_block_workspace_sizes(monkeypatch):
    lib = nat.lib()
    B, T, A, D = 16, 1024, 3072, 768
    # block-pair form: the products write the output (with its residual)
    # directly; the workspace holds the forward's operand tiles only
    assert lib.ulm_block_fm_fwd_workspace_bytes(B, T, A, D) == 2 * B * T * A * 2 + B * T * D * 2
    # the state form with a residual goes through fp32 partials of the 4 key groups
    with monkeypatch.context() as m:
        m.setenv("ULM_FM_PATH", "chunked")
        assert lib.ulm_block_fm_fwd_workspace_bytes(B, T, A, D) >= 4 * B * T * D * 4
    # one fp32 partial per split; one round of 256 workgroups of 256 x 256 tiles
    tiles = (768 // 256) * (3072 // 256)
    assert lib.ulm_wgrad_workspace_bytes(B * T, 768, 3072) == (256 // tiles) * 768 * 3072 * 4
    assert lib.ulm_wgrad_workspace_bytes(64, 8, 16) == 0   # too short to split: writes C directly
    # norm/conv backward: per-tile partials of dnorm_w and dconv_w, plus the column-sum staging
    assert lib.ulm_norm_conv_bwd_workspace_bytes(B, T, D, 4) >= B * (T // 16) * D * 5 * 4


def test_unified_block_input_checks():
    import kernel
    D, A = 8, 16
    args = dict(norm_w=torch.ones(D), conv_w=torch.zeros(D, 1, 4), key_w=torch.zeros(A, D), key_b=torch.zeros(A),
                log_eps=torch.zeros(()), val_w=torch.zeros(D, D), mu_w=torch.zeros(D, A), log_rate=torch.tensor(-2.3),
                log_w=torch.zeros(A), norm_eps=1e-5)
    with pytest.raises(ValueError, match="fp32"):
        kernel.unified_block(torch.zeros(2, 4, D, dtype=torch.bfloat16), **args)
    with pytest.raises(ValueError, match="disagree"):
        kernel.unified_block(torch.zeros(2, 4, D), **{**args, "mu_w": torch.zeros(A, D)})
    with pytest.raises(ValueError, match="log_rate"):
        kernel.unified_block(torch.zeros(2, 4, D), **{**args, "log_rate": torch.zeros(2)})
    with pytest.raises(ValueError, match="Kc"):
        kernel.unified_block(torch.zeros(2, 4, D), **{**args, "conv_w": torch.zeros(D, 1, 9)})
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        kernel.unified_block(torch.zeros(2, 4, D), **args)
