"""ulm_addr_bwd_noalloc (needs an MI355X): the address backward on the static
device scratch array against ulm_addr_bwd on a caller workspace, bit for bit,
on two calls in a row (the second smaller, so it runs on what the first left
in the array), and the rejection of a size past the array. Every case prints
its name before touching the GPU."""
import pytest
import torch

from helpers import say

pytestmark = pytest.mark.gpu

import ulm_native as nat  # noqa: E402
from ulm_native import call, ptr  # noqa: E402


def _inputs(M, A, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    pre = torch.randn(M, A, generator=gen).to(dtype).cuda()
    bias = (0.5 * torch.randn(A, generator=gen)).cuda()
    le = torch.tensor([0.3]).cuda()
    dr = torch.randn(M, A, generator=gen).cuda()
    denom = torch.empty(M, device="cuda")
    call("ulm_addr_fwd", ptr(pre), nat.dtype_code(dtype), ptr(bias), ptr(le), None, ptr(denom), M, A,
         nat.stream_of(pre))
    return pre, bias, le, dr, denom


def _both(M, A, dtype, seed):
    pre, bias, le, dr, denom = _inputs(M, A, dtype, seed)
    s = nat.stream_of(pre)
    cd = nat.dtype_code(dtype)
    outs = []
    for entry in ("ulm_addr_bwd", "ulm_addr_bwd_noalloc"):
        dpre = torch.full_like(pre, float("nan"))
        dbias = torch.full((A,), float("nan"), device="cuda")
        dle = torch.full((1,), float("nan"), device="cuda")
        if entry == "ulm_addr_bwd":
            wsb = nat.lib().ulm_addr_bwd_workspace_bytes(M, A)
            ws = torch.empty(wsb, device="cuda", dtype=torch.uint8)
            call(entry, ptr(pre), cd, ptr(bias), ptr(le), None, ptr(denom), ptr(dr), ptr(dpre), ptr(dbias), ptr(dle),
                 ptr(ws), wsb, M, A, s)
        else:
            call(entry, ptr(pre), cd, ptr(bias), ptr(le), None, ptr(denom), ptr(dr), ptr(dpre), ptr(dbias), ptr(dle),
                 M, A, s)
        torch.cuda.synchronize()
        outs.append((dpre, dbias, dle))
    return outs


def test_noalloc_matches_workspace_entry():
    # the 110M training shape (B*T = 16384 rows of 3072 slots), then a smaller fp32 call
    for M, A, dtype, seed in ((16384, 3072, torch.bfloat16, 1), (1000, 700, torch.float32, 2)):
        need = nat.lib().ulm_addr_bwd_workspace_bytes(M, A)
        say(f"ulm_addr_bwd_noalloc M={M} A={A} {dtype}: {need} bytes of scratch")
        assert need <= 8 << 20
        (a, b) = _both(M, A, dtype, seed)
        for x, y, name in zip(a, b, ("dpre", "dbias", "dlog_eps")):
            assert torch.isfinite(x).all(), name
            assert torch.equal(x, y), name


def test_noalloc_rejects_sizes_past_the_array():
    M, A = 65536, 3072   # 2048 row blocks of dbias partials: 24 MiB of scratch
    say(f"ulm_addr_bwd_noalloc M={M} A={A}: rejected on the host")
    assert nat.lib().ulm_addr_bwd_workspace_bytes(M, A) > 8 << 20
    x = torch.empty(1, device="cuda")
    with pytest.raises(RuntimeError, match="scratch"):
        call("ulm_addr_bwd_noalloc", ptr(x), nat.ULM_BF16, ptr(x), ptr(x), None, ptr(x), ptr(x), ptr(x), ptr(x),
             ptr(x), M, A, nat.stream_of(x))
