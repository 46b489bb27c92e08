#!/usr/bin/env python3
"""Benchmark of the MI355X fast-memory path.

One step = the fast-memory forward + backward (unified_memory and its
backward) of all 12 UnifiedBlocks of the 110M shape on one synthetic batch:
B=16, T=1024, D=768, A=3072 slots, v/dfast in bf16, r/q/stats fp32. Inputs
are resident in HBM before the timed region. Prints one JSON line:

  value      Mtok/s = B*T / step time
  products   which evaluation the library picks at this shape (ulm_fm_path):
             "pair" (block-pair tile GEMMs) or "chunked" (the chunked state form)
  roofline   the dominant kernel (pair_kernel, or la_kgroup_kernel on the
             chunked path): the algorithmic flops of every timed launch over
             their summed launch time, measured with HIP events on the stream
             each launch uses, against the 2516.6 TFLOP/s dense bf16 peak.
             The events run in a second pass of the same timed steps: an event
             record between two dependent kernels lengthens the gap between
             them, so the pass that gives value carries none.
             The algorithmic flops are those of the evaluation that runs: for
             the six block-pair products 6 (A + D) per causal pair (t, s) of a
             batch row (mfma_executed_tflops counts their whole 128 x 128 tiles,
             masked halves of the diagonal ones included); for the chunked
             products 4 K V + 2 C V per token and product.
             chunked_equivalent_tflops prices the same work in the chunked
             algorithm's 16AD + 8C(A + D) flops per token and block (a
             comparison with the reference's algorithm, not a utilisation);
             traffic is the HBM bytes per launch recorded under profiles/
  path_tflops / chunked_equivalent_tflops
             the whole step (statistics kernels included) in the chosen
             evaluation's algorithmic flops, and in the chunked form's
             16AD + 8C(A + D) flops per token (the same work priced as the
             reference's algorithm)
  chunked    the chunked state form (the reference's algorithm, `_la`) on
             the same 110M shape (forced by ULM_FM_PATH=chunked) and on
             B=2, T=8192 sequences of the same widths, which the library
             sends to it by itself; each with its la_kgroup_kernel roofline
  configs    one block of the 15M (B=32, T=256, D=288, A=1152) and 42M (B=16,
             T=1024, D=512, A=2048) shapes, and of the two shapes the reference
             publishes single-block times for (ref-15M: B=32, T=256, D=288,
             A=712, 1.56 ms; ref-42M: B=8, T=1024, D=512, A=1280, 3.18 ms; on an
             RTX 3090 Ti, docs/kernel.md:57-62)
  cpu_baseline  the oracle's chunked PyTorch form on the host cores (fp32,
             fwd+bwd of one block at B=1, T=1024), scaled to the 12-block step
  block      whole UnifiedBlocks (fused) fwd+bwd over the same shape under bf16
             autocast, and the same blocks op by op
  train_step one training step of the whole 12-layer UnifiedLM (embedding,
             fused blocks, 32000-way classifier, cross-entropy), fwd+bwd, bf16
             autocast, token ids uniform
  decode     batched recurrent decode at the 110M shape: 256 sequences, 12
             blocks, fp32 state (29 GB); the 512-position prompt in one
             parallel pass (UnifiedLM.prefill), then greedy steps; GB/s of the
             algorithmic bytes per step against 8 TB/s. Its cpu_baseline is
             the reference's own C decoder (run.c, built with its runomp
             flags by oracle/Makefile) on the host cores, one sequence, in the
             same algorithmic bytes per position; the oracle's
             forward_recurrent is reported beside it

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--decode-steps N]
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "unifiedlm.c_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "fast-memory fwd+bwd Mtokens/s at 110M shape (% bf16 MFMA peak); decode GB/s"
PEAK_BF16_TFLOPS = 2516.6
PEAK_HBM_GBPS = 8000.0
TRAFFIC_FILES = {"la_kgroup_kernel": os.path.join(ROOT, "profiles", "la_kgroup_kernel_traffic.txt"),
                 "pair_kernel": os.path.join(ROOT, "profiles", "pair_kernel_traffic.txt"),
                 "decode_read_kernel": os.path.join(ROOT, "profiles", "decode_read_kernel_traffic.txt")}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--shape", default="110M")
    p.add_argument("--decode-steps", type=int, default=256)
    p.add_argument("--prefill", type=int, default=512)
    p.add_argument("--decode-seqs", type=int, default=256)
    p.add_argument("--no-decode", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-block", action="store_true")
    p.add_argument("--no-step", action="store_true")
    p.add_argument("--no-configs", action="store_true")
    p.add_argument("--no-chunked", action="store_true")
    p.add_argument("--no-address", action="store_true")
    p.add_argument("--only", choices=("block", "step", "decode", "address"),
                   help="profiling: run one leg alone (the fused block leg without its op-by-op pass, the "
                        "training step, the decode leg without its CPU baselines, or the relu^2 address) and "
                        "print its record instead of the benchmark line")
    p.add_argument("--copy-probe", type=int, default=0, metavar="MB",
                   help="first run one plain fp32 copy kernel over MB megabytes (a known-size reference for "
                        "hardware byte counters)")
    return p.parse_args()


def fm_path_name(code):
    return {0: "generic", 1: "chunked", 2: "pair"}.get(code, "invalid")


def bench_training(torch, args, shape=None, steps=None, warmup=None):
    """unified_memory forward + backward of every block of a shape (r fp32, v
    and dfast bf16, the upstream gradient of q fp32). The roofline object
    prices the launches the library times (every chunked or block-pair
    product launch) with that evaluation's algorithmic flops."""
    import kernel
    import ulm_native
    import workloads
    shape = shape or args.shape
    steps = args.steps if steps is None else steps
    warmup = args.warmup if warmup is None else warmup
    cfg = workloads.SHAPES[shape]
    B, T, D, A, L = cfg["B"], cfg["T"], cfg["D"], cfg["A"], cfg["blocks"]
    dev = torch.device("cuda:0")
    path = fm_path_name(ulm_native.lib().ulm_fm_path(B, T, A, D))
    log(f"training workload {shape}: B={B} T={T} D={D} A={A} blocks={L}, {path} products")
    blocks = []
    for l in range(L):
        r, v, g, w = workloads.block_inputs(B, T, D, A, seed=1000 + l, device=dev, v_dtype=torch.bfloat16)
        blocks.append([t.requires_grad_(True) for t in (r, v, g, w)])
    gen = torch.Generator(device=dev).manual_seed(5)
    dq_up = (torch.randn(B, T, A, device=dev, generator=gen) * 0.01).contiguous()
    df_up = torch.randn(B, T, D, device=dev, generator=gen).to(torch.bfloat16)

    def step():
        outs = [kernel.unified_memory(*blk) for blk in blocks]
        for blk, (q, fast) in zip(reversed(blocks), reversed(outs)):
            torch.autograd.grad((q, fast), blk, (dq_up, df_up))

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # The timed steps run without the per-launch HIP events: each event record
    # sits between two dependent kernels on the stream and lengthens the gap
    # between them by several microseconds. A second pass of the same steps
    # carries the events that time every product launch for the roofline.
    t0 = time.perf_counter()
    for i in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / steps
    per_step = 6 if path == "pair" else 4
    with ulm_native.LaTimer(max_launches=per_step * L * steps + 16) as timer:
        t2 = time.perf_counter()
        for i in range(steps):
            step()
        torch.cuda.synchronize()
        t3 = time.perf_counter()
    ms_step_events = (t3 - t2) * 1e3 / steps
    launch_ms = timer.total_ms / max(timer.launches, 1)
    if path == "pair":
        kname = "pair_kernel"
        # the six block-pair products' own algorithmic flops, 6 (A + D) per
        # causal pair (t, s), over their summed launch time
        flops_launches = workloads.pair_flops(B, T, A, D) * L * steps
        tile_flops = workloads.pair_tile_flops(B, T, A, D) * L * steps
        flops_step = workloads.pair_flops(B, T, A, D) * L
        note = ("the six block-pair products (scores, apply, dscores, dq_f with the backward statistics, dk_f into dr, "
                "dv) of every block, 6 (A + D) flops per causal pair (t, s); mfma_executed_tflops counts their whole "
                "128 x 128 tiles (the diagonal ones computed in full and masked), "
                f"{workloads.pair_tile_flops(B, T, A, D) / workloads.pair_flops(B, T, A, D):.3f}x that")
    else:
        kname = "la_kgroup_kernel"
        # fwd and dv contract keys A into values D, dq and dk keys D into values A
        flops_launches = (workloads.la_kernel_flops(B, T, A, D) + workloads.la_kernel_flops(B, T, D, A)) / 2 * timer.launches
        tile_flops = None
        flops_step = 4 * workloads.la_flops(B, T, A, D) * L
        note = "the four chunked products of every block, 4 K V + 2 C V per token and product"
    secs = timer.total_ms * 1e-3
    achieved = flops_launches / secs / 1e12 if secs > 0 else 0.0
    # the same launches' work priced in the chunked algorithm's 16AD + 8C(A + D) per token and block
    chunked_eq_launch = (workloads.chunked_flops_per_token(A, D) * B * T * L * steps / secs / 1e12
                         if secs > 0 and path == "pair" else None)
    traffic = None
    tfile = TRAFFIC_FILES.get(kname)
    if tfile and os.path.exists(tfile) and shape == "110M":
        with open(tfile) as f:
            rec = json.load(f)
        if rec.get("path", path) == path:
            traffic = rec.get("bytes_per_launch")
    path_tflops = flops_step / (ms_step * 1e-3) / 1e12
    chunk_eq = workloads.chunked_flops_per_token(A, D) * L * B * T / (ms_step * 1e-3) / 1e12
    log(f"step {ms_step:.2f} ms ({ms_step_events:.2f} ms with the launch events), {kname} {launch_ms:.3f} ms x "
        f"{timer.launches} launches, {achieved:.1f} TFLOP/s")
    roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
            "traffic_source": "recorded (profiles/)" if traffic else None, "kernel": kname, "flops": note,
            "avg_launch_ms": round(launch_ms, 4), "launches_timed": timer.launches,
            "launch_events": "a second pass of the timed steps with a HIP event pair around every product launch on "
                             f"its stream ({ms_step_events:.3f} ms per step with them)"}
    if tile_flops and secs > 0:
        roof["mfma_executed_tflops"] = round(tile_flops / secs / 1e12, 2)
        roof["mfma_executed_frac"] = round(tile_flops / secs / 1e12 / PEAK_BF16_TFLOPS, 4)
    if chunked_eq_launch:
        roof["chunked_equivalent_tflops"] = round(chunked_eq_launch, 2)
        roof["chunked_equivalent_frac"] = round(chunked_eq_launch / PEAK_BF16_TFLOPS, 4)
    if path == "pair" and timer.products:
        roof["products"] = pair_product_rooflines(timer.products, B, T, A, D,
                                                  tfile if traffic is not None else None)
        log("  per product: " + ", ".join(f"{k} {v['avg_us']} us" + (f" {v['frac_hbm_peak']:.2f} HBM" if "GBps" in v
                                                                       else f" {v['frac_bf16_peak']:.2f} MFMA")
                                          for k, v in roof["products"].items()))
    return dict(B=B, T=T, D=D, A=A, L=L, path=path, ms_step=ms_step, value=B * T / (ms_step * 1e-3) / 1e6,
                roofline=roof, path_tflops=path_tflops, chunked_equivalent_tflops=chunk_eq)


def pair_product_rooflines(products, B, T, A, D, traffic_file):
    """Each block-pair product on its own: average launch time (the HIP events
    of the timed pass, on the stream it ran on), its own algorithmic flops
    (2A or 2D per causal pair) against the bf16 MFMA peak and, where the
    recorded counters of this shape are at hand, its HBM bytes per launch
    against the 8 TB/s peak. dv runs beside dscores on the second stream, so
    both times include their sharing of the CUs."""
    pairs = B * T * (T + 1) / 2
    width = {"scores": A, "apply": D, "dscores": D, "dv": D, "dq_f": A, "dk_f": A, "state": A}
    recorded = {}
    if traffic_file:
        with open(traffic_file) as f:
            for key, rec in json.load(f).get("products", {}).items():
                for name in ("dscores", "dq_f", "dk_f"):
                    if key.startswith(name):
                        recorded[name] = rec["bytes"]
                if key.startswith("scores ("):
                    recorded["scores"] = rec["bytes"]
                if key.startswith("apply and dv"):
                    recorded["apply"] = recorded["dv"] = rec["bytes"]
    out = {}
    for name, (ms, n) in products.items():
        secs = ms * 1e-3 / n
        tflops = 2 * width[name] * pairs / secs / 1e12
        row = {"avg_us": round(secs * 1e6, 1), "launches": n, "tflops": round(tflops, 1),
               "frac_bf16_peak": round(tflops / PEAK_BF16_TFLOPS, 4)}
        if name in recorded:
            gbps = recorded[name] / secs / 1e9
            row.update(hbm_MB=round(recorded[name] / 1e6, 1), GBps=round(gbps, 1),
                       frac_hbm_peak=round(gbps / PEAK_HBM_GBPS, 4))
        out[name] = row
    return out


def bench_address(torch, args):
    """The relu^2 slot address (model.py:70-72; ulm_addr_fwd / ulm_addr_bwd) on
    its own at the 110M training rows: M = B T = 16384 rows of A = 3072 slots,
    pre in bf16 as the block's key GEMM leaves it under autocast. HIP events
    around K launches each, on the stream they run on. Priced in the
    algorithmic bytes per element: forward 2 (pre in) + 4 (r out), backward
    4 (dr) + 4 (r) + 2 (pre) in and 2 (dpre) out."""
    import kernel
    import ulm_native as nat
    M, A = 16 * 1024, 3072
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(9)
    pre = torch.randn(M, A, device=dev, generator=gen).to(torch.bfloat16)
    bias = torch.randn(A, device=dev, generator=gen) * 0.5
    le = torch.tensor([0.3], device=dev)
    dr = torch.randn(M, A, device=dev, generator=gen)
    r = torch.empty(M, A, device=dev)
    denom = torch.empty(M, device=dev)
    dpre = torch.empty_like(pre)
    dbias = torch.empty(A, device=dev)
    dle = torch.empty(1, device=dev)
    wsb = nat.lib().ulm_addr_bwd_workspace_bytes(M, A)
    ws = torch.empty(max(wsb, 1), device=dev, dtype=torch.uint8)
    st = nat.stream_of(pre)
    pdt = nat.dtype_code(pre.dtype)

    def fwd():
        nat.call("ulm_addr_fwd", nat.ptr(pre), pdt, nat.ptr(bias), nat.ptr(le), nat.ptr(r), nat.ptr(denom), M, A, st)

    def bwd():
        nat.call("ulm_addr_bwd", nat.ptr(pre), pdt, nat.ptr(bias), nat.ptr(le), nat.ptr(r), nat.ptr(denom),
                 nat.ptr(dr), nat.ptr(dpre), nat.ptr(dbias), nat.ptr(dle), nat.ptr(ws), wsb, M, A, st)

    out = {"workload": f"relu^2 address of M={M} rows x A={A} slots (the 110M training rows), bf16 pre"}
    k = max(args.steps, 20)
    for name, fn, nbytes in (("forward", fwd, M * A * (2 + 4)), ("backward", bwd, M * A * (4 + 4 + 2 + 2))):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(k):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / k
        gbps = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"avg_launch_ms": round(ms, 4), "bytes": nbytes, "GBps": round(gbps, 1),
                     "frac_hbm_peak": round(gbps / PEAK_HBM_GBPS, 4), "launches_timed": k}
        log(f"address {name}: {ms * 1e3:.1f} us per call, {gbps:.0f} GB/s ({gbps / PEAK_HBM_GBPS:.2f} of HBM peak)")
    return out


def bench_chunked(torch, args):
    """The chunked state form (`_la`, kernel.py:183-196; the K-group kernel) at
    the 110M widths: the training shape with the form forced, and sequences of
    8192 positions (B=2, the same 16384 tokens per step), which the library
    sends to it by itself."""
    out = {}
    saved = os.environ.get("ULM_FM_PATH")
    try:
        os.environ["ULM_FM_PATH"] = "chunked"
        t = bench_training(torch, args, shape="110M", steps=max(args.steps // 2, 5), warmup=2)
    finally:
        if saved is None:
            os.environ.pop("ULM_FM_PATH", None)
        else:
            os.environ["ULM_FM_PATH"] = saved
    legs = [("110M (forced)", t)]
    if saved is None:
        legs.append(("110M-T8192", bench_training(torch, args, shape="110M-T8192", steps=max(args.steps // 2, 5),
                                                  warmup=2)))
    for name, t in legs:
        out[name] = {"workload": f"fast-memory fwd+bwd, {t['L']} blocks, B={t['B']} T={t['T']} D={t['D']} "
                                 f"A={t['A']}, chunked state form",
                     "path": t["path"], "ms_per_step": round(t["ms_step"], 3), "Mtok_per_s": round(t["value"], 4),
                     "tflops": round(t["path_tflops"], 2),
                     "frac_bf16_peak": round(t["path_tflops"] / PEAK_BF16_TFLOPS, 4),
                     "roofline": t["roofline"]}
    return out


def bench_configs(torch, args):
    """Single-block fast-memory fwd + bwd at the 15M (B=32, T=256, D=288,
    A=1152) and 42M (B=16, T=1024, D=512, A=2048) shapes, and at the two
    shapes the reference publishes single-block times for (D=288, A=712 and
    D=512, A=1280; docs/kernel.md:57-62, on an RTX 3090 Ti: other hardware)."""
    import workloads
    out = {}
    for shape in ("15M", "42M", "ref-15M", "ref-42M"):
        t = bench_training(torch, args, shape=shape, steps=max(args.steps, 50), warmup=max(args.warmup, 5))
        out[shape] = {"workload": f"fast-memory fwd+bwd, one block of the {shape} shape (B={t['B']}, T={t['T']}, "
                                  f"D={t['D']}, A={t['A']})",
                      "path": t["path"], "ms_per_block": round(t["ms_step"], 4), "Mtok_per_s": round(t["value"], 4),
                      "tflops": round(t["path_tflops"], 2),
                      "frac_bf16_peak": round(t["path_tflops"] / PEAK_BF16_TFLOPS, 4),
                      "chunked_equivalent_tflops": round(t["chunked_equivalent_tflops"], 2),
                      "roofline": t["roofline"]}
        ref_ms = workloads.SHAPES[shape].get("reference_ms")
        if ref_ms:
            out[shape]["reference_ms_per_block"] = ref_ms
            out[shape]["reference_hardware"] = "RTX 3090 Ti, Triton (docs/kernel.md:57-62)"
            out[shape]["speedup_vs_reference"] = round(ref_ms / t["ms_step"], 2)
    return out


def bench_block(torch, args, composed=True):
    """Whole UnifiedBlocks (model.py:77-85) forward + backward over the training
    workload's shape under bf16 autocast: the fused block and the op-by-op
    path (forward_composed) on the same weights and input."""
    import workloads
    from model import ModelArgs, UnifiedLM
    cfg = workloads.SHAPES[args.shape]
    B, T, D, A, L = cfg["B"], cfg["T"], cfg["D"], cfg["A"], cfg["blocks"]
    dev = torch.device("cuda:0")
    log(f"block workload {args.shape}: B={B} T={T} D={D} A={A} blocks={L}, bf16 autocast")
    model = UnifiedLM(ModelArgs(dim=D, n_layers=L, hidden_dim=A, vocab_size=256, max_seq_len=T))
    workloads.init_decode_model(model, seed=43)
    blocks = model.layers.to(dev).train()
    gen = torch.Generator(device=dev).manual_seed(7)
    x0 = torch.randn(B, T, D, device=dev, generator=gen)
    dout = torch.randn(B, T, D, device=dev, generator=gen)

    def step(fused):
        for prm in blocks.parameters():
            prm.grad = None
        x = x0.detach().requires_grad_(True)
        h = x
        with torch.autocast("cuda", dtype=torch.bfloat16):
            for blk in blocks:
                h = blk(h) if fused else blk.forward_composed(h)
        h.backward(dout)

    def timed(fused):
        for _ in range(args.warmup):
            step(fused)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step(fused)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / args.steps

    ms = timed(True)
    import ulm_native
    path = fm_path_name(ulm_native.lib().ulm_fm_path(B, T, A, D))
    ftok = workloads.block_flops_per_token(T, A, D, path=path) * L
    rec = {"workload": f"UnifiedBlock fwd+bwd, {L} blocks of the {args.shape} shape, bf16 autocast",
           "ms_per_step": round(ms, 3), "Mtok_per_s": round(B * T / (ms * 1e-3) / 1e6, 4),
           "tflops": round(ftok * B * T / (ms * 1e-3) / 1e12, 2)}
    if not composed:
        log(f"block step {ms:.2f} ms fused")
        return rec
    ms_c = timed(False)
    log(f"block step {ms:.2f} ms fused, {ms_c:.2f} ms op by op")
    return {**rec, "composed_ms_per_step": round(ms_c, 3),
            "composed_Mtok_per_s": round(B * T / (ms_c * 1e-3) / 1e6, 4), "speedup_vs_composed": round(ms_c / ms, 3)}


def bench_train_step(torch, args):
    """One training step of the whole 12-layer UnifiedLM at the 110M shape
    (model.py:149-162): embedding, the fused blocks, final RMSNorm, the tied
    32000-way classifier and the cross-entropy loss, forward + backward under
    bf16 autocast, token ids uniform over the vocabulary; no optimizer step."""
    import workloads
    from model import ModelArgs, UnifiedLM
    cfg = workloads.SHAPES[args.shape]
    B, T, D, A, L = cfg["B"], cfg["T"], cfg["D"], cfg["A"], cfg["blocks"]
    V = workloads.DECODE_110M["vocab"]
    dev = torch.device("cuda:0")
    log(f"training step {args.shape}: B={B} T={T} D={D} A={A} blocks={L} vocab={V}, bf16 autocast")
    torch.manual_seed(1)
    model = UnifiedLM(ModelArgs(dim=D, n_layers=L, hidden_dim=A, vocab_size=V, max_seq_len=T))
    workloads.init_decode_model(model, seed=44)
    model = model.to(dev).train()
    gen = torch.Generator(device=dev).manual_seed(9)
    tokens = torch.randint(0, V, (B, T + 1), device=dev, generator=gen)
    x, y = tokens[:, :-1].contiguous(), tokens[:, 1:].contiguous()

    def step():
        for prm in model.parameters():
            prm.grad = None
        with torch.autocast("cuda", dtype=torch.bfloat16):
            model(x, y)
        model.last_loss.backward()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    # per token: every block's GEMMs and fast memory, plus the classifier (2 V D forward, twice that backward)
    import ulm_native
    path = fm_path_name(ulm_native.lib().ulm_fm_path(B, T, A, D))
    ftok = workloads.block_flops_per_token(T, A, D, path=path) * L + 6 * V * D
    log(f"training step {ms:.2f} ms, loss {model.last_loss.item():.3f}")
    return {"workload": f"UnifiedLM {args.shape} training step fwd+bwd: embedding, {L} fused blocks, classifier "
                        f"over {V} tokens, cross-entropy; bf16 autocast; no optimizer",
            "ms_per_step": round(ms, 3), "Mtok_per_s": round(B * T / (ms * 1e-3) / 1e6, 4),
            "tflops": round(ftok * B * T / (ms * 1e-3) / 1e12, 2), "loss": round(model.last_loss.item(), 4)}


def bench_cpu_baseline(torch, train):
    """The oracle's chunked PyTorch form, fwd+bwd of one block at B=1, fp32."""
    from oracle import fastmem as fm
    import workloads
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    T, D, A, L = train["T"], train["D"], train["A"], train["L"]
    r, v, g, w = workloads.block_inputs(1, T, D, A, seed=1000, device="cpu", v_dtype=torch.float32)
    leaves = [t.detach().requires_grad_(True) for t in (r, v, g, w)]
    dq = torch.randn(1, T, A) * 0.01
    df = torch.randn(1, T, D)

    def run():
        q, fast = fm.fast_memory(*leaves, form="chunked", chunk=64)
        torch.autograd.grad((q, fast), leaves, (dq, df))

    run()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t_block = sorted(times)[1]
    value = T / (t_block * L) / 1e6   # Mtok/s of the 12-block fwd+bwd
    cpu = ""
    try:
        with open("/proc/cpuinfo") as f:
            cpu = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    log(f"cpu baseline: {t_block * 1e3:.1f} ms per block (B=1), {threads} threads, {cpu}")
    return {"value": round(value, 6), "unit": "Mtok/s", "cores": threads, "kind": "port",
            "sample": f"oracle chunked_fast_memory fp32 fwd+bwd, one block at B=1 T={T} D={D} A={A}, "
                      f"median of 3 after 1 warm-up ({t_block * 1e3:.1f} ms), scaled to {L} blocks per token",
            "cpu_model": cpu}


def bench_decode(torch, args):
    from model import ModelArgs, UnifiedLM
    import workloads
    c = workloads.DECODE_110M
    N, D, A, L, V = args.decode_seqs, c["D"], c["A"], c["blocks"], c["vocab"]
    dev = torch.device("cuda:0")
    log(f"decode workload: N={N} D={D} A={A} blocks={L} vocab={V} prefill={args.prefill} steps={args.decode_steps}")
    torch.manual_seed(0)
    model = UnifiedLM(ModelArgs(dim=D, n_layers=L, hidden_dim=A, vocab_size=V, max_seq_len=1024))
    workloads.init_decode_model(model, seed=42)
    model = model.to(dev).eval()
    gen = torch.Generator(device=dev).manual_seed(3)
    prompt = torch.randint(0, V, (N, args.prefill), device=dev, generator=gen)
    # the prompt in one parallel pass (UnifiedLM.prefill), which leaves the same
    # decode states as stepping through it position by position; its GEMMs take
    # bf16 operands under autocast, as the training step's do
    with torch.autocast("cuda", dtype=torch.bfloat16):
        warm = model.prefill(prompt)   # untimed: first launches and the allocator's first 40 GB
        del warm
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        logits, states = model.prefill(prompt)
        torch.cuda.synchronize()
    t_pre = time.perf_counter()
    import ulm_native
    pre_form = {1: "chunked state form", 2: "block-pair products, the state as one product over positions"}.get(
        ulm_native.lib().ulm_fm_prefill_path(N, args.prefill, A, D), "unsupported")
    log(f"  prefill {args.prefill} positions x {N} sequences in one pass ({pre_form}): {(t_pre - t0) * 1e3:.1f} ms")
    nxt = logits.argmax(-1)
    for _ in range(2):   # untimed: first launches of the decode kernels
        logits = model.step(nxt, states)
        nxt = logits.argmax(-1)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for i in range(args.decode_steps):
        logits = model.step(nxt, states)
        nxt = logits.argmax(-1)
        if i % 64 == 63:
            torch.cuda.synchronize()
            log(f"  decode {i + 1}/{args.decode_steps}")
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    import model as model_mod
    deferred = A % 4 == 0 and A <= 4096
    J = model_mod.DECODE_PENDING if deferred else 1
    bytes_step = workloads.decode_bytes_per_step(N, L, A, D, V, pending=J)
    bytes_each = workloads.decode_bytes_per_step(N, L, A, D, V, pending=1)
    step_ms = (t2 - t1) * 1e3 / max(args.decode_steps, 1)
    pre_ms = (t_pre - t0) * 1e3
    gbps = bytes_step / (step_ms * 1e-3) / 1e9
    log(f"decode {step_ms:.2f} ms/step, {gbps:.0f} GB/s ({J} positions per state write-back; "
        f"{bytes_each / (step_ms * 1e-3) / 1e9:.0f} GB/s in the bytes of a write at every position); "
        f"prefill {pre_ms:.1f} ms ({N * args.prefill / (pre_ms * 1e-3) / 1e6:.2f} Mtok/s)")
    # a second pass of 2 J positions with a HIP event pair around every state
    # launch, on the stream it runs on (torch's current stream)
    kernel_ms = {"decode_read_kernel": [], "decode_flush_kernel": []}
    if deferred:
        real = model_mod.decode_deferred

        def timed(S, pv, pr, m, flush, *rest, **kw):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            out = real(S, pv, pr, m, flush, *rest, **kw)
            e1.record()
            kernel_ms["decode_flush_kernel" if flush else "decode_read_kernel"].append((e0, e1))
            return out

        model_mod.decode_deferred = timed
        try:
            for _ in range(2 * J):
                logits = model.step(nxt, states)
                nxt = logits.argmax(-1)
            torch.cuda.synchronize()
        finally:
            model_mod.decode_deferred = real
    launch = {k: (sum(a.elapsed_time(b) for a, b in v) / len(v) if v else None) for k, v in kernel_ms.items()}
    # algorithmic bytes per launch: S read (and for the write-back, written), q, and the m pending terms
    read_bytes = N * D * A * 4 + N * A * 4 + N * (J + 1) // 2 * (D + 1) * 4
    flush_bytes = 2 * N * D * A * 4 + N * A * 4 + N * J * (A + D) * 4
    traffic = None
    tfile = TRAFFIC_FILES["decode_read_kernel"]
    if os.path.exists(tfile) and N == 256:
        with open(tfile) as f:
            traffic = json.load(f).get("bytes_per_launch")
    cpu = cpu_port = None
    if not args.no_cpu:
        cpu_port = bench_decode_cpu(torch, model, c)
        cpu = bench_decode_runc(torch, model, c)
    read_gbps = read_bytes / (launch["decode_read_kernel"] * 1e-3) / 1e9 if launch["decode_read_kernel"] else None
    flush_gbps = flush_bytes / (launch["decode_flush_kernel"] * 1e-3) / 1e9 if launch["decode_flush_kernel"] else None
    if read_gbps:
        log(f"  decode_read_kernel {launch['decode_read_kernel']:.3f} ms ({read_gbps:.0f} GB/s), "
            f"decode_flush_kernel {launch['decode_flush_kernel']:.3f} ms ({flush_gbps:.0f} GB/s)")
    roofline = {"bound": "hbm", "achieved": round(read_gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                "frac": round(read_gbps / PEAK_HBM_GBPS, 4), "traffic": traffic,
                "kernel": "decode_read_kernel",
                "bytes": "S read (N D A fp32), q, the pending terms' values and weights, per block and position",
                "avg_launch_ms": round(launch["decode_read_kernel"], 4),
                "launches_timed": len(kernel_ms["decode_read_kernel"]),
                "launch_events": "a second pass of 2 J positions with a HIP event pair around every state launch",
                "flush_kernel": "decode_flush_kernel", "flush_avg_launch_ms": round(launch["decode_flush_kernel"], 4),
                "flush_achieved": round(flush_gbps, 1), "flush_frac": round(flush_gbps / PEAK_HBM_GBPS, 4),
                "traffic_source": "recorded (profiles/)" if traffic else None} if read_gbps else \
        {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
         "frac": round(gbps / PEAK_HBM_GBPS, 4), "traffic": None, "kernel": "decode_state_kernel (whole step)"}
    return {"metric": "decode GB/s", "value": round(gbps, 1), "unit": "GB/s", "ms_per_step": round(step_ms, 3),
            "tok_per_s": round(N / (step_ms * 1e-3), 1),
            "state_write_back_every": J,
            "frac_hbm_peak": round(gbps / PEAK_HBM_GBPS, 4),
            "write_each_position_equivalent_GBps": round(bytes_each / (step_ms * 1e-3) / 1e9, 1),
            "prefill": f"one pass of the prompt (UnifiedLM.prefill, fused blocks, GEMMs bf16 under autocast; {pre_form})",
            "prefill_ms": round(pre_ms, 2), "prefill_ms_per_position": round(pre_ms / max(args.prefill, 1), 4),
            "prefill_Mtok_per_s": round(N * args.prefill / (pre_ms * 1e-3) / 1e6, 3), "bytes_per_step": bytes_step,
            "state_GB": round(N * L * D * A * 4 / 1e9, 2),
            "roofline": roofline,
            "cpu_baseline": cpu or cpu_port,
            "cpu_baseline_port": cpu_port if cpu else None,
            "config": {"N": N, "D": D, "A": A, "blocks": L, "vocab": V, "prefill": args.prefill,
                       "steps": args.decode_steps}}


def bench_decode_cpu(torch, model, c, n_seq=8, n_pos=12):
    """The oracle's forward_recurrent (model.py:164-175) in fp32 on the host
    cores: n_seq sequences of n_pos positions of the 110M decode model, timed
    after one position of warm-up, in GB/s of the same algorithmic bytes per
    decode position as the GPU figure (at N = n_seq)."""
    from oracle import fastmem as fm
    import workloads
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    params = {n: p.detach().float().cpu() for n, p in model.named_parameters()}
    gen = torch.Generator().manual_seed(11)
    tokens = torch.randint(0, c["vocab"], (n_seq, n_pos + 1), generator=gen)
    with torch.no_grad():
        fm.forward_recurrent(params, tokens[:, :1])   # warm-up
        t0 = time.perf_counter()
        fm.forward_recurrent(params, tokens[:, 1:])
        dt = time.perf_counter() - t0
    step_s = dt / n_pos
    bytes_step = workloads.decode_bytes_per_step(n_seq, c["blocks"], c["A"], c["D"], c["vocab"])
    log(f"decode cpu baseline: {step_s * 1e3:.1f} ms per position for {n_seq} sequences, {threads} threads")
    return {"value": round(bytes_step / step_s / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "tok_per_s": round(n_seq / step_s, 2),
            "sample": f"oracle forward_recurrent fp32 (the 110M decode model: D={c['D']}, A={c['A']}, "
                      f"{c['blocks']} blocks, vocab {c['vocab']}), {n_seq} sequences x {n_pos} positions from the "
                      f"prior state ({dt:.2f} s), algorithmic bytes per position at N={n_seq}"}


def bench_decode_runc(torch, model, c, n_pos=2048):
    """The reference's own C decoder (run.c:193-265, built unmodified from its
    source with its runomp flags by oracle/Makefile) on the host cores: the
    110M decode model exported to its ULMe v1 format, one sequence, n_pos
    positions from the prior state after 2 of warm-up, in GB/s of the
    algorithmic bytes per decode position at N=1. None where that build is
    absent."""
    import tempfile
    from oracle import runc
    import ulme
    import workloads
    if not runc.available(omp=True):
        log("decode cpu baseline: oracle/_ref/librunc_ref_omp.so not built, skipped")
        return None
    threads = int(os.environ.get("OMP_NUM_THREADS", len(os.sched_getaffinity(0))))
    gen = torch.Generator().manual_seed(12)
    tokens = torch.randint(0, c["vocab"], (n_pos + 2,), generator=gen).tolist()
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "decode_110M.bin")
        ulme.export_ulme(model, path)
        ref = runc.RuncReference(path, omp=True)
    ref.reset()
    for tok in tokens[:2]:
        ref.forward(tok)
    t0 = time.perf_counter()
    for tok in tokens[2:]:
        ref.forward(tok)
    dt = time.perf_counter() - t0
    step_s = dt / n_pos
    bytes_step = workloads.decode_bytes_per_step(1, c["blocks"], c["A"], c["D"], c["vocab"])
    log(f"decode cpu baseline (run.c, OpenMP): {step_s * 1e3:.1f} ms per position, {threads} threads")
    return {"value": round(bytes_step / step_s / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "reference",
            "tok_per_s": round(1 / step_s, 2),
            "sample": f"run.c forward() (built with -Ofast -fopenmp, its runomp target) on the 110M decode model "
                      f"exported to ULMe v1 (D={c['D']}, A={c['A']}, {c['blocks']} blocks, vocab {c['vocab']}), one "
                      f"sequence x {n_pos} positions from the prior state after 2 of warm-up ({dt:.2f} s), "
                      "algorithmic bytes per position at N=1"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: the library has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the fast-memory path shards by sequence with no communication for decode and a DDP "
              "all-reduce for training, which is not built here.", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if args.copy_probe > 0:
        n = args.copy_probe * (1 << 20) // 4
        x = torch.ones(n, device="cuda:0")
        y = torch.empty_like(x)
        torch.mul(x, 1.0, out=y)   # reads and writes exactly 4 n bytes
        torch.cuda.synchronize()
        log(f"copy probe: {4 * n} bytes read, {4 * n} bytes written")
        del x, y
    if args.only:
        if args.only == "decode":
            args.no_cpu = True
        legs = {"block": lambda: bench_block(torch, args, composed=False),
                "step": lambda: bench_train_step(torch, args), "decode": lambda: bench_decode(torch, args),
                "address": lambda: bench_address(torch, args)}
        rec = legs[args.only]()
        print(json.dumps({"leg": args.only, "steps": args.steps, "warmup": args.warmup, **rec}), flush=True)
        return
    train = bench_training(torch, args)
    configs = None if args.no_configs else bench_configs(torch, args)
    chunked = None if args.no_chunked else bench_chunked(torch, args)
    address = None if args.no_address else bench_address(torch, args)
    cpu = None if args.no_cpu else bench_cpu_baseline(torch, train)
    block = None if args.no_block else bench_block(torch, args)
    train_step = None if args.no_step else bench_train_step(torch, args)
    decode = None if args.no_decode else bench_decode(torch, args)
    out = {
        "metric": METRIC,
        "value": round(train["value"], 4),
        "unit": "Mtok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(train["ms_step"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"fast-memory fwd+bwd, {train['L']} blocks of the {args.shape} shape",
                   "global_batch": train["B"], "seq_len": train["T"], "dim": train["D"], "slots": train["A"],
                   "blocks": train["L"],
                   **({"position_block": 128} if train["path"] == "pair" else {"chunk": 64}),
                   "parallelism": "single GPU"},
        "products": train["path"],
        "path_tflops": round(train["path_tflops"], 2),
        "path_frac_bf16_peak": round(train["path_tflops"] / PEAK_BF16_TFLOPS, 4),
        "chunked_equivalent_tflops": round(train["chunked_equivalent_tflops"], 2),
        "chunked_equivalent_frac_bf16_peak": round(train["chunked_equivalent_tflops"] / PEAK_BF16_TFLOPS, 4),
        "roofline": train["roofline"],
        "configs": configs,
        "chunked": chunked,
        "address": address,
        "cpu_baseline": cpu,
        "block": block,
        "train_step": train_step,
        "decode": decode,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
