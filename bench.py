"""Benchmark: achieved HBM GB/s of the mHC-lite K1/K3/K4 forward+backward
kernels at T=65536, n=4, C=1024 (bf16) on one MI355X.

One "step" is one pass of the hot path over one batch: the six HIP kernels
K1 fwd, K1 bwd-dx, K3 fwd, K3 bwd, K4 fwd, K4 bwd, each on its own synthetic
input resident in HBM (the kernel microbenchmark of the reference's
scripts/benchmark_kernels.py, with its mandatory-bytes model, :64-105).

Prints ONE JSON line.  ``value`` = sum of the six kernels' algorithmic bytes /
measured step time (K steps of bare launches between two events).  Per-kernel
durations come from a second pass of K steps with an event pair around each
launch; ``roofline`` describes the dominant kernel (largest average duration),
timed with those HIP events on the stream it runs on.  ``kernels_isolated``
times each kernel alone (repeated launches of that kernel), ``kernels_cold``
each kernel after a flush of L2 and the memory-side cache (CacheFlush), and
``step_cold`` the whole step after such a flush.
``ceilings_GBps`` are 1 GiB streaming probes with the nontemporal hint, as the
kernels' streaming loads and stores carry (ordinary-access probes beside them
are labelled ``*_ordinary``).
Extra fields report K1's full backward (fused grad_W vs the reference's matmul), a whole
MHCLiteBlock forward + backward with the fused path vs the reference's rules
(at C and at 2C, i.e. the C=2048 block configuration), the same step at
T=4096 eager and replayed from a HIP graph,
and the eval-mode forward latency of the inference shapes (C=4096,
T = 1, 64, 257, 65537; eager and HIP-graph replay).
``cpu_baseline`` times the reference's PyTorch formulation of the same six ops
(fp32 autograd, restated in oracle/) on the host's cores, by default on the
whole workload (--cpu-tokens, --cpu-iters bound it), reported with the same
bytes model; ``cpu_block_config1`` the fp32 plain-path MHCLiteBlock forward +
backward at T=4096, C=1024 on the same cores (the golden configuration).

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--T 65536] [--C 1024]
The reference benchmark's command line (--T --C --n 4 --iters --seed --peak-gbps) is accepted.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "flash-mhc_amd"))
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

PEAK_GBPS = 8000.0  # MI355X HBM3E
METRIC = "achieved HBM GB/s (% of peak) for K1/K3/K4 fwd+bwd at T=65536,n=4,C=1024"
KERNELS = ("k1_fwd", "k1_bwd_dx", "k3_fwd", "k3_bwd", "k4_fwd", "k4_bwd")


def bytes_model(T: int, n: int, C: int, D: int) -> dict[str, int]:
    """Mandatory HBM bytes per launch (reference scripts/benchmark_kernels.py:64-105)."""
    bf, f4 = 2, 4
    nC = n * C
    return {
        "k1_fwd": bf * T * nC + bf * D * nC + bf * T * D + f4 * T,
        "k1_bwd_dx": bf * T * nC + bf * D * nC + 2 * bf * T * D + f4 * T + bf * T * nC,
        "k3_fwd": bf * T * nC + f4 * T * n + bf * T * C,
        "k3_bwd": 2 * bf * T * nC + 2 * f4 * T * n + bf * T * C,
        "k4_fwd": 2 * bf * T * nC + bf * T * C + f4 * T * n * n + f4 * T * n,
        "k4_bwd": 3 * bf * T * nC + 2 * bf * T * C + 2 * f4 * T * n * n + 2 * f4 * T * n,
    }


def make_inputs(T: int, C: int, seed: int = 0):
    """Synthetic inputs of the kernel-microbench config, generated on the GPU."""
    n, D = 4, 32
    nC = n * C
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(seed)

    def rn(*shape, scale=1.0, dtype=torch.bfloat16):
        return (torch.randn(*shape, generator=g, device=dev) * scale).to(dtype)

    x = rn(T, n, C)
    # Projection weight (D, nC) ~ N(0, 0.02) with an RMSNorm weight 1 + N(0, 0.02)
    # folded in: rmsnorm(x) * g @ W^T == rmsnorm(x) @ (W * g)^T.
    W = (rn(D, nC, scale=0.02, dtype=torch.float32) * (1 + rn(nC, scale=0.02, dtype=torch.float32))).to(torch.bfloat16)
    lo = rn(T, C)
    logits = rn(T, D, dtype=torch.float32)
    h_pre = torch.sigmoid(logits[:, :n]).contiguous()
    h_post = (2 * torch.sigmoid(logits[:, n : 2 * n])).contiguous()
    perm = build_perm(n).to(dev)
    H_res = (torch.softmax(logits[:, 2 * n :], -1) @ perm).view(T, n, n)
    H = (H_res - h_post[:, :, None] * h_pre[:, None, :]).contiguous()
    go1 = rn(T, D)
    go3 = rn(T, C)
    go4 = rn(T, n, C)
    return dict(x=x, W=W, lo=lo, h_pre=h_pre, h_post=h_post, H=H, go1=go1, go3=go3, go4=go4)


def build_perm(n: int) -> torch.Tensor:
    from flash_mhc import build_permutation_matrices

    return build_permutation_matrices(n)[0]


def make_step(inp: dict, T: int, C: int):
    """Closures launching each kernel once, with preallocated outputs."""
    from flash_mhc import kernels as K

    n = 4
    x, W = inp["x"], inp["W"]
    xf = x.view(T, n * C)
    proj, inv = K.k1_fwd(xf, W)
    bufs = dict(
        gx1=torch.empty_like(xf),
        out3=torch.empty((T, C), dtype=torch.bfloat16, device=x.device),
        gx3=torch.empty_like(x),
        gh3=torch.empty((T, n), dtype=torch.float32, device=x.device),
        out4=torch.empty_like(x),
        gx4=torch.empty_like(x),
        glo4=torch.empty((T, C), dtype=torch.bfloat16, device=x.device),
        gH4=torch.empty((T, n, n), dtype=torch.float32, device=x.device),
        ghp4=torch.empty((T, n), dtype=torch.float32, device=x.device),
    )
    proj2, inv2 = torch.empty_like(proj), torch.empty_like(inv)
    return {
        "k1_fwd": lambda: K.k1_fwd(xf, W, proj2, inv2),
        "k1_bwd_dx": lambda: K.k1_bwd_dx(inp["go1"], xf, W, proj, inv, bufs["gx1"]),
        "k3_fwd": lambda: K.k3_fwd(x, inp["h_pre"], bufs["out3"]),
        "k3_bwd": lambda: K.k3_bwd(inp["go3"], x, inp["h_pre"], bufs["gx3"], bufs["gh3"]),
        "k4_fwd": lambda: K.k4_fwd(x, inp["lo"], inp["H"], inp["h_post"], bufs["out4"]),
        "k4_bwd": lambda: K.k4_bwd(inp["go4"], x, inp["lo"], inp["H"], inp["h_post"],
                                   bufs["gx4"], bufs["glo4"], bufs["gH4"], bufs["ghp4"]),
    }


def k1_backward_paths(inp: dict, T: int, C: int, iters: int = 20) -> dict:
    """K1's full backward (grad_x and grad_W): the fused kernel vs the
    reference's two-step rule (bwd_dx kernel + torch.matmul for grad_W,
    ops.py:680-684).  Algorithmic bytes: bwd_dx's plus the bf16 grad_W write."""
    from flash_mhc import kernels as K

    n, D = 4, 32
    nC = n * C
    x, W, go = inp["x"].view(T, nC), inp["W"], inp["go1"]
    proj, inv = K.k1_fwd(x, W)
    gx = torch.empty_like(x)
    gW = torch.empty((D, nC), dtype=torch.bfloat16, device=x.device)

    def fused():
        K.k1_bwd(go, x, W, proj, inv, gx, gW)

    def two_step():
        K.k1_bwd_dx(go, x, W, proj, inv, gx)
        torch.matmul((go * inv[:, None]).to(x.dtype).t().contiguous(), x)

    out = {}
    nbytes = bytes_model(T, n, C, D)["k1_bwd_dx"] + 2 * D * nC
    for name, fn in (("fused", fused), ("two_step", two_step)):
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / iters * 1e3
        out[name] = {"avg_us": round(us, 2), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
    out["bytes"] = nbytes
    return out


def isolated_kernels(launch: dict, bm: dict, iters: int = 20, warmup: int = 5) -> dict:
    """Each kernel alone: ``iters`` back-to-back launches of the same kernel
    between two events.  The reference's microbenchmark times one launch per
    event pair with a synchronize after each (scripts/benchmark_kernels.py:43-57);
    here that pair also spans the host's launch of the kernel after an idle
    GPU (K1 bwd-dx: 199 us that way, 167 us in the step), so repeats are timed
    as a batch.  In the six-kernel step each kernel instead starts while the
    memory-side cache still holds the previous kernel's dirty lines."""
    out = {}
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for name in KERNELS:
        for _ in range(warmup):
            launch[name]()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(iters):
            launch[name]()
        e1.record()
        torch.cuda.synchronize()
        avg = e0.elapsed_time(e1) / iters
        out[name] = {"avg_us": round(avg * 1e3, 2), "GBps": round(bm[name] / (avg * 1e-3) / 1e9, 1),
                     "frac": round(bm[name] / (avg * 1e-3) / 1e9 / PEAK_GBPS, 4)}
    return out


def block_step(T: int, C: int, iters: int = 10, variants=("fused", "reference_rules")) -> dict:
    """MHCLiteBlock(4, C, Linear(C, C)) forward + backward (bf16, random
    weights) with the fused path as shipped, and with the reference's rules
    (K2 as PyTorch ops, K1's grad_W as a matmul, separate pre-map ops)."""
    import flash_mhc

    torch.manual_seed(0)
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False)).cuda().bfloat16()
    x = torch.randn(T, 4, C, device="cuda", dtype=torch.bfloat16).requires_grad_(True)
    up = torch.randn(T, 4, C, device="cuda", dtype=torch.bfloat16)
    flags = ("FLASH_MHC_FUSED_K2", "FLASH_MHC_FUSED_DW", "FLASH_MHC_FUSED_PREMAP")
    saved = {f: os.environ.get(f) for f in flags}
    out = {}
    try:
        for name, val in (("fused", "1"), ("reference_rules", "0")):
            if name not in variants:
                continue
            for f in flags:
                os.environ[f] = val

            def one():
                blk.zero_grad(set_to_none=True)
                x.grad = None
                blk(x).backward(up)

            for _ in range(3):
                one()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(iters):
                one()
            e1.record()
            torch.cuda.synchronize()
            out[name + "_ms"] = round(e0.elapsed_time(e1) / iters, 3)
    finally:
        for f, v in saved.items():
            if v is None:
                os.environ.pop(f, None)
            else:
                os.environ[f] = v
    out["workload"] = f"MHCLiteBlock(4, {C}, Linear({C}, {C})) forward + backward, T={T}, bf16"
    return out


def placement_sweep(T: int, C: int, pads: tuple[int, ...], iters: int = 10) -> dict:
    """K3 and K4 forward and backward at (T, C) with their tensors placed back
    to back in one allocation, `pad` bytes apart (each start rounded up to
    4 KiB first), for each pad: the kernels' GB/s (algorithmic bytes of
    bytes_model over the event time of `iters` back-to-back launches, after
    one untimed launch).  Shows how much the HBM rate depends on where the
    tensors lie relative to each other."""
    from flash_mhc import kernels as K

    n = 4
    bf, f4 = torch.bfloat16, torch.float32
    specs = [("go", (T, n, C), bf), ("x", (T, n, C), bf), ("lo", (T, C), bf), ("gx", (T, n, C), bf),
             ("glo", (T, C), bf), ("H", (T, n, n), f4), ("hp", (T, n), f4), ("hq", (T, n), f4),
             ("gH", (T, n, n), f4), ("ghq", (T, n), f4), ("ghp", (T, n), f4)]
    bm = bytes_model(T, n, C, 32)
    out = {}
    for pad in pads:
        sizes = [math.prod(shape) * torch.empty((), dtype=dt).element_size() for _, shape, dt in specs]
        offs, o = [], 0
        for nb in sizes:
            offs.append(o)
            o += (nb + 4095) // 4096 * 4096 + pad
        pool = torch.empty(o, dtype=torch.uint8, device="cuda")
        t = {name: pool[off:off + nb].view(dt).view(shape) for (name, shape, dt), off, nb in zip(specs, offs, sizes)}
        g = torch.Generator(device="cuda").manual_seed(0)
        for k in ("go", "x", "lo", "H"):
            t[k].normal_(generator=g)
        t["hp"].uniform_(0, 1, generator=g)
        t["hq"].uniform_(0, 2, generator=g)
        launch = {
            "k3_fwd": lambda: K.k3_fwd(t["x"], t["hp"], t["glo"]),
            "k3_bwd": lambda: K.k3_bwd(t["lo"], t["x"], t["hp"], t["gx"], t["ghp"]),
            "k4_fwd": lambda: K.k4_fwd(t["x"], t["lo"], t["H"], t["hq"], t["gx"]),
            "k4_bwd": lambda: K.k4_bwd(t["go"], t["x"], t["lo"], t["H"], t["hq"], t["gx"], t["glo"], t["gH"],
                                       t["ghq"]),
        }
        row = {}
        for name, fn in launch.items():
            fn()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(iters):
                fn()
            e1.record()
            torch.cuda.synchronize()
            row[name] = round(bm[name] / (e0.elapsed_time(e1) * 1e-3 / iters) / 1e9, 1)
        out[str(pad)] = row
        del pool, t, launch
        torch.cuda.empty_cache()
    return {"GBps_by_pad_bytes": out,
            "workload": f"K3/K4 fwd+bwd, T={T}, n=4, C={C}, bf16, tensors back to back in one allocation "
                        f"with pad bytes between them, {iters} launches per kernel"}


def train_stack(T: int, C: int, layers: int = 12, iters: int = 3, warmup: int = 1, compiled: bool = True) -> dict:
    """layers x MHCLiteBlock(4, C, Linear(C, C, bias=False)) forward + backward
    (bf16, random weights, activation checkpointing on), eager or under
    torch.compile (the first warmup step compiles): milliseconds per step and
    the peak HBM allocated."""
    import flash_mhc

    torch.manual_seed(0)
    blocks = torch.nn.Sequential(*[
        flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False), activation_checkpointing=True)
        for _ in range(layers)
    ]).to("cuda", torch.bfloat16)
    g = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(T, 4, C, device="cuda", generator=g).to(torch.bfloat16).requires_grad_(True)
    up = torch.randn(T, 4, C, device="cuda", generator=g).to(torch.bfloat16)
    run = torch.compile(blocks) if compiled else blocks

    def one():
        for p in blocks.parameters():
            p.grad = None
        x.grad = None
        run(x).backward(up)

    for _ in range(max(1, warmup)):
        one()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        one()
    e1.record()
    torch.cuda.synchronize()
    return {"ms_per_step": round(e0.elapsed_time(e1) / iters, 2),
            "peak_GB": round(torch.cuda.max_memory_allocated() / 1e9, 1),
            "workload": (f"{layers} x MHCLiteBlock(4, {C}, Linear({C}, {C}, bias=False)), activation checkpointing, "
                         f"forward + backward, T={T}, bf16, {'torch.compile' if compiled else 'eager'}")}


def block_step_graphed(T: int = 4096, C: int = 1024, iters: int = 20) -> dict:
    """MHCLiteBlock(4, C, Linear(C, C)) forward + backward at few tokens, where
    the host's launches bound an eager step: eager, and the whole step (forward
    and backward) captured once in a HIP graph and replayed."""
    import flash_mhc

    torch.manual_seed(0)
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False)).cuda().bfloat16()
    x = torch.randn(T, 4, C, device="cuda", dtype=torch.bfloat16).requires_grad_(True)
    up = torch.randn(T, 4, C, device="cuda", dtype=torch.bfloat16)

    def step():
        blk.zero_grad(set_to_none=True)
        x.grad = None
        blk(x).backward(up)

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return round(e0.elapsed_time(e1) / iters, 4)

    out = {"eager_ms": timed(step)}
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    blk.zero_grad(set_to_none=True)
    x.grad = None
    with torch.cuda.graph(g, stream=s):  # the warm-up's stream (autograd's AccumulateGrad streams)
        blk(x).backward(up)
    out["graph_ms"] = timed(g.replay)
    out["workload"] = f"MHCLiteBlock(4, {C}, Linear({C}, {C})) forward + backward, T={T}, bf16"
    return out


def premap_alone(T: int, C: int, iters: int = 10) -> dict:
    """The block's pre-map forward (K1 + K2 + K3, the launch of
    flash_mhc::mhc_pre_map) alone at (T, C), each launch after a cache flush,
    for profiler runs that compare builds.  Beside it, two references for the
    latency of reads past L2: an ordinary 128 MiB read repeated (served by
    the 256 MB memory-side cache after its first pass) and an ordinary 1 GiB
    read (HBM)."""
    from flash_mhc import build_permutation_matrices
    from flash_mhc import kernels as K

    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(T, 4, C, device="cuda", generator=g).to(torch.bfloat16)
    W = (torch.randn(32, 4 * C, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    p = [torch.tensor([0.8], device="cuda"), torch.tensor([1.2], device="cuda"), torch.tensor([1.7], device="cuda"),
         torch.randn(32, device="cuda", generator=g) * 0.5, build_permutation_matrices(4)[0].cuda()]
    probe = Probe()
    flush = CacheFlush(probe)
    times = []
    for _ in range(iters):
        flush()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        K.premap_fwd(x, W, *p)
        e1.record()
        times.append((e0, e1))
    torch.cuda.synchronize()
    small = torch.ones(128 << 20, dtype=torch.uint8, device="cuda")
    big = torch.ones(1 << 30, dtype=torch.uint8, device="cuda")
    sink = torch.empty(4096, dtype=torch.uint8, device="cuda")
    for _ in range(4):
        probe.run(PROBE_READ_CACHED, small, sink, small.numel())
    probe.run(PROBE_READ_CACHED, big, sink, big.numel())
    torch.cuda.synchronize()
    ts = [a.elapsed_time(b) * 1e3 for a, b in times]
    return {"premap_fwd_cold_us": round(statistics.median(ts), 1), "min_us": round(min(ts), 1),
            "workload": f"pre-map forward, T={T}, n=4, C={C}, bf16, each launch after a cache flush"}


def premap_bwd_alone(T: int, C: int, iters: int = 10) -> dict:
    """The block's pre-map backward (flash_mhc::mhc_pre_map_coeffs's backward:
    K3's grad_h_pre, K2's backward, K1's backward with grad_W, and x's
    incoming gradient added in grad_x's store) alone at (T, C), each launch
    after a cache flush, for profiler runs that compare builds.  Algorithmic
    bytes: x, the incoming gradient, grad_layer_input, proj, inv_rms, h_pre,
    grad_h_post, grad_H_merged and W read once, grad_x and grad_W written
    once."""
    from flash_mhc import build_permutation_matrices
    from flash_mhc import kernels as K

    g = torch.Generator(device="cuda").manual_seed(0)
    nC = 4 * C
    x = torch.randn(T, 4, C, device="cuda", generator=g).to(torch.bfloat16)
    W = (torch.randn(32, nC, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    p = [torch.tensor([0.8], device="cuda"), torch.tensor([1.2], device="cuda"), torch.tensor([1.7], device="cuda"),
         torch.randn(32, device="cuda", generator=g) * 0.5, build_permutation_matrices(4)[0].cuda()]
    _, _, _, hp, proj, inv = K.premap_fwd(x, W, *p)
    g_li = torch.randn(T, C, device="cuda", generator=g).to(torch.bfloat16)
    g_hq = torch.randn(T, 4, device="cuda", generator=g)
    g_H = torch.randn(T, 4, 4, device="cuda", generator=g)
    g_in = torch.randn(T, 4, C, device="cuda", generator=g).to(torch.bfloat16)
    flush = CacheFlush(Probe())
    times = []
    for _ in range(iters):
        flush()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        K.premap_bwd(x, W, *p, hp, proj, inv, g_li, g_hq, g_H, g_in)
        e1.record()
        times.append((e0, e1))
    torch.cuda.synchronize()
    nbytes = (3 * T * nC * 2 + T * C * 2 + T * 32 * 2 + T * 4 + T * 4 * 4 * 2 + T * 16 * 4
              + 2 * 32 * nC * 2)
    ts = [a.elapsed_time(b) * 1e3 for a, b in times]
    med = statistics.median(ts)
    return {"premap_bwd_cold_us": round(med, 1), "min_us": round(min(ts), 1), "bytes": nbytes,
            "GBps": round(nbytes / (med * 1e-6) / 1e9, 1),
            "workload": f"pre-map backward with x's incoming gradient, T={T}, n=4, C={C}, bf16, "
                        "each launch after a cache flush"}


def eval_latency(C: int = 4096, tokens=(1, 64, 257, 65537), variants=("fused", "reference_rules")) -> dict:
    """Eval-mode forward latency of MHCLiteBlock(4, C, Linear(C, C)) (bf16,
    random weights), the inference / ragged-tail shapes: eager and replayed from
    a captured HIP graph, for the fused path and for the reference's rules
    (K2 as PyTorch ops, separate pre-map ops; graph replay)."""
    import flash_mhc

    torch.manual_seed(0)
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False)).cuda().bfloat16().eval()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn, n, batches=5):
        # Median over batches of n back-to-back calls: one slow batch (host
        # or clock hiccup) does not move a latency of a few tens of us.
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        per = []
        for _ in range(batches):
            e0.record()
            for _ in range(n):
                fn()
            e1.record()
            torch.cuda.synchronize()
            per.append(e0.elapsed_time(e1) / n)
        return round(statistics.median(per) * 1e3, 1)

    def graphed(x):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                blk(x)
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            blk(x)
        return g

    flags = ("FLASH_MHC_FUSED_K2", "FLASH_MHC_FUSED_PREMAP")
    saved = {f: os.environ.get(f) for f in flags}
    out = {}
    try:
        with torch.no_grad():
            for T in tokens:
                n = 20 if T < 4096 else 4
                x = torch.randn(T, 4, C, device="cuda", dtype=torch.bfloat16)
                row = {}
                for name, val in (("fused", "1"), ("reference_rules", "0")):
                    if name not in variants:
                        continue
                    for f in flags:
                        os.environ[f] = val
                    if name == "fused":
                        row["eager_us"] = timed(lambda: blk(x), n)
                    g = graphed(x)
                    row[("graph_us" if name == "fused" else "reference_rules_graph_us")] = timed(g.replay, n)
                    del g
                out[f"T={T}"] = row
    finally:
        for f, v in saved.items():
            if v is None:
                os.environ.pop(f, None)
            else:
                os.environ[f] = v
    out["workload"] = f"MHCLiteBlock(4, {C}, Linear({C}, {C})) eval forward, bf16"
    return out


def read_write_split(T: int, n: int, C: int, D: int) -> dict[str, tuple[int, int]]:
    """(bytes read, bytes written) per launch; sums to bytes_model."""
    bf, f4 = 2, 4
    nC = n * C
    return {
        "k1_fwd": (bf * T * nC + bf * D * nC, bf * T * D + f4 * T),
        "k1_bwd_dx": (bf * T * nC + bf * D * nC + 2 * bf * T * D + f4 * T, bf * T * nC),
        "k3_fwd": (bf * T * nC + f4 * T * n, bf * T * C),
        "k3_bwd": (bf * T * nC + f4 * T * n + bf * T * C, bf * T * nC + f4 * T * n),
        "k4_fwd": (bf * T * nC + bf * T * C + f4 * T * n * n + f4 * T * n, bf * T * nC),
        "k4_bwd": (2 * bf * T * nC + bf * T * C + f4 * T * n * n + f4 * T * n,
                   bf * T * nC + bf * T * C + f4 * T * n * n + f4 * T * n),
    }


PROBE_READ, PROBE_WRITE, PROBE_COPY, PROBE_READ_CACHED, PROBE_WRITE_CACHED = 0, 1, 2, 3, 4


class Probe:
    """The bandwidth probe and cache flush (include/flash_mhc_probe.h), a
    library of its own that only this benchmark loads."""

    def __init__(self):
        import ctypes

        from flash_mhc import _abi, build

        path = build.PROBE_LIB_PATH
        if not path.exists():
            raise _abi.ExtensionMissingError(f"probe library not found at {path}; run flash_mhc.build")
        self.lib = ctypes.CDLL(str(path))
        self.lib.fmhc_stream_probe.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                               ctypes.c_void_p]
        if self.lib.fmhc_probe_abi_version() != 2:
            raise _abi.ExtensionMissingError(f"{path} is stale; rebuild it")
        self._check = _abi.check

    def run(self, kind: int, src, dst, nbytes: int) -> None:
        st = torch.cuda.current_stream().cuda_stream
        s = self.lib.fmhc_stream_probe(kind, None if src is None else src.data_ptr(), dst.data_ptr(), nbytes, st)
        self._check(s, "stream_probe")


class CacheFlush:
    """Evicts L2 and the 256 MB memory-side cache: a 512 MiB write (ordinary
    stores) and then a 1 GiB read (ordinary loads) of scratch buffers, so the
    caches hold neither the next kernel's inputs nor dirty lines it would
    have to write back."""

    def __init__(self, probe: Probe, write_bytes: int = 512 << 20, read_bytes: int = 1 << 30):
        self.probe = probe
        self.w = torch.empty(write_bytes, dtype=torch.uint8, device="cuda")
        self.r = torch.empty(read_bytes, dtype=torch.uint8, device="cuda").fill_(1)

    def __call__(self) -> None:
        self.probe.run(PROBE_WRITE_CACHED, None, self.w, self.w.numel())
        self.probe.run(PROBE_READ_CACHED, self.r, self.w, self.r.numel())


def cold_step(step, nbytes: int, flush: CacheFlush, reps: int = 10) -> dict:
    """The six-kernel step with cold caches: before every step the caches are
    flushed (CacheFlush), then the step's six launches between two events."""
    step()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    torch.cuda.synchronize()
    for e0, e1 in evs:
        flush()
        e0.record()
        step()
        e1.record()
    torch.cuda.synchronize()
    ts = [e0.elapsed_time(e1) for e0, e1 in evs]
    med = statistics.median(ts)
    return {"median_ms": round(med, 4), "min_ms": round(min(ts), 4),
            "GBps": round(nbytes / (med * 1e-3) / 1e9, 1), "frac": round(nbytes / (med * 1e-3) / 1e9 / PEAK_GBPS, 4)}


def cold_kernels(launch: dict, bm: dict, flush: CacheFlush, reps: int = 10) -> dict:
    """Each kernel with cold caches: before every launch the caches are flushed
    (CacheFlush), then one launch between two events (the flush is queued
    ahead of the first event, so the pair spans the kernel alone)."""
    out = {}
    for name in KERNELS:
        launch[name]()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        torch.cuda.synchronize()
        for e0, e1 in evs:
            flush()
            e0.record()
            launch[name]()
            e1.record()
        torch.cuda.synchronize()
        ts = [e0.elapsed_time(e1) for e0, e1 in evs]
        med = statistics.median(ts)
        out[name] = {"median_us": round(med * 1e3, 2), "min_us": round(min(ts) * 1e3, 2),
                     "GBps": round(bm[name] / (med * 1e-3) / 1e9, 1),
                     "frac": round(bm[name] / (med * 1e-3) / 1e9 / PEAK_GBPS, 4)}
    return out


def stream_ceilings(probe: Probe, nbytes: int = 1 << 30, iters: int = 10) -> dict[str, float]:
    """Measured HBM GB/s of 16-byte streaming read / write / copy with the
    nontemporal hint (the kernels' streaming loads and stores carry it), and
    ordinary-load / ordinary-store read and write as labelled extras."""
    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    out = {}
    for name, kind, moved in (("read", PROBE_READ, nbytes), ("write", PROBE_WRITE, nbytes),
                              ("copy", PROBE_COPY, 2 * nbytes), ("read_ordinary", PROBE_READ_CACHED, nbytes),
                              ("write_ordinary", PROBE_WRITE_CACHED, nbytes)):
        run = lambda: probe.run(kind, a, b, nbytes)  # noqa: E731
        for _ in range(3):
            run()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            run()
        e1.record()
        torch.cuda.synchronize()
        out[name] = round(moved / (e0.elapsed_time(e1) / iters * 1e-3) / 1e9, 1)
    del a, b
    return out


def cpu_model() -> str:
    try:
        return next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except (OSError, StopIteration):
        return "unknown"


def cpu_block_config1(T: int = 4096, C: int = 1024, iters: int = 5) -> dict:
    """The golden configuration on the host: MHCLiteBlock(4, C, bias-free
    Linear(C, C)) in fp32 on the CPU, which takes the block's plain PyTorch
    path (the reference's fallback, block.py:82-148), x (T, 4, C) ~ N(0, 1)
    from seed 0, forward + backward of sum(out); median wall time of `iters`
    after one warm-up, on all host cores."""
    import flash_mhc

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    torch.manual_seed(0)
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False))
    x = torch.randn(T, 4, C, generator=torch.Generator().manual_seed(0)).requires_grad_(True)

    def one():
        blk.zero_grad(set_to_none=True)
        x.grad = None
        blk(x).sum().backward()

    one()
    ts = []
    for _ in range(iters):
        t0 = time.perf_counter()
        one()
        ts.append(time.perf_counter() - t0)
    med = statistics.median(ts)
    return {"workload": f"MHCLiteBlock(4, {C}, Linear({C}, {C})) fp32 plain path, T={T}, forward + backward "
                        f"of sum(out), x ~ N(0,1) seed 0", "median_ms": round(med * 1e3, 2),
            "min_ms": round(min(ts) * 1e3, 2), "tokens_per_s": round(T / med, 1), "cores": cores,
            "cpu": cpu_model(), "iters": iters}


def cpu_baseline(C: int, tokens: int, iters: int = 3) -> dict:
    """The reference's PyTorch formulation of the six ops, fp32 autograd on the host."""
    from oracle import mhc_oracle as O

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    n, D, T = 4, 32, tokens
    nC = n * C
    g = torch.Generator().manual_seed(0)
    x = torch.randn(T, n, C, generator=g)
    W = torch.randn(D, nC, generator=g) * 0.02
    lo = torch.randn(T, C, generator=g)
    hpre = torch.rand(T, n, generator=g)
    hp = torch.rand(T, n, generator=g) * 2
    H = torch.randn(T, n, n, generator=g) * 0.3
    go1, go3, go4 = torch.randn(T, D, generator=g), torch.randn(T, C, generator=g), torch.randn(T, n, C, generator=g)

    def leaf(t):
        return t.clone().requires_grad_(True)

    def k1():
        xf, w = leaf(x.view(T, nC)), leaf(W)
        O.k1_torch(xf, w).backward(go1)

    def k3():
        xs, h = leaf(x), leaf(hpre)
        O.k3_torch(xs, h).backward(go3)

    def k4():
        xs, l, Hm, h = leaf(x), leaf(lo), leaf(H), leaf(hp)
        O.k4_torch(xs, l, Hm, h).backward(go4)

    total = 0.0
    per = {}
    for name, fn in (("k1", k1), ("k3", k3), ("k4", k4)):
        fn()
        ts = []
        for _ in range(iters):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        per[name] = statistics.median(ts)
        total += per[name]
    bm = bytes_model(T, n, C, D)
    nbytes = sum(bm.values())
    return {
        "value": round(nbytes / total / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"T={T} tokens of the same n=4, C={C} workload, fp32 on the host CPU ({cpu_model()}); "
                   f"K1/K3/K4 forward+autograd backward with the reference's PyTorch formulas; "
                   f"median of {iters} after 1 warmup; bytes from the same model as the GPU kernels"),
        "tokens_per_s": round(T / total, 1),
        "seconds_per_pass": {k: round(v, 4) for k, v in per.items()},
    }


def main() -> None:
    global PEAK_GBPS  # --peak-gbps
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", "--iters", dest="steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--T", type=int, default=65536)
    ap.add_argument("--C", type=int, default=1024)
    # The reference benchmark's flags (scripts/benchmark_kernels.py:145-151), so
    # its documented command line runs here too; --iters is --steps.
    ap.add_argument("--n", type=int, default=4, help="streams; the kernels are built for n = 4 only")
    ap.add_argument("--seed", type=int, default=0, help="seed of the synthetic inputs")
    ap.add_argument("--peak-gbps", type=float, default=PEAK_GBPS,
                    help="HBM peak the fractions are quoted against (default: MI355X, 8000 GB/s)")
    ap.add_argument("--cpu-tokens", type=int, default=65536,
                    help="tokens of the CPU baseline's sample (default: the whole metric workload)")
    ap.add_argument("--cpu-iters", type=int, default=10, help="timed passes of the CPU baseline (median)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--columns", action="store_true",
                    help="with --no-extras: still time each kernel alone and cold")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the K1-backward and block-step fields (profiler runs: only the six kernels)")
    ap.add_argument("--traffic", type=str, default=str(ROOT / "profiles" / "traffic_k4_bwd_T65536_C1024.json"),
                    help="measured HBM traffic summary (rocprofv3 --pmc) for the dominant kernel")
    ap.add_argument("--only", choices=("block", "eval", "premap", "premap_bwd", "train", "placement"), default=None,
                    help="run one extra alone, fused path only, and print its JSON (profiler runs of the "
                         "block step at --T/--C for --steps iterations, or of the eval latency at --eval-T)")
    ap.add_argument("--layers", type=int, default=12, help="blocks of the --only train stack")
    ap.add_argument("--eager", action="store_true", help="--only train without torch.compile")
    ap.add_argument("--pads", type=str, default="0,4096,65536,262144,1048576,2097152,3149824",
                    help="--only placement: bytes between consecutive tensors")
    ap.add_argument("--eval-T", type=str, default="1,64,257,65537", help="token counts of the eval latency")
    args = ap.parse_args()
    if args.n != 4:
        print("bench.py: the K1/K3/K4 kernels support n = 4 only (the reference's fused ops raise "
              "ValueError for other n)", file=sys.stderr)
        sys.exit(2)
    if not args.peak_gbps > 0:
        print("bench.py: --peak-gbps must be positive", file=sys.stderr)
        sys.exit(2)
    PEAK_GBPS = args.peak_gbps

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the K1/K3/K4 path is independent per token, "
              "so N GPUs would each run this same per-GPU workload on T/N tokens with no "
              "communication; run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)

    from flash_mhc import _abi

    _abi.load()  # fail loudly if the extension is missing
    eval_tokens = tuple(int(t) for t in args.eval_T.split(","))
    if args.only == "block":
        print(json.dumps({"block_step": block_step(args.T, args.C, iters=args.steps, variants=("fused",))}),
              flush=True)
        return
    if args.only == "premap":
        print(json.dumps({"premap_alone": premap_alone(args.T, args.C, iters=args.steps)}), flush=True)
        return
    if args.only == "premap_bwd":
        print(json.dumps({"premap_bwd_alone": premap_bwd_alone(args.T, args.C, iters=args.steps)}), flush=True)
        return
    if args.only == "train":
        print(json.dumps({"train_stack": train_stack(args.T, args.C, layers=args.layers, iters=args.steps,
                                                     warmup=args.warmup, compiled=not args.eager)}), flush=True)
        return
    if args.only == "placement":
        pads = tuple(int(p) for p in args.pads.split(","))
        print(json.dumps({"placement": placement_sweep(args.T, args.C, pads, iters=args.steps)}), flush=True)
        return
    if args.only == "eval":
        print(json.dumps({"eval_latency": eval_latency(tokens=eval_tokens, variants=("fused",))}), flush=True)
        return
    T, C, n, D = args.T, args.C, 4, 32
    inp = make_inputs(T, C, seed=args.seed)
    launch = make_step(inp, T, C)
    bm = bytes_model(T, n, C, D)

    def step(events=None):
        for i, k in enumerate(KERNELS):
            if events is not None:
                events[i][0].record()
            launch[k]()
            if events is not None:
                events[i][1].record()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Timed region: exactly K steps, nothing but the six launches per step.
    K_steps = args.steps
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    s0 = torch.cuda.Event(enable_timing=True)
    s1 = torch.cuda.Event(enable_timing=True)
    s0.record()
    for k in range(K_steps):
        step()
    s1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    ms_total = s0.elapsed_time(s1)
    ms_per_step = ms_total / K_steps

    # Per-kernel durations: a second pass of K steps with an event pair around
    # each launch on the launch stream (events between launches would add
    # their own gaps to the step above).
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in KERNELS]
           for _ in range(K_steps)]
    for k in range(K_steps):
        step(evs[k])
    torch.cuda.synchronize()

    per = {}
    for i, name in enumerate(KERNELS):
        ts = [evs[k][i][0].elapsed_time(evs[k][i][1]) for k in range(K_steps)]
        avg = sum(ts) / len(ts)
        per[name] = {
            "avg_us": round(avg * 1e3, 2),
            "median_us": round(statistics.median(ts) * 1e3, 2),
            "GBps": round(bm[name] / (avg * 1e-3) / 1e9, 1),
            "frac": round(bm[name] / (avg * 1e-3) / 1e9 / PEAK_GBPS, 4),
            "bytes": bm[name],
        }
    total_bytes = sum(bm.values())
    value = total_bytes / (ms_per_step * 1e-3) / 1e9
    sum_kernel_ms = sum(p["avg_us"] for p in per.values()) / 1e3
    dom = max(per, key=lambda k: per[k]["avg_us"])

    traffic = None
    tpath = Path(args.traffic)
    if tpath.exists():
        try:
            tr = json.loads(tpath.read_text())
            if tr.get("kernel") == dom and tr.get("T") == T and tr.get("C") == C:
                traffic = tr.get("traffic_bytes")
        except (OSError, ValueError):
            traffic = None

    def extra(fn, *a, **kw):
        # An extra that raises is reported in its field; the kernel step,
        # which is the metric, is measured either way.
        if args.no_extras:
            return None
        try:
            return fn(*a, **kw)
        except Exception as e:  # noqa: BLE001
            torch.cuda.synchronize()
            return {"error": f"{type(e).__name__}: {e}"[:300]}

    # The latency-bound eval shapes first: after the block steps' seconds of
    # full-bandwidth work the same graph replays measure up to 25% slower.
    lat = extra(eval_latency, tokens=eval_tokens)
    columns = args.columns or not args.no_extras
    alone = isolated_kernels(launch, bm) if columns else None
    probe = Probe()
    flush = CacheFlush(probe) if columns else None
    cold = cold_kernels(launch, bm, flush) if columns else None
    step_cold = cold_step(step, total_bytes, flush) if columns else None
    k1_full_bwd = extra(k1_backward_paths, inp, T, C)
    blk = extra(block_step, T, C)
    # The block configuration at C = 2048 (same T), with its own layer width.
    blk2 = extra(block_step, T, 2 * C)
    blk_small = extra(block_step_graphed)
    ceil = stream_ceilings(probe)
    split = read_write_split(T, n, C, D)
    for name in KERNELS:
        rd, wr = split[name]
        mix = (rd + wr) / (rd / ceil["read"] + wr / ceil["write"])
        per[name]["mix_ceiling_GBps"] = round(mix, 1)
        per[name]["frac_of_mix_ceiling"] = round(per[name]["GBps"] / mix, 4)
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K_steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": (f"mHC-lite K1/K3/K4 forward+backward kernel microbench: six HIP kernels per step, "
                         f"T={T}, n=4, C={C}, D_out=32, bf16 activations, fp32 coefficients"),
            "T": T, "n": n, "C": C, "D_out": D,
        },
        "frac_of_peak": round(value / PEAK_GBPS, 4),
        "tokens_per_s": round(T / (ms_per_step * 1e-3), 1),
        "sum_kernel_ms": round(sum_kernel_ms, 4),
        "ceilings_GBps": ceil,
        "k1_backward_with_grad_W": k1_full_bwd,
        "block_step": blk,
        "block_step_2C": blk2,
        "block_step_T4096": blk_small,
        "eval_latency": lat,
        "kernels": per,
        "kernels_isolated": alone,
        "kernels_cold": cold,
        "step_cold": step_cold,
        "roofline": {
            "kernel": dom,
            "bound": "hbm",
            "achieved": per[dom]["GBps"],
            "peak": PEAK_GBPS,
            "unit": "GB/s",
            "frac": per[dom]["frac"],
            "traffic": traffic,
        },
        "wall_s": round(wall, 3),
    }
    del inp, launch
    torch.cuda.empty_cache()
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(C, args.cpu_tokens, args.cpu_iters)
        line["cpu_block_config1"] = cpu_block_config1()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
