"""Training-scale stack on the GPU: 12 MHCLiteBlocks wrapping bias-free
Linear(4096, 4096), T = 262144 tokens (batch 64 x sequence 4096), n = 4,
C = 4096, bf16, activation checkpointing on, under torch.compile (inductor).

Checks that the fused path runs at this size (x alone is 8.6 GB per block
input), that every parameter receives a finite gradient, that the compiled
stack's forward and gradients (x's and every parameter's) equal the eager
stack's on the same weights -- bit for bit, or, where torch.compile orders
the autograd graph's own additions differently, within the reference's
gradient tolerance (tests/test_correctness.py:296 of the reference: 5e-2
relative, 1e-1 of each row's RMS) -- and reports the forward + backward time
per step and the peak HBM allocated, beside the same stack eager and under
the reference's rules, eager and compiled.
"""

from __future__ import annotations

import os
import time

import pytest
import torch

import flash_mhc

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16 = torch.bfloat16


def _grad_agrees(name: str, a: torch.Tensor, b: torch.Tensor, rtol: float = 5e-2, atol: float = 1e-1) -> bool:
    """True when a equals b bit for bit; otherwise asserts
    |a - b| <= rtol |b| + atol rms_row(b) elementwise (rows: dim 0), on the
    GPU in chunks of rows (x's gradient alone is 4.3 G elements), and returns
    False."""
    assert a.shape == b.shape, name
    if torch.equal(a, b):
        return True
    rows = a.shape[0]
    step = max(1, (1 << 26) // max(1, a[0].numel()))
    for r0 in range(0, rows, step):
        ra = a[r0:r0 + step].float().reshape(min(step, rows - r0), -1)
        rb = b[r0:r0 + step].float().reshape(min(step, rows - r0), -1)
        rms = rb.pow(2).mean(dim=1, keepdim=True).sqrt()
        bad = (ra - rb).abs() > rtol * rb.abs() + atol * rms
        assert not bool(bad.any()), f"{name}: {int(bad.sum())} elements beyond tolerance in rows {r0}.."
    return False


@pytest.mark.timeout(900)
def test_training_scale_stack():
    T, C, L = 262144, 4096, 12
    torch.manual_seed(0)
    blocks = torch.nn.Sequential(*[
        flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False), activation_checkpointing=True)
        for _ in range(L)
    ]).to(DEV, BF16)
    g = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn(T, 4, C, device=DEV, generator=g).to(BF16).requires_grad_(True)
    up = torch.randn(T, 4, C, device=DEV, generator=g).to(BF16)

    with torch.no_grad():
        eager_out = blocks(x)
    compiled = torch.compile(blocks)

    def step():
        for p in blocks.parameters():
            p.grad = None
        x.grad = None
        out = compiled(x)
        out.backward(up)
        return out

    t0 = time.perf_counter()
    out = step()  # compiles
    torch.cuda.synchronize()
    compile_s = time.perf_counter() - t0
    assert torch.equal(out.detach(), eager_out), "compiled forward differs from eager"
    del eager_out, out

    # The compiled step's gradients against the eager stack's on the same
    # weights and inputs.
    names = ["x"] + [n for n, _ in blocks.named_parameters()]
    compiled_grads = [x.grad.clone()] + [p.grad.clone() for p in blocks.parameters()]
    for p in blocks.parameters():
        p.grad = None
    x.grad = None
    blocks(x).backward(up)
    torch.cuda.synchronize()
    eager_grads = [x.grad] + [p.grad for p in blocks.parameters()]
    bitwise = [_grad_agrees(n, a, b) for n, a, b in zip(names, compiled_grads, eager_grads)]
    print(f"\n[train-scale] compiled vs eager gradients: {sum(bitwise)} of {len(bitwise)} bit for bit, "
          f"the rest within tolerance: {[n for n, ok in zip(names, bitwise) if not ok][:6]}", flush=True)
    del compiled_grads, eager_grads

    torch.cuda.reset_peak_memory_stats()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = 2
    e0.record()
    for _ in range(n):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / n
    peak_gb = torch.cuda.max_memory_allocated() / 1e9
    for name, p in blocks.named_parameters():
        assert p.grad is not None, name
        assert bool(torch.isfinite(p.grad).all()), name
    assert bool(torch.isfinite(x.grad).all())
    print(f"\n[train-scale] 12 x MHCLiteBlock(4, 4096, Linear(4096, 4096)), T=262144, bf16, "
          f"checkpointing, torch.compile: fwd+bwd {ms:.1f} ms/step, peak HBM allocated {peak_gb:.1f} GB, "
          f"first (compiling) step {compile_s:.1f} s", flush=True)

    # The fused stack eager, for comparison with the compiled one.
    def eager_step():
        for p in blocks.parameters():
            p.grad = None
        x.grad = None
        blocks(x).backward(up)

    eager_step()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    e0.record()
    for _ in range(n):
        eager_step()
    e1.record()
    torch.cuda.synchronize()
    print(f"[train-scale] same stack, fused, eager: fwd+bwd {e0.elapsed_time(e1) / n:.1f} ms/step, "
          f"peak HBM allocated {torch.cuda.max_memory_allocated() / 1e9:.1f} GB", flush=True)

    # The same stack with the reference's rules (K2 as PyTorch ops, K1's
    # grad_W as a matmul, separate pre-map ops), for comparison: eager, then
    # under torch.compile like the fused stack above (the switches are read
    # while tracing, so the compiled stack is traced again after a reset).
    flags = ("FLASH_MHC_FUSED_K2", "FLASH_MHC_FUSED_DW", "FLASH_MHC_FUSED_PREMAP")
    saved = {f: os.environ.get(f) for f in flags}
    try:
        for f in flags:
            os.environ[f] = "0"
        del compiled
        torch._dynamo.reset()

        def timed(run, label):
            def one():
                for p in blocks.parameters():
                    p.grad = None
                x.grad = None
                run(x).backward(up)

            t0 = time.perf_counter()
            one()
            torch.cuda.synchronize()
            first_s = time.perf_counter() - t0
            torch.cuda.reset_peak_memory_stats()
            e0.record()
            for _ in range(n):
                one()
            e1.record()
            torch.cuda.synchronize()
            print(f"[train-scale] same stack, reference rules, {label}: fwd+bwd {e0.elapsed_time(e1) / n:.1f} "
                  f"ms/step, peak HBM allocated {torch.cuda.max_memory_allocated() / 1e9:.1f} GB, first step "
                  f"{first_s:.1f} s", flush=True)

        timed(blocks, "eager")
        timed(torch.compile(blocks), "torch.compile")
        torch._dynamo.reset()
    finally:
        for f, v in saved.items():
            if v is None:
                os.environ.pop(f, None)
            else:
                os.environ[f] = v
