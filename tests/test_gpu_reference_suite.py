"""The reference's own correctness suite, restated for the HIP kernels: the same
shapes, comparisons and tolerances as tests/test_correctness.py of
alint77/flash-mHC (K1 / K3 / K4 forward and backward against PyTorch
formulations of the paper's precision rules, and MHCLiteBlock's fused path
against its plain PyTorch path).  The oracle-based tests elsewhere hold the
kernels to tighter, per-element bounds; this file shows they also pass the
reference's own bar.

Tolerances (tests/test_correctness.py:45-48): forward atol 1e-2, rtol 1.6e-2
(about 2 bf16 ulps); backward atol 5e-2, rtol 2e-2; end to end (:282, :294,
:316) forward atol 5e-2, rtol 2e-2, gradients atol 1e-1, rtol 5e-2; an
element passes when |a - b| <= atol + rtol |b| (torch.allclose).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import flash_mhc

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16 = torch.bfloat16
FWD = dict(atol=1e-2, rtol=1.6e-2)
BWD = dict(atol=5e-2, rtol=2e-2)
T_OPS, N, C_OPS = 2048, 4, 256


def close(name, got, want, atol, rtol):
    got = got.to(want.dtype).float()
    want = want.float()
    diff = (got - want).abs()
    ok = bool((diff <= atol + rtol * want.abs()).all())
    assert ok, f"{name}: max |diff| {float(diff.max()):.4e} (atol {atol}, rtol {rtol})"


def randn(*shape, dtype=BF16, grad=False, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    t = torch.randn(*shape, device=DEV, generator=g).to(dtype)
    return t.requires_grad_(grad)


def k1_paper(x_flat, W):
    """Matmul first (bf16 inputs, the GEMM's bf16 result), then the fp32 RMS
    factor, product in fp32, stored as bf16 (the paper's Eq. 5-7)."""
    raw = torch.matmul(x_flat, W.t().contiguous())
    inv = (x_flat.float() * x_flat.float()).mean(-1, keepdim=True).add(1e-6).rsqrt()
    return (raw.float() * inv).to(x_flat.dtype)


def k3_paper(x, h_pre):
    return (h_pre.unsqueeze(-1) * x.float()).sum(-2).to(x.dtype)


def k4_paper(x, lo, H, h_post):
    out = torch.matmul(H, x.float()) + h_post.unsqueeze(-1) * lo.float().unsqueeze(-2)
    return out.to(x.dtype)


def test_k1_forward():
    x = randn(T_OPS, N * C_OPS, seed=1)
    W = randn(32, N * C_OPS, seed=2)
    out, _ = torch.ops.flash_mhc.fused_rmsnorm_project(x, W)
    close("K1 forward", out, k1_paper(x, W), **FWD)


def test_k1_backward():
    x = randn(T_OPS, N * C_OPS, grad=True, seed=3)
    W = randn(32, N * C_OPS, grad=True, seed=4)
    xr = x.detach().clone().requires_grad_(True)
    Wr = W.detach().clone().requires_grad_(True)
    out, _ = torch.ops.flash_mhc.fused_rmsnorm_project(x, W)
    out.float().sum().backward()
    k1_paper(xr, Wr).float().sum().backward()
    close("K1 grad_x", x.grad, xr.grad, **BWD)
    close("K1 grad_W", W.grad, Wr.grad, **BWD)


def test_k3_forward_backward():
    x = randn(T_OPS, N, C_OPS, grad=True, seed=5)
    h = randn(T_OPS, N, dtype=torch.float32, grad=True, seed=6)
    xr = x.detach().clone().requires_grad_(True)
    hr = h.detach().clone().requires_grad_(True)
    out = torch.ops.flash_mhc.fused_pre_map(x, h)
    ref = k3_paper(xr, hr)
    close("K3 forward", out, ref, **FWD)
    out.float().sum().backward()
    ref.float().sum().backward()
    close("K3 grad_x", x.grad, xr.grad, **BWD)
    close("K3 grad_h_pre", h.grad, hr.grad, **BWD)


def test_k4_forward_backward():
    x = randn(T_OPS, N, C_OPS, grad=True, seed=7)
    lo = randn(T_OPS, C_OPS, grad=True, seed=8)
    H = randn(T_OPS, N, N, dtype=torch.float32, grad=True, seed=9)
    hp = randn(T_OPS, N, dtype=torch.float32, grad=True, seed=10)
    leaves = [t.detach().clone().requires_grad_(True) for t in (x, lo, H, hp)]
    out = torch.ops.flash_mhc.fused_post_res(x, lo, H, hp)
    ref = k4_paper(*leaves)
    close("K4 forward", out, ref, **FWD)
    out.float().sum().backward()
    ref.float().sum().backward()
    for name, got, want in (("grad_x", x, leaves[0]), ("grad_lo", lo, leaves[1]), ("grad_H", H, leaves[2]),
                            ("grad_h_post", hp, leaves[3])):
        close("K4 " + name, got.grad, want.grad, **BWD)


class _LinearGelu(torch.nn.Module):
    """The reference suite's stand-in layer: bias-free linear, then GELU."""

    def __init__(self, dim):
        super().__init__()
        self.proj = torch.nn.Linear(dim, dim, bias=False)

    def forward(self, x, **kwargs):
        return F.gelu(self.proj(x))


def _e2e_block():
    torch.manual_seed(0)
    C = 256
    return flash_mhc.MHCLiteBlock(n_streams=4, hidden_size=C, layer=_LinearGelu(C), triton_fused=True).to(DEV, BF16)


def test_block_fused_vs_plain_forward():
    blk = _e2e_block()
    x = randn(1024, 4, 256, seed=11)
    with torch.no_grad():
        close("block forward", blk._forward_triton(x.clone()), blk._forward_pytorch(x.clone()), atol=5e-2, rtol=2e-2)


def test_block_fused_vs_plain_backward_and_parameter_grads():
    blk = _e2e_block()
    x = randn(1024, 4, 256, seed=12)
    grads = {}
    for path in ("fused", "plain"):
        blk.zero_grad(set_to_none=True)
        xs = x.clone().requires_grad_(True)
        out = blk._forward_triton(xs) if path == "fused" else blk._forward_pytorch(xs)
        out.float().sum().backward()
        grads[path] = (xs.grad, {n: p.grad.clone() for n, p in blk.named_parameters() if p.grad is not None})
    close("block grad_x", grads["fused"][0], grads["plain"][0], atol=1e-1, rtol=5e-2)
    for name, ref in grads["plain"][1].items():
        assert name in grads["fused"][1], f"no fused-path gradient for {name}"
        close(f"block grad {name}", grads["fused"][1][name], ref, atol=1e-1, rtol=5e-2)
