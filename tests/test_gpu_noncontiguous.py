"""Strided (non-contiguous) operands on the GPU.

The reference's CUDA impls make the upstream gradients contiguous
(ops.py:279, 426, 583 of the reference) and hand x and the coefficients to
kernels that index them as dense row-major arrays.  These ops make every
operand contiguous before a launch, so a strided view gives the results of
its contiguous copy.  Each case feeds the same values once as contiguous
tensors and once as transposed or sliced views (inputs, upstream gradients
and the block's x) and requires the same bits in every output and gradient:
the ops, the block's eager autograd path, its checkpointed path through the
ops, the three-op path (FLASH_MHC_FUSED_PREMAP=0) and the no-grad forward.
"""

from __future__ import annotations

import os
from contextlib import contextmanager

import pytest
import torch

import flash_mhc

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16 = torch.bfloat16


def strided(t: torch.Tensor) -> torch.Tensor:
    """The values of t in a non-contiguous layout: dimensions stored in reverse
    order (a transposed view), or every other element of a 1-D buffer."""
    if t.dim() == 1:
        buf = torch.zeros(2 * t.numel(), dtype=t.dtype, device=t.device)
        view = buf[::2]
    else:
        buf = torch.zeros(tuple(reversed(t.shape)), dtype=t.dtype, device=t.device)
        view = buf.permute(*reversed(range(t.dim())))
    view.copy_(t)
    assert not view.is_contiguous() and torch.equal(view, t)
    return view


def rn(shape, seed, scale=1.0, dtype=BF16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=DEV) * scale).to(dtype)


@contextmanager
def env(**flags):
    old = {k: os.environ.get(k) for k in flags}
    os.environ.update({k: str(v) for k, v in flags.items()})
    try:
        yield
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def grads_of(op, inputs, upstream):
    """Outputs of op(*inputs) and the gradients of sum(out * upstream) for
    every input, with inputs as leaves in the layout they come in."""
    leaves = [t.detach().requires_grad_(t.is_floating_point()) for t in inputs]
    outs = op(*leaves)
    outs = outs if isinstance(outs, tuple) else (outs,)
    torch.autograd.backward([o for o in outs if o.requires_grad][: len(upstream)], upstream)
    return [o.detach() for o in outs], [None if l.grad is None else l.grad for l in leaves]


def assert_same(a, b, what):
    assert len(a) == len(b), what
    for i, (u, v) in enumerate(zip(a, b)):
        if u is None or v is None:
            assert u is None and v is None, f"{what}[{i}]"
            continue
        assert u.shape == v.shape and u.dtype == v.dtype, f"{what}[{i}]"
        assert torch.equal(u, v), f"{what}[{i}] differs"


@pytest.mark.parametrize("T,C", [(1000, 256), (3, 1024), (5000, 1024)])
def test_ops_with_strided_operands(T, C):
    nC = 4 * C
    x, W = rn((T, 4, C), 1), rn((32, nC), 2, 0.02)
    lo, go3, go4 = rn((T, C), 3), rn((T, C), 4), rn((T, 4, C), 5)
    h = torch.rand(T, 4, device=DEV)
    H, hp = torch.randn(T, 4, 4, device=DEV), torch.rand(T, 4, device=DEV)
    gproj = rn((T, 32), 6)
    ops = torch.ops.flash_mhc
    cases = {
        "fused_rmsnorm_project": (lambda a, b: ops.fused_rmsnorm_project(a, b)[0], (x.view(T, nC), W), (gproj,)),
        "fused_pre_map": (ops.fused_pre_map, (x, h), (go3,)),
        "fused_post_res": (ops.fused_post_res, (x, lo, H, hp), (go4,)),
    }
    for name, (op, inputs, up) in cases.items():
        print(f"[strided] {name} T={T} C={C}", flush=True)
        out_c, g_c = grads_of(op, inputs, up)
        out_s, g_s = grads_of(op, [strided(t) for t in inputs], [strided(u) for u in up])
        assert_same(out_c, out_s, f"{name} outputs")
        assert_same(g_c, g_s, f"{name} gradients")
    # The backward ops called directly with strided gradients.
    xf = x.view(T, nC)
    proj, inv = ops.fused_rmsnorm_project(xf, W)
    a = ops.fused_rmsnorm_project_bwd_dx(gproj, xf, W, proj, inv)
    b = ops.fused_rmsnorm_project_bwd_dx(strided(gproj), strided(xf), strided(W), strided(proj), strided(inv))
    assert torch.equal(a, b), "fused_rmsnorm_project_bwd_dx"
    a = ops.fused_pre_map_backward(go3, x, h)
    b = ops.fused_pre_map_backward(strided(go3), strided(x), strided(h))
    assert_same(list(a), list(b), "fused_pre_map_backward")
    a = ops.fused_post_res_backward(go4, x, lo, H, hp)
    b = ops.fused_post_res_backward(strided(go4), strided(x), strided(lo), strided(H), strided(hp))
    assert_same(list(a), list(b), "fused_post_res_backward")


def _block(C, ckpt, seed=0):
    torch.manual_seed(seed)
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False), activation_checkpointing=ckpt)
    return blk.to(DEV, BF16)


def _block_grads(blk, x, up):
    """out, x.grad and every parameter gradient; x comes in as given (a
    contiguous leaf or a strided view of a leaf)."""
    leaf = x._base if x._base is not None else x
    leaf = leaf.detach().requires_grad_(True)
    xin = leaf if x._base is None else leaf.permute(*reversed(range(leaf.dim())))
    blk.zero_grad(set_to_none=True)
    out = blk(xin)
    out.backward(up)
    gx = leaf.grad if x._base is None else leaf.grad.permute(*reversed(range(leaf.dim())))
    return [out.detach(), gx] + [p.grad for p in blk.parameters()]


@pytest.mark.parametrize("T,C,ckpt,premap", [(4096, 256, False, "1"), (4096, 256, True, "1"),
                                             (700, 512, False, "0"), (16500, 512, False, "1")])
def test_block_with_strided_input_and_gradient(T, C, ckpt, premap):
    print(f"[strided] block T={T} C={C} ckpt={ckpt} FLASH_MHC_FUSED_PREMAP={premap}", flush=True)
    with env(FLASH_MHC_FUSED_PREMAP=premap):
        blk = _block(C, ckpt)
        x, up = rn((T, 4, C), 10), rn((T, 4, C), 11)
        ref = _block_grads(blk, x, up)
        got = _block_grads(blk, strided(x), strided(up))
    assert_same(ref, got, "block output / x.grad / parameter grads")


@pytest.mark.parametrize("T,C", [(1, 4096), (64, 1024), (20000, 256)])
def test_block_nograd_forward_with_strided_input(T, C):
    print(f"[strided] eval forward T={T} C={C}", flush=True)
    blk = _block(C, False).eval()
    x = rn((T, 4, C), 12)
    with torch.no_grad():
        a = blk(x)
        b = blk(strided(x))
    assert torch.equal(a, b)
