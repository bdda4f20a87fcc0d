"""GPU tests of the autograd paths that the other suites reach only on the CPU
or only inside timing runs.

* K1's two-step backward rule of the reference (FLASH_MHC_FUSED_DW=0: the
  bwd_dx kernel, then grad_W as a matmul, ops.py:678-685 of the reference)
  against the oracle's grad_x and grad_W.
* The block's x-gradient sink (post-res's x-gradient added inside the pre-map
  backward instead of by autograd) under uses of autograd that a plain
  forward + backward does not exercise: retain_graph with two backward
  passes, torch.autograd.grad for x alone or for some parameters, a hook on x,
  x consumed a third time outside the block, and two stacked blocks.  Each is
  compared bit for bit with FLASH_MHC_FUSED_XGRAD=0 (autograd adds x's
  gradients itself).
* mhc_pre_map's backward when gradients also reach its h_pre and proj outputs
  (the branch that composes the K3, K2 and K1 backward kernels), compared bit
  for bit with the reference's separate ops in the same graph.
"""

from __future__ import annotations

import os
from contextlib import contextmanager

import pytest
import torch

import flash_mhc
from oracle import mhc_oracle as O
from parity import check_bf16, check_chain

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16 = torch.bfloat16


def randn(shape, seed, scale=1.0, dtype=BF16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


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


# ---------------------------------------------------------------------------
# K1: the reference's two-step backward rule


@pytest.mark.parametrize("T,C", [(4096, 1024), (257, 256), (1, 4096), (300, 100)])
def test_k1_two_step_rule_matches_oracle(T, C):
    """fused_rmsnorm_project's autograd with FLASH_MHC_FUSED_DW=0: grad_x from
    the bwd_dx op and grad_W = bf16(grad_out * inv_rms)^T @ x as a matmul,
    each against the oracle; grad_x equals the fused rule's bit for bit (the
    same dx arithmetic) and grad_W agrees with it to fp32 summation order."""
    nC = 4 * C
    x = randn((T, nC), 700 + T + C)
    x[:: max(1, T // 50)] *= 100  # 2% of the tokens far from unit RMS
    W = randn((32, nC), 701 + C, 0.02)
    go = randn((T, 32), 702 + T)
    grads = {}
    for flag in ("0", "1"):
        with env(FLASH_MHC_FUSED_DW=flag):
            xs = x.to(DEV).requires_grad_(True)
            Ws = W.to(DEV).requires_grad_(True)
            proj, inv = torch.ops.flash_mhc.fused_rmsnorm_project(xs, Ws)
            proj.backward(go.to(DEV))
            torch.cuda.synchronize()
            grads[flag] = (xs.grad, Ws.grad, proj.detach(), inv.detach())
    gx, gW, proj, inv = grads["0"]
    R, S = O.k1_bwd_dx(go, x, W, proj.cpu(), inv.cpu())
    check_bf16("two-step grad_x", gx, R, S, 64)
    R, S = O.k1_grad_W(go, x, inv.cpu())
    check_bf16("two-step grad_W", gW, R, S, T)
    assert torch.equal(gx, grads["1"][0])
    check_chain("two-step vs fused grad_W", gW.float().t(), grads["1"][1].float().t(), max_rate=1.0)


# ---------------------------------------------------------------------------
# The x-gradient sink under other uses of autograd


T_BLK, C_BLK = 1024, 512


def _block(seed=90, ckpt=False):
    torch.manual_seed(seed)
    blk = flash_mhc.MHCLiteBlock(4, C_BLK, torch.nn.Linear(C_BLK, C_BLK, bias=False),
                                 activation_checkpointing=ckpt).to(DEV, BF16)
    with torch.no_grad():
        blk.alpha_pre.fill_(0.8)
        blk.alpha_post.fill_(1.2)
        blk.alpha_res.fill_(1.7)
    return blk


def _both_modes(run, reordered=()):
    """run() under FLASH_MHC_FUSED_XGRAD=1 and =0; both return lists of
    tensors, equal bit for bit except those at the indices `reordered`: bf16
    sums of the same gradients in another order, held to the bf16 chain bound
    (a dropped or doubled gradient of O(1) fails it)."""
    with env(FLASH_MHC_FUSED_XGRAD="1"):
        a = run()
    with env(FLASH_MHC_FUSED_XGRAD="0"):
        b = run()
    torch.cuda.synchronize()
    assert len(a) == len(b)
    for i, (u, v) in enumerate(zip(a, b)):
        assert (u is None) == (v is None), i
        if u is None:
            continue
        if i in reordered:
            check_chain(f"output {i} (summation order)", u.float(), v.float(), max_rate=1.0)
        else:
            assert torch.equal(u, v), f"output {i}: max diff {float((u.float() - v.float()).abs().max()):.3e}"
    return a


@pytest.mark.parametrize("ckpt", [False, True])
def test_sink_retain_graph_two_backwards(ckpt):
    """Two backward passes through one graph (retain_graph=True): the sink's
    gradient reaches x on both, and x.grad accumulates the two sums."""
    x0 = randn((T_BLK, 4, C_BLK), 91)
    g1, g2 = randn((T_BLK, 4, C_BLK), 92), randn((T_BLK, 4, C_BLK), 93)

    def run():
        blk = _block(ckpt=ckpt)
        x = x0.to(DEV).requires_grad_(True)
        out = blk(x)
        out.backward(g1.to(DEV), retain_graph=True)
        first = x.grad.clone()
        out.backward(g2.to(DEV))
        return [out.detach(), first, x.grad, blk.W_all.weight.grad, blk.alpha_res.grad]

    _, first, total, *_ = _both_modes(run)
    assert not torch.equal(first, total)


def test_sink_autograd_grad_x_alone_and_some_parameters():
    """torch.autograd.grad for x alone, and for x with two parameters, instead
    of .backward(): the same gradients as autograd's own sum of x's three
    gradients, and no parameter's .grad is written."""
    x0 = randn((T_BLK, 4, C_BLK), 94)
    g = randn((T_BLK, 4, C_BLK), 95)

    def run():
        blk = _block()
        x = x0.to(DEV).requires_grad_(True)
        out = blk(x)
        (gx_only,) = torch.autograd.grad(out, x, g.to(DEV), retain_graph=True)
        gx, gW, gar = torch.autograd.grad(out, (x, blk.W_all.weight, blk.alpha_res), g.to(DEV))
        assert all(p.grad is None for p in blk.parameters())
        return [gx_only, gx, gW, gar]

    gx_only, gx, *_ = _both_modes(run)
    assert torch.equal(gx_only, gx)


def test_sink_hook_on_x_sees_the_summed_gradient_once():
    """A hook on x runs once, on x's whole gradient, and may replace it."""
    x0 = randn((T_BLK, 4, C_BLK), 96)
    g = randn((T_BLK, 4, C_BLK), 97)

    def run():
        blk = _block()
        x = x0.to(DEV).requires_grad_(True)
        seen = []

        def hook(grad):
            seen.append(grad.clone())
            return grad * 2

        x.register_hook(hook)
        blk(x).backward(g.to(DEV))
        assert len(seen) == 1
        return [seen[0], x.grad]

    seen, doubled = _both_modes(run)
    assert torch.equal(doubled, seen * 2)


def test_sink_x_with_a_consumer_outside_the_block():
    """x also feeds terms outside the block: their gradients are added to the
    block's.  Autograd adds x's gradients in the order they arrive; with the
    sink, post-res's and the pre-map's gradients arrive already summed, so
    x.grad is the same bf16 sum in another association (held to the bf16
    chain bound); everything else is equal bit for bit."""
    x0 = randn((T_BLK, 4, C_BLK), 98)
    g = randn((T_BLK, 4, C_BLK), 99)

    def run():
        blk = _block()
        x = x0.to(DEV).requires_grad_(True)
        out = blk(x) + 0.5 * x
        loss = (out.float() * g.to(DEV).float()).sum() + (x.float() ** 2).sum() * 1e-3
        loss.backward()
        return [out.detach(), x.grad, blk.W_all.weight.grad, blk.W_all.bias.grad]

    _both_modes(run, reordered=(1,))


@pytest.mark.parametrize("ckpt", [False, True])
def test_sink_two_stacked_blocks(ckpt):
    """Block 2's x is block 1's output (not a leaf): each block's sink brings
    its post-res x-gradient into its own pre-map backward."""
    x0 = randn((T_BLK, 4, C_BLK), 100)
    g = randn((T_BLK, 4, C_BLK), 101)

    def run():
        b1, b2 = _block(seed=102, ckpt=ckpt), _block(seed=103, ckpt=ckpt)
        x = x0.to(DEV).requires_grad_(True)
        out = b2(b1(x))
        out.backward(g.to(DEV))
        return [out.detach(), x.grad, b1.W_all.weight.grad, b2.W_all.weight.grad, b1.layer.weight.grad,
                b2.alpha_pre.grad]

    _both_modes(run)


# ---------------------------------------------------------------------------
# mhc_pre_map with gradients reaching h_pre and proj


@pytest.mark.parametrize("T,C", [(2048, 1024), (37, 256), (300, 100)])
@pytest.mark.parametrize("with_layer_input", [True, False])
def test_pre_map_op_gradients_through_h_pre_and_proj(T, C, with_layer_input):
    """Gradients into mhc_pre_map's h_pre and proj outputs (besides the layer
    input, H_merged and h_post) take the backward's compose branch: the same
    outputs and gradients, bit for bit, as the reference's separate ops
    (fused_rmsnorm_project, the coefficient op, fused_pre_map) in the same
    graph, where autograd adds the extra gradients of proj and h_pre."""
    nC = 4 * C
    x0 = randn((T, 4, C), 110 + T + C)
    W0 = randn((32, nC), 111 + C, 0.02)
    g = torch.Generator().manual_seed(112)
    params0 = [torch.tensor([0.8]), torch.tensor([1.2]), torch.tensor([1.7]), torch.randn(32, generator=g) * 0.5]
    perm = O.permutation_matrices(4)[0].to(DEV)
    g_li = randn((T, C), 113)
    g_H = randn((T, 4, 4), 114, dtype=torch.float32)
    g_hq = randn((T, 4), 115, dtype=torch.float32)
    g_hp = randn((T, 4), 116, dtype=torch.float32)
    g_proj = randn((T, 32), 117)

    def loss_of(li, H, hq, hp, proj):
        terms = [(H * g_H.to(DEV)).sum(), (hq * g_hq.to(DEV)).sum(), (hp * g_hp.to(DEV)).sum(),
                 (proj.float() * g_proj.to(DEV).float()).sum()]
        if with_layer_input:
            terms.append((li.float() * g_li.to(DEV).float()).sum())
        return sum(terms)

    def leaves():
        return ([x0.to(DEV).requires_grad_(True), W0.to(DEV).requires_grad_(True)]
                + [p.to(DEV).requires_grad_(True) for p in params0])

    # The pre-map op.
    x, W, ap, apo, ar, b = leaves()
    li, H, hq, hp, proj, inv, _sink = torch.ops.flash_mhc.mhc_pre_map(x, W, ap, apo, ar, b, perm)
    loss_of(li, H, hq, hp, proj).backward()
    got = [li, H, hq, hp, proj, inv] + [t.grad for t in (x, W, ap, apo, ar, b)]

    # The reference's separate ops.
    x, W, ap, apo, ar, b = leaves()
    proj_r, inv_r = torch.ops.flash_mhc.fused_rmsnorm_project(x.reshape(T, nC), W)
    hp_r, hq_r, H_r = torch.ops.flash_mhc.mhc_coefficients(proj_r, ap, apo, ar, b, perm)
    li_r = torch.ops.flash_mhc.fused_pre_map(x, hp_r)
    loss_of(li_r, H_r, hq_r, hp_r, proj_r).backward()
    want = [li_r, H_r, hq_r, hp_r, proj_r, inv_r] + [t.grad for t in (x, W, ap, apo, ar, b)]
    torch.cuda.synchronize()

    names = ["layer_input", "H_merged", "h_post", "h_pre", "proj", "inv_rms", "grad_x", "grad_W", "grad_alpha_pre",
             "grad_alpha_post", "grad_alpha_res", "grad_bias"]
    for name, a, r in zip(names, got, want):
        assert torch.equal(a.detach(), r.detach()), f"{name}: max diff {float((a.float() - r.float()).abs().max()):.3e}"
