"""GPU parity of the pre-map entry points (flash_mhc::mhc_pre_map: K1, K2, K3
forward; K3's reduction, K2 and K1 with K3's term folded into grad_x backward)
against the oracle stage by stage and against the separate kernels.

Stage checks use the kernel's own upstream outputs as the oracle's inputs, so
each stage is held to its own rule (tests/parity.py): proj to the K1 bf16 rule
with nC terms, inv_rms to a relative bound, the K2 outputs to the chain rule
against oracle/k2_oracle.py, layer_input to the K3 bf16 rule.
"""

from __future__ import annotations

import os

import pytest
import torch

import flash_mhc
from flash_mhc import kernels as K
from oracle import k2_oracle as K2O
from oracle import mhc_oracle as O
from parity import check_bf16, check_chain, check_rel

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16 = torch.bfloat16
PERM = O.permutation_matrices(4)[0]


def randn(shape, seed, scale=1.0, dtype=BF16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def _params(seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.tensor([0.8]), torch.tensor([1.2]), torch.tensor([1.7]), torch.randn(32, generator=g) * 0.5]


# (T, C): the metric width, narrow and wide rows, ragged token counts, and
# C % 8 != 0 (the element-wise paths).
SHAPES = [(1, 1024), (37, 1024), (4096, 1024), (300, 256), (33, 512), (100, 2048), (37, 4096),
          (5, 8192), (45, 100), (3, 16384)]


@pytest.mark.parametrize("T,C", SHAPES)
def test_premap_fwd_stages(T, C):
    nC = 4 * C
    x = randn((T, 4, C), 1000 + T + C)
    g = torch.Generator().manual_seed(7)
    idx = torch.randperm(T, generator=g)[: max(1, T // 100)]
    x[idx] = (x[idx].float() * 100).to(BF16)  # 1% of the tokens x100
    W = randn((32, nC), 2000 + C, 0.02)
    ap, apo, ar, b = _params(C)
    li, H, hq, hp, proj, inv = K.premap_fwd(x.to(DEV), W.to(DEV), *[t.to(DEV) for t in (ap, apo, ar, b, PERM)])
    torch.cuda.synchronize()
    R, S, invR = O.k1_fwd(x.view(T, nC), W)
    check_bf16("premap proj", proj, R, S, nC)
    check_rel("premap inv_rms", inv, invR, rtol=4 * nC ** 0.5 * 2.0 ** -24 + 4 * 2.0 ** -24)
    f = K2O.k2_fwd(proj.cpu(), ap, apo, ar, b, PERM)
    check_chain("premap h_pre", hp, f["h_pre"])
    check_chain("premap h_post", hq, f["h_post"])
    check_chain("premap H_merged", H, f["H_merged"])
    R, S = O.k3_fwd(x, hp.cpu())
    check_bf16("premap layer_input", li, R, S, 4)


@pytest.mark.parametrize("T,C", [(8192, 1024), (300, 1024), (1, 4096), (64, 4096), (257, 4096), (5, 8192),
                                 (3, 1000), (2721, 1024), (4000, 1024), (6000, 512), (8193, 1024), (12000, 512),
                                 (16000, 1024), (16383, 512), (33000, 2048),
                                 (24576, 256), (28000, 256), (28673, 256)])
def test_premap_matches_three_kernels(T, C):
    """Same outputs as K1 + K2 + K3 launched separately (few tokens: both
    take K1's column-split kernel; where no split is planned the pre-map runs
    its one-kernel tile path, K2 and K3 inside K1's workgroups, on tiles of
    16 to 64 tokens; from 513 tiles on the K1 op walks its tiles with two
    workgroups per CU, k1_fwd_persist, which must give the tile's bits)."""
    x = randn((T, 4, C), 3).to(DEV)
    W = randn((32, 4 * C), 4, 0.02).to(DEV)
    p = [t.to(DEV) for t in (*_params(5), PERM)]
    li, H, hq, hp, proj, inv = K.premap_fwd(x, W, *p)
    proj1, inv1 = K.k1_fwd(x.view(T, -1), W)
    hp1, hq1, H1 = K.k2_fwd(proj1, *p)
    li1 = K.k3_fwd(x, hp1)
    for a, b in ((proj, proj1), (inv, inv1), (H, H1), (hq, hq1), (hp, hp1), (li, li1)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("T,C", [(1, 4096), (300, 1024), (8192, 256)])
def test_premap_ops_zero_their_sinks(T, C):
    """mhc_pre_map and mhc_pre_map_coeffs return zero-stride gradient sinks
    whose one stored element the pre-map launches set to zero (no fill kernel
    of their own): zero even when the allocator hands out memory that held
    other values (few tokens: K1's split path; T = 8192: the one-pass path)."""
    x = randn((T, 4, C), 11).to(DEV)
    W = randn((32, 4 * C), 12, 0.02).to(DEV)
    p = [t.to(DEV) for t in (*_params(13), PERM)]
    for _ in range(2):
        junk = torch.full((1 << 16,), -3.0, device=DEV, dtype=BF16)  # dirty blocks for the next allocations
        del junk
        x_sink = torch.ops.flash_mhc.mhc_pre_map(x, W, *p)[-1]
        outs = torch.ops.flash_mhc.mhc_pre_map_coeffs(x, W, *p)
        torch.cuda.synchronize()
        for name, sink, shape in (("mhc_pre_map x_sink", x_sink, (T, 4, C)),
                                  ("coeffs x_sink", outs[-2], (T, 4, C)), ("coeffs li_sink", outs[-1], (T, C))):
            assert tuple(sink.shape) == shape and all(st == 0 for st in sink.stride()), name
            assert float(sink.as_strided((1,), (1,)).float().item()) == 0.0, name


def _block_run(flag, T, C, ckpt=False, seed=80):
    old = os.environ.get("FLASH_MHC_FUSED_PREMAP")
    os.environ["FLASH_MHC_FUSED_PREMAP"] = flag
    try:
        torch.manual_seed(seed)
        layer = torch.nn.Linear(C, C, bias=False).to(BF16)
        blk = flash_mhc.MHCLiteBlock(4, C, layer, activation_checkpointing=ckpt).to(DEV)
        with torch.no_grad():
            blk.alpha_pre.fill_(0.8)
            blk.alpha_post.fill_(1.2)
            blk.alpha_res.fill_(1.7)
        x = randn((T, 4, C), seed).to(DEV).requires_grad_(True)
        out = blk(x)
        out.backward(randn(out.shape, seed + 1).to(DEV))
        torch.cuda.synchronize()
        return out.detach(), x.grad, {n: p.grad for n, p in blk.named_parameters()}
    finally:
        if old is None:
            os.environ.pop("FLASH_MHC_FUSED_PREMAP", None)
        else:
            os.environ["FLASH_MHC_FUSED_PREMAP"] = old


@pytest.mark.parametrize("T,C", [(4096, 1024), (20000, 2048), (257, 256), (5, 4096)])
def test_checkpointed_two_op_region_equals_eager_block(T, C):
    """With activation checkpointing the eager block runs the pre-map region
    as the single op mhc_pre_map; under torch.compile and other dispatch
    modes it runs mhc_pre_map_coeffs and a checkpointed mhc_pre_map_mix.  At
    token counts where both take the same K1 kernel (below the single-read
    forward's, or C above 1024) the two give the same output, x gradient and
    parameter gradients, bit for bit."""
    from contextlib import nullcontext

    torch.manual_seed(81)
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False), activation_checkpointing=True)
    blk = blk.to(DEV, BF16)
    x0 = randn((T, 4, C), 82).to(DEV, BF16)
    up = randn((T, 4, C), 83).to(DEV, BF16)
    res = []
    for two_op in (False, True):
        blk.zero_grad(set_to_none=True)
        x = x0.clone().requires_grad_(True)
        if two_op:
            out = blk._run(x, blk._mhc_pre_map_triton, blk._mhc_post_res_triton, nullcontext(), {},
                           checkpoint_post_res=False)
        else:
            out = blk(x)
        out.backward(up)
        torch.cuda.synchronize()
        res.append([out.detach(), x.grad] + [p.grad for p in blk.parameters()])
    names = ["out", "grad_x"] + [n for n, _ in blk.named_parameters()]
    for name, a, b in zip(names, *res):
        assert torch.equal(a, b), f"{name}: {int((a != b).sum())} of {a.numel()} differ"


@pytest.mark.parametrize("ckpt", [False, True])
def test_block_premap_equals_separate_ops(ckpt):
    """The block with the pre-map op vs K1, K2, K3 as separate ops: the same
    forward; gradients to the bf16 chain bound (x's three gradients are summed
    as g4 + (g3 + g1) instead of (g4 + g3) + g1)."""
    T, C = 4096, 1024
    o1, gx1, gp1 = _block_run("1", T, C, ckpt)
    o0, gx0, gp0 = _block_run("0", T, C, ckpt)
    assert torch.equal(o1, o0)
    check_chain("block grad_x", gx1.float(), gx0.float(), max_rate=1.0)
    for n in gp0:
        a, b = gp1[n].float().cpu(), gp0[n].float().cpu()
        tol = 2e-2 * b.abs() + 1e-2 * float(b.abs().max()) + 1e-6
        assert bool(((a - b).abs() <= tol).all()), f"{n}: max diff {float((a - b).abs().max()):.3e}"


@pytest.mark.parametrize("T,C", [(4096, 1024), (257, 1024), (1, 256), (777, 256), (6144, 1024), (6145, 1024),
                                 (2000, 2048), (300, 1000), (333, 100), (45, 24)])
def test_premap_bwd_equals_composed_kernels(T, C):
    """The fused pre-map backward equals K3 backward + K2 backward + K1
    backward (with grad_W) + the bf16 sum of x's two gradients: bit for bit on
    the MFMA path (K1 adds bf16(h_pre go) to bf16(dx) in its store).  For
    C % 8 != 0 K3 writes its term and K1's element-wise kernel adds dx to it,
    while the separate K1 op can still take its MFMA kernel (n C % 8 == 0):
    their fp32 summation orders differ, so those shapes are held to the bf16
    chain bound.  Up to 6144 tokens with 32 or 64 lanes per token in K3's
    backward (C = 256 ... 2040) K3's reduce and K2's backward run as one kernel
    (T = 777 at C = 256: half a wave per token, a ragged last workgroup;
    6144 / 6145: the last fused size and the first separate one)."""
    nC = 4 * C
    x = randn((T, 4, C), 3000 + T + C).to(DEV)
    W = randn((32, nC), 3001 + C, 0.02).to(DEV)
    p = [t.to(DEV) for t in (*_params(C), PERM)]
    li, H, hq, hp, proj, inv = K.premap_fwd(x, W, *p)
    g_li = randn((T, C), 3002 + T).to(DEV)
    g_hq = randn((T, 4), 3003, dtype=torch.float32).to(DEV)
    g_H = randn((T, 4, 4), 3004, dtype=torch.float32).to(DEV)
    gx, gW, ga1, ga2, ga3, gb = K.premap_bwd(x, W, *p, hp, proj, inv, g_li, g_hq, g_H)
    gx3, gh = K.k3_bwd(g_li, x, hp)
    gp, ra1, ra2, ra3, rb_ = K.k2_bwd(proj, *p, gh, g_hq, g_H)
    gx1, rW = K.k1_bwd(gp, x.view(T, nC), W, proj, inv)
    torch.cuda.synchronize()
    for a, b in ((ga1, ra1), (ga2, ra2), (ga3, ra3), (gb, rb_)):
        assert torch.equal(a, b)
    if C % 8 == 0:
        assert torch.equal(gx, gx3 + gx1.view(T, 4, C))
        assert torch.equal(gW, rW)
    else:
        check_chain("grad_x (element-wise paths)", gx.float(), (gx3 + gx1.view(T, 4, C)).float(), max_rate=1.0)
        check_chain("grad_W (element-wise paths)", gW.float().t(), rW.float().t(), max_rate=1.0)


def test_premap_bwd_null_grads_and_empty():
    T, C = 300, 256
    x = randn((T, 4, C), 40).to(DEV)
    W = randn((32, 4 * C), 41, 0.02).to(DEV)
    p = [t.to(DEV) for t in (*_params(C), PERM)]
    li, H, hq, hp, proj, inv = K.premap_fwd(x, W, *p)
    g_li = randn((T, C), 42).to(DEV)
    gx, gW, *_ = K.premap_bwd(x, W, *p, hp, proj, inv, g_li, None, None)
    gx3, gh = K.k3_bwd(g_li, x, hp)
    gp = K.k2_bwd(proj, *p, gh, None, None)[0]
    gx1, rW = K.k1_bwd(gp, x.view(T, -1), W, proj, inv)
    assert torch.equal(gx, gx3 + gx1.view(T, 4, C)) and torch.equal(gW, rW)
    e = torch.empty((0, 4, C), dtype=BF16, device=DEV)
    f32 = lambda *s: torch.empty(*s, device=DEV)
    g0 = K.premap_bwd(e, W, *p, f32(0, 4), torch.empty((0, 32), dtype=BF16, device=DEV), f32(0),
                      torch.empty((0, C), dtype=BF16, device=DEV), None, None)
    assert g0[0].shape == (0, 4, C) and all(float(t.float().abs().sum()) == 0.0 for t in g0[1:])


@pytest.mark.parametrize("T,C", [(4096, 1024), (257, 1024), (1, 256), (300, 1000), (333, 100), (45, 24)])
def test_premap_bwd_incoming_grad(T, C):
    """grad_x_in (post-res's x-gradient in a block) is added in K1's store:
    grad_x = bf16(grad_x_in + the pre-map gradient), bit for bit the sum
    autograd forms, on the MFMA path and on the element-wise path (C % 8 != 0);
    the other gradients are unchanged."""
    nC = 4 * C
    x = randn((T, 4, C), 5000 + T + C).to(DEV)
    W = randn((32, nC), 5001 + C, 0.02).to(DEV)
    p = [t.to(DEV) for t in (*_params(C), PERM)]
    li, H, hq, hp, proj, inv = K.premap_fwd(x, W, *p)
    g_li = randn((T, C), 5002 + T).to(DEV)
    g_hq = randn((T, 4), 5003, dtype=torch.float32).to(DEV)
    g_H = randn((T, 4, 4), 5004, dtype=torch.float32).to(DEV)
    g_in = randn((T, 4, C), 5005 + T).to(DEV)
    a = K.premap_bwd(x, W, *p, hp, proj, inv, g_li, g_hq, g_H, g_in)
    b = K.premap_bwd(x, W, *p, hp, proj, inv, g_li, g_hq, g_H)
    torch.cuda.synchronize()
    assert torch.equal(a[0], g_in + b[0])
    for u, v in zip(a[1:], b[1:]):
        assert torch.equal(u, v)


def test_premap_bwd_rejects_overlapping_incoming_grad():
    """grad_x_in must not overlap grad_x: the entry point returns an error
    before launching anything."""
    from flash_mhc import _abi

    T, C = 64, 256
    x = randn((T, 4, C), 60).to(DEV)
    W = randn((32, 4 * C), 61, 0.02).to(DEV)
    p = [t.to(DEV) for t in (*_params(C), PERM)]
    li, H, hq, hp, proj, inv = K.premap_fwd(x, W, *p)
    g_li = randn((T, C), 62).to(DEV)
    gW = torch.empty_like(W)
    ga = [torch.empty(1, device=DEV) for _ in range(3)]
    gb = torch.empty(32, device=DEV)
    lib = _abi.load()
    nbytes = int(lib.fmhc_premap_bwd_workspace_bytes(T, C))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    P = lambda t: t.data_ptr()
    shifted = torch.empty(x.numel() + 8, dtype=BF16, device=DEV)
    gx = shifted[8:].view(T, 4, C)
    for g_in in (gx, shifted[:-8]):  # the same buffer, and one shifted by 16 bytes
        st = lib.fmhc_premap_bwd(P(x), P(W), *[P(t) for t in p], 0, P(hp), P(proj), P(inv), P(g_li), None, None,
                                 P(g_in), P(gx), P(gW), *[P(t) for t in ga], P(gb), P(ws), nbytes, T, C, 4,
                                 _abi.stream_of(x))
        assert st == 1  # FMHC_ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("ckpt", [False, True])
def test_block_xgrad_sink_equals_autograd_sum(ckpt):
    """The block with post-res's x-gradient added in the pre-map backward
    (FLASH_MHC_FUSED_XGRAD=1) and with autograd adding it (=0): identical
    outputs and gradients, bit for bit."""
    old = os.environ.get("FLASH_MHC_FUSED_XGRAD")
    try:
        os.environ["FLASH_MHC_FUSED_XGRAD"] = "1"
        o1, gx1, gp1 = _block_run("1", 4096, 1024, ckpt)
        os.environ["FLASH_MHC_FUSED_XGRAD"] = "0"
        o0, gx0, gp0 = _block_run("1", 4096, 1024, ckpt)
    finally:
        if old is None:
            os.environ.pop("FLASH_MHC_FUSED_XGRAD", None)
        else:
            os.environ["FLASH_MHC_FUSED_XGRAD"] = old
    assert torch.equal(o1, o0)
    assert torch.equal(gx1, gx0)
    for n in gp0:
        assert torch.equal(gp1[n], gp0[n]), n
