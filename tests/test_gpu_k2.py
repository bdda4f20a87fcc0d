"""GPU parity of the fused K2 kernels (flash_mhc::mhc_coefficients and its
backward) against the oracle's step-by-step bf16 chain (oracle/k2_oracle.py),
and of the block with K2 fused against the block running the reference's
PyTorch ops for K2 (FLASH_MHC_FUSED_K2=0).

The oracle's backward follows the rounding of PyTorch's GPU kernels for the
sigmoid and softmax backward steps (rounding="gpu"); test_oracle_gpu_rounding
pins those two steps against torch's own GPU ops, and
test_k2_matches_torch_gpu_chain compares the kernels with torch's GPU autograd
through the reference's op sequence.

Rules (tests/parity.py): chain outputs may differ from the oracle only by rare
last-bit flips (exp, fp32 summation order) -- at most 1e-3 of the elements,
each within 1 ulp of itself plus 4 ulps of its token's largest value; the
alpha / bias gradients (sums over tokens) are held to the bf16 rule with the
summation-order term of their T * lanes terms.
"""

from __future__ import annotations

import os

import pytest
import torch

import flash_mhc
from flash_mhc import kernels as K
from oracle import k2_oracle as K2O
from oracle import mhc_oracle as O
from parity import check_bf16, check_chain

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16 = torch.bfloat16
F64 = torch.float64


def _case(T, seed, proj_scale=3.0, block_init=False):
    g = torch.Generator().manual_seed(seed)
    proj = (torch.randn(T, 32, generator=g) * proj_scale).to(BF16)
    if block_init:  # MHCLiteBlock's initial alphas and nn.Linear's bias range
        alphas = [torch.tensor([0.01])] * 3
        bias = (torch.rand(32, generator=g) * 2 - 1) / 64.0
    else:
        alphas = [torch.tensor([v]) for v in (0.9, 1.3, 2.1)]
        bias = torch.randn(32, generator=g) * 0.5
    grads = [torch.randn(T, 4, generator=g), torch.randn(T, 4, generator=g), torch.randn(T, 4, 4, generator=g)]
    return proj, alphas, bias, grads


def _dev(ts):
    return [t.to(DEV) for t in ts]


PERM = O.permutation_matrices(4)[0]


@pytest.mark.parametrize("T,seed,block_init", [(1, 0, False), (255, 1, False), (4096, 2, False),
                                                (4096, 3, True), (8192, 5, False), (65536, 4, False)])
def test_k2_fwd_matches_chain(T, seed, block_init):
    proj, alphas, bias, _ = _case(T, seed, block_init=block_init)
    hp, hq, H = K.k2_fwd(*_dev([proj, *alphas, bias, PERM]))
    torch.cuda.synchronize()
    f = K2O.k2_fwd(proj, *alphas, bias, PERM)
    check_chain("k2 h_pre", hp, f["h_pre"])
    check_chain("k2 h_post", hq, f["h_post"])
    check_chain("k2 H_merged", H, f["H_merged"])


@pytest.mark.parametrize("T,seed,block_init", [(1, 10, False), (255, 11, False), (4096, 12, False),
                                                (4096, 13, True), (8192, 15, False), (65536, 14, False)])
def test_k2_bwd_matches_chain(T, seed, block_init):
    proj, alphas, bias, grads = _case(T, seed, block_init=block_init)
    gp, ga1, ga2, ga3, gb = K.k2_bwd(*_dev([proj, *alphas, bias, PERM, *grads]))
    torch.cuda.synchronize()
    r = K2O.k2_bwd(proj, *alphas, bias, PERM, *grads)
    check_chain("k2 grad_proj", gp, r["grad_proj"])
    for name, got, n in (("grad_alpha_pre", ga1, 4 * T), ("grad_alpha_post", ga2, 4 * T),
                         ("grad_alpha_res", ga3, 24 * T)):
        R, S = r[name]
        check_bf16(name, got.to(BF16), torch.tensor([R], dtype=F64), torch.tensor([S], dtype=F64), n)
    R, S = r["grad_bias"]
    check_bf16("grad_bias", gb.to(BF16), torch.as_tensor(R), torch.as_tensor(S), T)


def test_k2_null_grads_misaligned_and_empty():
    T = 300
    proj, alphas, bias, grads = _case(T, 20)
    # proj at a 2-byte offset: the element-wise load / store path.
    buf = torch.empty(T * 32 + 1, dtype=BF16, device=DEV)
    pm = buf[1:].view(T, 32)
    pm.copy_(proj.to(DEV))
    assert pm.data_ptr() % 16 != 0
    hp, hq, H = K.k2_fwd(pm, *_dev([*alphas, bias, PERM]))
    f = K2O.k2_fwd(proj, *alphas, bias, PERM)
    check_chain("k2 H_merged (misaligned)", H, f["H_merged"])
    gp, ga1, ga2, ga3, gb = K.k2_bwd(pm, *_dev([*alphas, bias, PERM]), None, grads[1].to(DEV), None)
    r = K2O.k2_bwd(proj, *alphas, bias, PERM, None, grads[1], None)
    check_chain("k2 grad_proj (h_post grad only)", gp, r["grad_proj"])
    R, S = r["grad_alpha_post"]
    check_bf16("grad_alpha_post", ga2.to(BF16), torch.tensor([R], dtype=F64), torch.tensor([S], dtype=F64), 4 * T)
    e = torch.empty((0, 32), dtype=BF16, device=DEV)
    hp0, _, H0 = K.k2_fwd(e, *_dev([*alphas, bias, PERM]))
    assert hp0.shape == (0, 4) and H0.shape == (0, 4, 4)
    g0 = K.k2_bwd(e, *_dev([*alphas, bias, PERM]), None, None, None)
    assert g0[0].shape == (0, 32) and all(float(t.abs().sum()) == 0.0 for t in g0[1:])


@pytest.mark.parametrize("T", [8193, 9001])
def test_k2_misaligned_many_tokens_equals_aligned(T):
    """Above 6144 tokens (four lanes per token, 64 per workgroup; T = 9001
    leaves a ragged last workgroup) proj at a 2-byte offset takes the
    element-wise loads and stores and gives the aligned call's bits: outputs,
    grad_proj and the parameter gradients."""
    proj, alphas, bias, grads = _case(T, 30)
    prm = _dev([*alphas, bias, PERM])
    g = _dev(list(grads))
    buf = torch.empty(T * 32 + 1, dtype=BF16, device=DEV)
    pm = buf[1:].view(T, 32)
    pm.copy_(proj.to(DEV))
    assert pm.data_ptr() % 16 != 0
    pa = proj.to(DEV)
    for u, v in zip(K.k2_fwd(pm, *prm), K.k2_fwd(pa, *prm)):
        assert torch.equal(u, v)
    for u, v in zip(K.k2_bwd(pm, *prm, *g), K.k2_bwd(pa, *prm, *g)):
        assert torch.equal(u, v)


@pytest.mark.parametrize("which", ["h_post only", "h_pre and H"])
def test_k2_bwd_many_tokens_null_grads(which):
    """Above 6144 tokens (four lanes per token) a missing output gradient counts
    as zero, as in the 32-lane kernel: grad_proj and the parameter gradients
    against the chain's oracle, T = 7001 (a ragged last workgroup)."""
    T = 7001
    proj, alphas, bias, grads = _case(T, 40)
    g = list(grads)
    if which == "h_post only":
        g[0], g[2] = None, None
    else:
        g[1] = None
    gp, ga1, ga2, ga3, gb = K.k2_bwd(*_dev([proj, *alphas, bias, PERM]), *[None if t is None else t.to(DEV) for t in g])
    torch.cuda.synchronize()
    r = K2O.k2_bwd(proj, *alphas, bias, PERM, *g)
    check_chain("k2 grad_proj (null grads)", gp, r["grad_proj"])
    for name, got, n in (("grad_alpha_pre", ga1, 4 * T), ("grad_alpha_post", ga2, 4 * T),
                         ("grad_alpha_res", ga3, 24 * T)):
        R, S = r[name]
        check_bf16(name, got.to(BF16), torch.tensor([R], dtype=F64), torch.tensor([S], dtype=F64), n)


def test_k2_deterministic():
    proj, alphas, bias, grads = _case(20000, 30)
    args = _dev([proj, *alphas, bias, PERM, *grads])
    a = K.k2_bwd(*args)
    b = K.k2_bwd(*args)
    assert all(torch.equal(u, v) for u, v in zip(a, b))


def _block_run(flag, T, C, seed=50):
    # K2 alone: the one-pass pre-map (which also fuses K1 and K3) stays off.
    old = {k: os.environ.get(k) for k in ("FLASH_MHC_FUSED_K2", "FLASH_MHC_FUSED_PREMAP")}
    os.environ["FLASH_MHC_FUSED_K2"] = flag
    os.environ["FLASH_MHC_FUSED_PREMAP"] = "0"
    try:
        torch.manual_seed(seed)
        layer = torch.nn.Linear(C, C, bias=False).to(BF16)
        blk = flash_mhc.MHCLiteBlock(4, C, layer).to(DEV)  # fp32 block parameters, bf16 layer
        with torch.no_grad():  # away from the tiny initial alphas, so every path matters
            blk.alpha_pre.fill_(0.8)
            blk.alpha_post.fill_(1.2)
            blk.alpha_res.fill_(1.7)
        x = (torch.randn(T, 4, C, generator=torch.Generator().manual_seed(seed)) * 1.0).to(BF16).to(DEV)
        x.requires_grad_(True)
        out = blk(x)
        g = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed + 1)).to(BF16).to(DEV)
        out.backward(g)
        torch.cuda.synchronize()
        return out.detach(), x.grad, {n: p.grad for n, p in blk.named_parameters()}
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def test_block_fused_k2_equals_reference_ops():
    """Same block, K2 fused vs K2 as the reference's PyTorch ops: the forward
    is equal up to rare last-bit flips, and so are the gradients."""
    T, C = 4096, 1024
    o1, gx1, gp1 = _block_run("1", T, C)
    o0, gx0, gp0 = _block_run("0", T, C)
    check_chain("block out (fused K2 vs reference ops)", o1.float(), o0.float())
    check_chain("block grad_x (fused K2 vs reference ops)", gx1.float(), gx0.float(), max_rate=1e-2)
    for n in gp0:
        a, b = gp1[n].float().cpu(), gp0[n].float().cpu()
        tol = 2e-2 * b.abs() + 1e-2 * float(b.abs().max()) + 1e-6
        assert bool(((a - b).abs() <= tol).all()), f"{n}: max diff {float((a - b).abs().max()):.3e}"


def test_oracle_gpu_rounding():
    """The oracle's rounding="gpu" sigmoid / softmax backward steps equal torch's
    GPU aten ops on bf16 (up to fp32 summation order in the softmax sum)."""
    g = torch.Generator().manual_seed(60)
    z = (torch.randn(1 << 14, 24, generator=g) * 3).to(BF16)
    gr = torch.randn(1 << 14, 24, generator=g).to(BF16)
    y = torch.sigmoid(z.to(DEV))
    got = torch.ops.aten.sigmoid_backward(gr.to(DEV), y).float().cpu()
    check_chain("sigmoid_backward", K2O.sigmoid_bwd(gr.float().numpy(), y.float().cpu().numpy()), got, max_rate=0.0)
    y = torch.softmax(z.to(DEV), -1)
    got = torch.ops.aten._softmax_backward_data(gr.to(DEV), y, -1, BF16).float().cpu()
    check_chain("softmax_backward", K2O.softmax_bwd(gr.float().numpy(), y.float().cpu().numpy()), got, max_rate=1e-4)


def test_k2_matches_torch_gpu_chain():
    """Kernels vs torch's GPU forward + autograd through the reference's op
    sequence (mhc_oracle.coefficients = block.py:161-170, then .float())."""
    T = 65536
    proj, alphas, bias, grads = _case(T, 70)
    p = proj.to(DEV).requires_grad_(True)
    a = [t.to(DEV).requires_grad_(True) for t in alphas]
    b = bias.to(DEV).requires_grad_(True)
    h1, h2, h3, _ = O.coefficients(p, b, a[0], a[1], a[2], PERM.to(DEV), 4)
    outs = (h1.float(), h2.float(), h3.float())
    sum((o * t.to(DEV)).sum() for o, t in zip(outs, grads)).backward()
    hp, hq, H = K.k2_fwd(*_dev([proj, *alphas, bias, PERM]))
    gp, ga1, ga2, ga3, gb = K.k2_bwd(*_dev([proj, *alphas, bias, PERM, *grads]))
    for name, got, ref in (("h_pre", hp, outs[0]), ("h_post", hq, outs[1]), ("H_merged", H, outs[2]),
                           ("grad_proj", gp, p.grad)):
        check_chain(name + " vs torch GPU", got.float(), ref.float())
    for name, got, ref in (("grad_alpha_pre", ga1, a[0].grad), ("grad_alpha_post", ga2, a[1].grad),
                           ("grad_alpha_res", ga3, a[2].grad), ("grad_bias", gb, b.grad)):
        u = ref.double().cpu()
        assert bool(((got.double().cpu() - u).abs() <= 2.0 ** -7 * u.abs() + 1e-6).all()), name


def test_k2_bf16_parameters_equal_fp32():
    """Parameters stored in bf16 (a bf16 block) are read as they are, with no
    conversion launches: outputs and gradients equal those from the same values
    in fp32 (the kernels round every parameter to bf16 on use), and the
    parameter gradients come back in bf16, the fp32 ones' values rounded."""
    T = 3000
    proj, alphas, bias, grads = _case(T, 80)
    p32 = [t.to(BF16).float() for t in (*alphas, bias, PERM)]  # bf16-representable values
    p16 = [t.to(BF16) for t in p32]
    a = K.k2_fwd(*_dev([proj, *p32]))
    b = K.k2_fwd(*_dev([proj, *p16]))
    assert all(torch.equal(u, v) for u, v in zip(a, b))
    ga = K.k2_bwd(*_dev([proj, *p32, *grads]))
    gb = K.k2_bwd(*_dev([proj, *p16, *grads]))
    assert torch.equal(ga[0], gb[0])
    for u, v in zip(ga[1:], gb[1:]):
        assert v.dtype == BF16 and torch.equal(u, v.float())
    x = (torch.randn(T, 4, 256, generator=torch.Generator().manual_seed(81))).to(BF16).to(DEV)
    W = (torch.randn(32, 1024, generator=torch.Generator().manual_seed(82)) * 0.02).to(BF16).to(DEV)
    fa = K.premap_fwd(x, W, *_dev(p32))
    fb = K.premap_fwd(x, W, *_dev(p16))
    assert all(torch.equal(u, v) for u, v in zip(fa, fb))
    li, H, hq, hp, pj, inv = fa
    g_li = torch.randn(T, 256, generator=torch.Generator().manual_seed(83)).to(BF16).to(DEV)
    ba = K.premap_bwd(x, W, *_dev(p32), hp, pj, inv, g_li, *_dev(grads[1:]))
    bb = K.premap_bwd(x, W, *_dev(p16), hp, pj, inv, g_li, *_dev(grads[1:]))
    assert torch.equal(ba[0], bb[0]) and torch.equal(ba[1], bb[1])
    for u, v in zip(ba[2:], bb[2:]):
        assert v.dtype == BF16 and torch.equal(u, v.float())


@pytest.mark.parametrize("n", [2048, 8192])
def test_k2_fwd_small_and_large_kernels_agree(n):
    """Up to 2048 tokens the forward gives each token 32 lanes (one per logit),
    beyond that four; both keep the same operation order, so the first n
    tokens of an (n + 1)-token call equal an n-token call bit for bit (n = 2048:
    the two kernels; 8192: four lanes both)."""
    proj, alphas, bias, _ = _case(n + 1, 90)
    prm = _dev([*alphas, bias, PERM])
    big = K.k2_fwd(proj.to(DEV), *prm)
    small = K.k2_fwd(proj[:n].to(DEV), *prm)
    for u, v in zip(small, big):
        assert torch.equal(u, v[:n])


@pytest.mark.parametrize("n", [6144, 8192])
def test_k2_bwd_small_and_large_kernels_agree(n):
    """The backward likewise: 32 lanes per token up to 6144 tokens, four lanes
    per token beyond, with the same per-token operation order, so grad_proj of
    the first n tokens of an (n + 1)-token call equals an n-token call bit for
    bit (the parameter gradients add the tokens in a different, fixed, order)."""
    proj, alphas, bias, grads = _case(n + 1, 91)
    prm = _dev([*alphas, bias, PERM])
    g = _dev(list(grads))
    big = K.k2_bwd(proj.to(DEV), *prm, *g)
    small = K.k2_bwd(proj[:n].to(DEV), *prm, *[t[:n] for t in g])
    assert torch.equal(small[0], big[0][:n])
