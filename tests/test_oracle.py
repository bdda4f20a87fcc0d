"""Pins for the CPU oracle (oracle/mhc_oracle.py).

Each vectorised oracle formula is checked against something independent of
its own text: pure-Python loops on tiny shapes, float64 autograd of the
forward formula (so the hand-derived backward formulas are tested by
differentiation, not by retyping them), closed forms, textbook routines
(F.rms_norm) and structural invariants.  A planted mistake in the oracle must
make the GPU parity rule fail (test_parity_rule_catches_planted_mistakes).
"""

from __future__ import annotations

import itertools
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import k2_oracle as K2O
from oracle import mhc_oracle as O
from parity import bf16_ulp, check_bf16, check_chain, check_fp32

F64 = torch.float64


def rnd(shape, seed, scale=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


# ---------------------------------------------------------------------------
# permutation matrices


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5])
def test_permutation_matrices(n):
    P, idx = O.permutation_matrices(n)
    assert P.shape == (math.factorial(n), n * n) and idx == 0
    mats = P.view(-1, n, n)
    assert torch.equal(mats[0], torch.eye(n))
    assert torch.equal(mats.sum(1), torch.ones(mats.shape[0], n))
    assert torch.equal(mats.sum(2), torch.ones(mats.shape[0], n))
    # row m applied to a vector permutes it exactly as itertools' m-th permutation
    v = torch.arange(n, dtype=torch.float32)
    for m, p in enumerate(itertools.permutations(range(n))):
        assert torch.equal(mats[m] @ v, torch.tensor(p, dtype=torch.float32))
    assert len({tuple(r.tolist()) for r in P}) == P.shape[0]


def test_package_permutations_equal_oracle():
    from flash_mhc import build_permutation_matrices

    for n in range(1, 6):
        a, ia = build_permutation_matrices(n)
        b, ib = O.permutation_matrices(n)
        assert torch.equal(a, b) and ia == ib


# ---------------------------------------------------------------------------
# K1


def test_k1_fwd_loops():
    x, W = rnd((3, 16), 1), rnd((5, 16), 2)
    R, S, inv = O.k1_fwd(x, W)
    Rl, invl = O.k1_fwd_loops(x, W)
    torch.testing.assert_close(R, Rl, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(inv, invl, rtol=1e-12, atol=1e-12)
    assert torch.all(S >= R.abs())


def test_k1_fwd_is_rmsnorm_then_linear():
    x, W = rnd((64, 512), 3), rnd((32, 512), 4, 0.02)
    R, _, _ = O.k1_fwd(x, W)
    ref = F.rms_norm(x.double(), (512,), eps=1e-6) @ W.double().T
    torch.testing.assert_close(R, ref, rtol=1e-10, atol=1e-12)


def test_k1_fwd_closed_forms():
    nC = 64
    # selector rows: W[d] = e_{k_d}  ->  proj[:, d] = x[:, k_d] * inv_rms
    ks = torch.arange(32) * 2
    W = torch.zeros(32, nC)
    W[torch.arange(32), ks] = 1.0
    x = rnd((8, nC), 5)
    R, _, inv = O.k1_fwd(x, W.to(torch.bfloat16))
    torch.testing.assert_close(R, x.double()[:, ks] * inv[:, None], rtol=1e-12, atol=1e-14)
    # constant rows x = a * 1  ->  inv_rms = 1 / sqrt(a^2 + 1e-6)
    a = torch.tensor([0.5, 1.0, 2.0, 3.0])
    xc = (a[:, None] * torch.ones(4, nC)).to(torch.bfloat16)
    _, _, inv = O.k1_fwd(xc, W.to(torch.bfloat16))
    torch.testing.assert_close(inv, 1.0 / torch.sqrt(a.double() ** 2 + 1e-6), rtol=1e-12, atol=0)
    # scale invariance (eps negligible for |x| ~ 1)
    x = rnd((8, nC), 6, dtype=F64)
    R1, _, _ = O.k1_fwd(x, W)
    R2, _, _ = O.k1_fwd(4.0 * x, W)
    torch.testing.assert_close(R1, R2, rtol=1e-5, atol=1e-7)


def test_k1_bwd_dx_is_autograd():
    T, nC = 6, 32
    x = rnd((T, nC), 7, dtype=F64).requires_grad_(True)
    W = rnd((32, nC), 8, 0.1, dtype=F64)
    go = rnd((T, 32), 9, dtype=F64)
    proj = O.k1_torch(x, W)
    (gx_auto,) = torch.autograd.grad(proj, x, go)
    _, _, inv = O.k1_fwd(x.detach(), W)
    gx, _ = O.k1_bwd_dx(go, x.detach(), W, proj.detach(), inv)
    torch.testing.assert_close(gx, gx_auto, rtol=1e-10, atol=1e-12)
    assert torch.autograd.gradcheck(lambda t: O.k1_torch(t, W), (x,))


def test_k1_grad_W_formula():
    # With inv_rms a power of two and bf16 upstream grads, bf16(go * inv) is
    # exact, so the rule equals plain autograd of proj wrt W at fixed inv_rms.
    T, nC = 10, 48
    x = rnd((T, nC), 10)
    go = rnd((T, 32), 11)
    inv = torch.full((T,), 0.5)
    W = rnd((32, nC), 12, dtype=F64).requires_grad_(True)
    proj = (x.double() @ W.T) * inv.double()[:, None]
    (gW_auto,) = torch.autograd.grad(proj, W, go.double())
    gW, S = O.k1_grad_W(go, x, inv)
    torch.testing.assert_close(gW, gW_auto, rtol=1e-12, atol=1e-12)
    # and the rounding of go * inv to bf16 is applied (ops.py:683)
    inv2 = torch.full((T,), 1.0 / 3.0)
    gW2, _ = O.k1_grad_W(go, x, inv2)
    manual = (go.float() * inv2[:, None]).to(torch.bfloat16).double().T @ x.double()
    torch.testing.assert_close(gW2, manual, rtol=0, atol=0)


# ---------------------------------------------------------------------------
# K3 / K4


def test_k3_loops_and_closed_forms():
    x = rnd((3, 4, 8), 20)
    h = rnd((3, 4), 21, dtype=torch.float32)
    R, S = O.k3_fwd(x, h)
    torch.testing.assert_close(R, O.k3_fwd_loops(x, h), rtol=1e-12, atol=1e-12)
    assert torch.all(S >= R.abs())
    for j in range(4):  # one-hot h_pre selects stream j
        e = torch.zeros(3, 4)
        e[:, j] = 1.0
        Rj, _ = O.k3_fwd(x, e)
        assert torch.equal(Rj, x[:, j].double())


def test_k3_bwd_is_autograd():
    x = rnd((4, 4, 6), 22, dtype=F64).requires_grad_(True)
    h = rnd((4, 4), 23, dtype=F64).requires_grad_(True)
    go = rnd((4, 6), 24, dtype=F64)
    gx_a, gh_a = torch.autograd.grad(O.k3_torch(x, h), (x, h), go)
    gx, _, gh, _ = O.k3_bwd(go, x.detach(), h.detach())
    torch.testing.assert_close(gx, gx_a, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(gh, gh_a, rtol=1e-12, atol=1e-12)
    assert torch.autograd.gradcheck(O.k3_torch, (x, h))


def test_k4_loops_and_closed_forms():
    T, C = 3, 8
    x = rnd((T, 4, C), 30)
    lo = rnd((T, C), 31)
    H = rnd((T, 4, 4), 32, dtype=torch.float32)
    hp = rnd((T, 4), 33, dtype=torch.float32)
    R, S = O.k4_fwd(x, lo, H, hp)
    torch.testing.assert_close(R, O.k4_fwd_loops(x, lo, H, hp), rtol=1e-12, atol=1e-12)
    assert torch.all(S >= R.abs())
    # H = I, h_post = 0: identity
    I = torch.eye(4).expand(T, 4, 4).contiguous()
    R, _ = O.k4_fwd(x, lo, I, torch.zeros(T, 4))
    assert torch.equal(R, x.double())
    # H = a permutation matrix: streams permuted; h_post adds lo
    P = O.permutation_matrices(4)[0][7].view(4, 4)
    R, _ = O.k4_fwd(x, lo, P.expand(T, 4, 4).contiguous(), torch.ones(T, 4))
    expect = (P.double() @ x.double()) + lo.double()[:, None, :]
    torch.testing.assert_close(R, expect, rtol=0, atol=1e-12)


def test_k4_bwd_is_autograd_and_loops():
    T, C = 3, 5
    x = rnd((T, 4, C), 34, dtype=F64).requires_grad_(True)
    lo = rnd((T, C), 35, dtype=F64).requires_grad_(True)
    H = rnd((T, 4, 4), 36, dtype=F64).requires_grad_(True)
    hp = rnd((T, 4), 37, dtype=F64).requires_grad_(True)
    go = rnd((T, 4, C), 38, dtype=F64)
    grads = torch.autograd.grad(O.k4_torch(x, lo, H, hp), (x, lo, H, hp), go)
    ref = O.k4_bwd(go, x.detach(), lo.detach(), H.detach(), hp.detach())
    loops = O.k4_bwd_loops(go, x.detach(), lo.detach(), H.detach(), hp.detach())
    for name, g in zip(("grad_x", "grad_lo", "grad_H", "grad_hp"), grads):
        torch.testing.assert_close(ref[name][0], g, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(ref[name][0], loops[name], rtol=1e-12, atol=1e-12)
    assert torch.autograd.gradcheck(O.k4_torch, (x, lo, H, hp))


# ---------------------------------------------------------------------------
# K2 + block


def _params(n, C, seed):
    g = torch.Generator().manual_seed(seed)
    nf = math.factorial(n)
    return {
        "W": torch.randn(2 * n + nf, n * C, generator=g, dtype=F64) * 0.05,
        "b": torch.randn(2 * n + nf, generator=g, dtype=F64) * 0.1,
        "alpha_pre": torch.tensor([0.7], dtype=F64),
        "alpha_post": torch.tensor([0.4], dtype=F64),
        "alpha_res": torch.tensor([0.9], dtype=F64),
        "perm": O.permutation_matrices(n)[0].double(),
    }


def test_coefficients_invariants():
    n, T = 4, 16
    p = _params(n, 8, 40)
    proj = torch.randn(T, 2 * n + 24, generator=torch.Generator().manual_seed(41), dtype=F64)
    h_pre, h_post, H_merged, H_res = O.coefficients(
        proj, p["b"], p["alpha_pre"], p["alpha_post"], p["alpha_res"], p["perm"], n)
    assert torch.all((h_pre > 0) & (h_pre < 1)) and torch.all((h_post > 0) & (h_post < 2))
    # Birkhoff-von Neumann: a convex combination of permutations is doubly stochastic
    torch.testing.assert_close(H_res.sum(-1), torch.ones(T, n, dtype=F64))
    torch.testing.assert_close(H_res.sum(-2), torch.ones(T, n, dtype=F64))
    torch.testing.assert_close(H_merged, H_res - h_post[..., :, None] * h_pre[..., None, :])
    # H_res = a @ P with a = softmax(alpha_res * r + b): closed form per token
    a = torch.softmax(p["alpha_res"] * proj[:, 8:] + p["b"][8:], -1)
    torch.testing.assert_close(H_res, (a[:, :, None, None] * p["perm"].view(24, n, n)).sum(1))


def test_block_identity_and_gradcheck():
    n, C, T = 4, 4, 3
    p = _params(n, C, 50)
    lin = torch.nn.Linear(C, C, bias=False).double()
    x = torch.randn(T, n, C, generator=torch.Generator().manual_seed(51), dtype=F64).requires_grad_(True)
    out = O.block_forward(x, p, lin, n)
    # out = H_res x + h_post (layer(h_pre^T x) - h_pre^T x)
    xf = x.detach().reshape(T, n * C)
    proj = F.rms_norm(xf, (n * C,)) @ p["W"].T
    h_pre, h_post, _, H_res = O.coefficients(
        proj, p["b"], p["alpha_pre"], p["alpha_post"], p["alpha_res"], p["perm"], n)
    li = (h_pre[:, :, None] * x.detach()).sum(1)
    expect = H_res @ x.detach() + h_post[:, :, None] * (lin(li) - li)[:, None, :]
    torch.testing.assert_close(out.detach(), expect, rtol=1e-12, atol=1e-12)
    assert torch.autograd.gradcheck(lambda t: O.block_forward(t, p, lin, n), (x,))


# ---------------------------------------------------------------------------
# The parity rule itself


def test_bf16_ulp():
    R = torch.tensor([1.0, 1.5, 2.0, 0.75, -3.0, 1e-3], dtype=F64)
    expect = torch.tensor([2**-7, 2**-7, 2**-6, 2**-8, 2**-6, 2.0 ** (-10 - 7)], dtype=F64)
    torch.testing.assert_close(bf16_ulp(R), expect, rtol=0, atol=0)


def test_parity_rule_accepts_rounded_reference():
    x = rnd((64, 4, 256), 60)
    lo = rnd((64, 256), 61)
    H = rnd((64, 4, 4), 62, dtype=torch.float32)
    hp = rnd((64, 4), 63, dtype=torch.float32)
    R, S = O.k4_fwd(x, lo, H, hp)
    f32 = O.k4_torch(x.float(), lo.float(), H, hp)  # fp32 evaluation, another order
    check_bf16("fp32 rounded", f32.to(torch.bfloat16), R, S, 5)
    go = rnd((64, 4, 256), 64)
    ref = O.k4_bwd(go, x, lo, H, hp)
    gH32 = torch.matmul(go.float(), x.float().transpose(1, 2))
    check_fp32("fp32 grad_H", gH32, *ref["grad_H"], 256)


def test_parity_rule_catches_planted_mistakes():
    """Plausible kernel mistakes, planted in the oracle's output, must fail."""
    x = rnd((64, 4, 256), 70)
    lo = rnd((64, 256), 71)
    H = rnd((64, 4, 4), 72, dtype=torch.float32)
    hp = rnd((64, 4), 73, dtype=torch.float32)
    R, S = O.k4_fwd(x, lo, H, hp)
    # dropped j = 3 term
    dropped = R - (H.double()[:, :, 3:4] * x.double()[:, None, 3, :])
    with pytest.raises(AssertionError):
        check_bf16("dropped term", dropped.to(torch.bfloat16), R, S, 5)
    # transposed H
    Rt, _ = O.k4_fwd(x, lo, H.transpose(1, 2).contiguous(), hp)
    with pytest.raises(AssertionError):
        check_bf16("transposed H", Rt.to(torch.bfloat16), R, S, 5)
    # wrong sign of the h_post term
    Rs, _ = O.k4_fwd(x, lo, H, -hp)
    with pytest.raises(AssertionError):
        check_bf16("sign", Rs.to(torch.bfloat16), R, S, 5)
    # K1: eps dropped / wrong normaliser (nC vs C)
    xk, Wk = rnd((32, 1024), 74), rnd((32, 1024), 75, 0.02)
    Rk, Sk, _ = O.k1_fwd(xk, Wk)
    wrong = Rk * 2.0  # mean over C instead of nC scales by sqrt(4)
    with pytest.raises(AssertionError):
        check_bf16("normaliser", wrong.to(torch.bfloat16), Rk, Sk, 1024)
    # one k-chunk (8 terms) of the contraction dropped
    part = (xk.double()[:, 8:16] @ Wk.double()[:, 8:16].T) * O.k1_fwd(xk, Wk)[2][:, None]
    with pytest.raises(AssertionError):
        check_bf16("dropped chunk", (Rk - part).to(torch.bfloat16), Rk, Sk, 1024)
    # off-by-one stream index in K3
    h = rnd((64, 4), 76, dtype=torch.float32)
    R3, S3 = O.k3_fwd(x, h)
    R3b, _ = O.k3_fwd(x.roll(1, dims=1), h)
    with pytest.raises(AssertionError):
        check_bf16("stream index", R3b.to(torch.bfloat16), R3, S3, 4)


# ---------------------------------------------------------------------------
# K2 coefficient chain with bf16 rounding points (oracle/k2_oracle.py), pinned
# against torch's own bf16 CPU forward + autograd through the reference's op
# sequence (mhc_oracle.coefficients, i.e. block.py:161-170 + the .float()
# casts of block.py:176-177).  The GPU rounding of the sigmoid / softmax
# backward steps is pinned against torch's GPU ops in tests/test_gpu_k2.py.


def test_k2_rounding_variants_differ_only_in_two_steps():
    """The GPU and CPU variants of the two backward steps: identical on values
    that need no intermediate rounding, different (and each within 2 ulps of
    the other) in general."""
    g = torch.Generator().manual_seed(9)
    y = torch.rand(4096, 24, generator=g).to(torch.bfloat16).float().numpy()
    gr = torch.randn(4096, 24, generator=g).to(torch.bfloat16).float().numpy()
    for fn in (K2O.sigmoid_bwd, K2O.softmax_bwd):
        a, b = fn(gr, y, "gpu"), fn(gr, y, "cpu")
        assert (a != b).mean() > 0.05
        check_chain(fn.__name__ + " gpu vs cpu", a, b, max_rate=1.0)
    half = 0.5 * torch.ones(8, 4).numpy()
    ones = torch.ones(8, 4).numpy()
    assert (K2O.sigmoid_bwd(ones, half, "gpu") == 0.25).all() and (K2O.sigmoid_bwd(ones, half, "cpu") == 0.25).all()


def _k2_case(T, seed, proj_scale=3.0):
    g = torch.Generator().manual_seed(seed)
    proj = (torch.randn(T, 32, generator=g) * proj_scale).to(torch.bfloat16)
    bias = torch.randn(32, generator=g) * 0.5
    alphas = [torch.tensor([v]) for v in (0.9, 1.3, 2.1)]
    gh = [torch.randn(T, 4, generator=g), torch.randn(T, 4, generator=g), torch.randn(T, 4, 4, generator=g)]
    return proj, alphas, bias, gh


def _k2_torch_cpu(proj, alphas, bias, perm, gh):
    """The reference's chain on CPU in bf16, with torch autograd."""
    p = proj.clone().requires_grad_(True)
    a = [x.clone().requires_grad_(True) for x in alphas]
    b = bias.clone().requires_grad_(True)
    h_pre, h_post, H, _ = O.coefficients(p, b, a[0], a[1], a[2], perm, 4)
    outs = (h_pre.float(), h_post.float(), H.float())
    loss = sum((o * g).sum() for o, g in zip(outs, gh))
    loss.backward()
    return outs, p.grad, [x.grad for x in a], b.grad


@pytest.mark.parametrize("seed", [0, 1])
def test_k2_chain_matches_torch_bf16_autograd(seed):
    T = 4096
    proj, alphas, bias, gh = _k2_case(T, seed)
    perm, _ = O.permutation_matrices(4)
    outs, gproj, galpha, gbias = _k2_torch_cpu(proj, alphas, bias, perm, gh)
    f = K2O.k2_fwd(proj, *alphas, bias, perm)
    check_chain("k2 h_pre", f["h_pre"], outs[0])
    check_chain("k2 h_post", f["h_post"], outs[1])
    check_chain("k2 H_merged", f["H_merged"], outs[2])
    b = K2O.k2_bwd(proj, *alphas, bias, perm, *gh, rounding="cpu")  # torch's CPU kernels
    check_chain("k2 grad_proj", b["grad_proj"], gproj)
    for name, got in zip(("grad_alpha_pre", "grad_alpha_post", "grad_alpha_res"), galpha):
        R, S = b[name]
        check_bf16(name, got.to(torch.bfloat16), torch.tensor([R], dtype=F64), torch.tensor([S], dtype=F64), 24 * T)
    R, S = b["grad_bias"]
    check_bf16("grad_bias", gbias.to(torch.bfloat16), torch.as_tensor(R), torch.as_tensor(S), T)


def test_k2_chain_closed_forms():
    """Saturated logits: h_pre, h_post reach their limits and the softmax puts
    all weight on one permutation, so H_res is that permutation matrix."""
    T = 24
    perm, _ = O.permutation_matrices(4)
    proj = torch.zeros(T, 32)
    proj[:, :4] = 200.0  # exp(-200) and exp(-200 - 0) underflow in fp32
    proj[:, 4:8] = -200.0
    for t in range(T):
        proj[t, 8 + t] = 200.0
    f = K2O.k2_fwd(proj.to(torch.bfloat16), torch.tensor([1.0]), torch.tensor([1.0]), torch.tensor([1.0]),
                   torch.zeros(32), perm)
    assert (f["h_pre"] == 1.0).all() and (f["h_post"] == 0.0).all()
    assert torch.equal(torch.from_numpy(f["H_res"]), perm)
    assert torch.equal(torch.from_numpy(f["H_merged"]).reshape(T, 16), perm)


@pytest.mark.parametrize("plant", ["no_round_scale", "transpose_perm", "sigmoid_derivative"])
def test_k2_chain_catches_planted_mistakes(plant):
    T = 4096
    proj, alphas, bias, gh = _k2_case(T, 3)
    perm, _ = O.permutation_matrices(4)
    outs, gproj, _, _ = _k2_torch_cpu(proj, alphas, bias, perm, gh)
    with pytest.raises(AssertionError):
        if plant == "sigmoid_derivative":
            check_chain("planted", K2O.k2_bwd(proj, *alphas, bias, perm, *gh, rounding="cpu", _plant=plant)["grad_proj"], gproj)
        else:
            f = K2O.k2_fwd(proj, *alphas, bias, perm, _plant=plant)
            check_chain("planted h_pre", f["h_pre"], outs[0])
            check_chain("planted H", f["H_merged"], outs[2])
