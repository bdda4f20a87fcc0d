"""The kernels at the largest configuration, T = 262144 tokens, n = 4,
C = 4096 (the training-scale stack's shape: x is 8.6 GB, 2^32 elements), where
every byte offset past 2^31 and 2^32 is exercised.

* K1 forward, backward dx and the fused backward, K3 and K4 forward and
  backward: per-token outputs on sampled tokens (random ones, the tokens
  either side of the 2^31-, 2^32- and 3 * 2^31-byte offsets of x and the last
  tokens) against the oracle, to its usual bounds; K1's grad_W, a sum over all
  tokens, against a float64 reference of the same formula computed on the GPU
  in chunks of tokens.
* The pre-map forward (one kernel at this size) against K1, K2 and K3 run
  separately, and the pre-map backward against the same composition of
  kernels, bit for bit on every token.
"""

from __future__ import annotations

import pytest
import torch

from flash_mhc import build_permutation_matrices
from flash_mhc import kernels as K
from oracle import mhc_oracle as O
from parity import check_bf16, check_fp32, check_rel

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16 = torch.bfloat16
T, C = 262144, 4096
NC = 4 * C


def _randn(shape, gen, scale=1.0, dtype=BF16):
    return (torch.randn(shape, device=DEV, generator=gen) * scale).to(dtype)


@pytest.fixture(scope="module")
def big():
    gen = torch.Generator(device=DEV).manual_seed(2024)
    x = _randn((T, 4, C), gen)
    W = _randn((32, NC), gen, 0.02)
    params = [torch.tensor([0.8], device=DEV), torch.tensor([1.2], device=DEV), torch.tensor([1.7], device=DEV),
              torch.randn(32, device=DEV, generator=gen) * 0.5, build_permutation_matrices(4)[0].to(DEV)]
    g = torch.Generator().manual_seed(7)
    row = T * NC * 2 // T  # bytes per token row of x
    edges = [(1 << 31) // row, (1 << 32) // row, 3 * (1 << 31) // row]
    idx = torch.cat([torch.randperm(T, generator=g)[:384]] + [torch.arange(e - 8, e + 8) for e in edges]
                    + [torch.arange(T - 32, T)]).unique()
    yield {"x": x, "W": W, "params": params, "gen": gen, "idx": idx}
    torch.cuda.empty_cache()


def _grad_W_reference(go, x_flat, inv):
    """R and S of bf16(go * inv)^T @ x (ops.py:683-684 of the reference) in
    float64 on the GPU, 16384 tokens at a time."""
    G = (go.float() * inv[:, None]).to(BF16).double()
    R = torch.zeros(32, NC, dtype=torch.float64, device=DEV)
    S = torch.zeros_like(R)
    for t0 in range(0, T, 16384):
        xs = x_flat[t0:t0 + 16384].double()
        g = G[t0:t0 + 16384]
        R += g.t() @ xs
        S += g.abs().t() @ xs.abs()
        del xs
    return R.cpu(), S.cpu()


@pytest.mark.timeout(600)
def test_kernels_sampled_at_largest(big):
    x, W, gen, idx = big["x"], big["W"], big["gen"], big["idx"]
    i = idx.to(DEV)
    xf = x.view(T, NC)
    xs = x[i].cpu()
    proj, inv = K.k1_fwd(xf, W)
    R, S, invR = O.k1_fwd(xs.view(-1, NC), W.cpu())
    check_bf16("k1 proj @largest", proj[i], R, S, NC)
    check_rel("k1 inv_rms @largest", inv[i], invR, rtol=1e-5)

    go1 = _randn((T, 32), gen)
    gx = K.k1_bwd_dx(go1, xf, W, proj, inv)
    R, S = O.k1_bwd_dx(go1[i].cpu(), xs.view(-1, NC), W.cpu(), proj[i].cpu(), inv[i].cpu())
    check_bf16("k1 grad_x @largest", gx[i], R, S, 64)
    gx2, gW = K.k1_bwd(go1, xf, W, proj, inv)
    assert torch.equal(gx2, gx)  # the fused kernel's grad_x is the dx kernel's
    del gx, gx2
    R, S = _grad_W_reference(go1, xf, inv)
    check_bf16("k1 grad_W @largest", gW, R, S, T)

    hpre = torch.rand(T, 4, device=DEV, generator=gen)
    out3 = K.k3_fwd(x, hpre)
    R, S = O.k3_fwd(xs, hpre[i].cpu())
    check_bf16("k3 out @largest", out3[i], R, S, 4)
    del out3
    go3 = _randn((T, C), gen)
    gx3, gh3 = K.k3_bwd(go3, x, hpre)
    gxR, gxS, ghR, ghS = O.k3_bwd(go3[i].cpu(), xs, hpre[i].cpu())
    check_bf16("k3 grad_x @largest", gx3[i], gxR, gxS, 1)
    check_fp32("k3 grad_h_pre @largest", gh3[i], ghR, ghS, C)
    del gx3, gh3, go3

    lo = _randn((T, C), gen)
    H = torch.randn(T, 4, 4, device=DEV, generator=gen)
    hp = torch.rand(T, 4, device=DEV, generator=gen)
    out4 = K.k4_fwd(x, lo, H, hp)
    R, S = O.k4_fwd(xs, lo[i].cpu(), H[i].cpu(), hp[i].cpu())
    check_bf16("k4 out @largest", out4[i], R, S, 5)
    del out4
    go4 = _randn((T, 4, C), gen)
    gx4, glo4, gH4, ghp4 = K.k4_bwd(go4, x, lo, H, hp)
    ref = O.k4_bwd(go4[i].cpu(), xs, lo[i].cpu(), H[i].cpu(), hp[i].cpu())
    check_bf16("k4 grad_x @largest", gx4[i], *ref["grad_x"], 4)
    check_bf16("k4 grad_lo @largest", glo4[i], *ref["grad_lo"], 4)
    check_fp32("k4 grad_H @largest", gH4[i], *ref["grad_H"], C)
    check_fp32("k4 grad_hp @largest", ghp4[i], *ref["grad_hp"], C)


@pytest.mark.timeout(600)
def test_premap_at_largest_equals_kernels(big):
    x, W, p, gen = big["x"], big["W"], big["params"], big["gen"]
    li, H, hq, hp, proj, inv = K.premap_fwd(x, W, *p)
    proj1, inv1 = K.k1_fwd(x.view(T, NC), W)
    assert torch.equal(proj, proj1) and torch.equal(inv, inv1)
    hp2, hq2, H2 = K.k2_fwd(proj1, *p)
    assert torch.equal(hp, hp2) and torch.equal(hq, hq2) and torch.equal(H, H2)
    assert torch.equal(li, K.k3_fwd(x, hp2))
    del li, proj1, inv1, hp2, hq2, H2

    g_li = _randn((T, C), gen)
    g_hq = torch.randn(T, 4, device=DEV, generator=gen)
    g_H = torch.randn(T, 4, 4, device=DEV, generator=gen)
    g_in = _randn((T, 4, C), gen)
    gx, gW, ga1, ga2, ga3, gb = K.premap_bwd(x, W, *p, hp, proj, inv, g_li, g_hq, g_H, g_in)
    # The same gradients from the separate kernels: K3's, K2's and K1's
    # backward, and the two bf16 sums autograd would form.
    gx3, gh = K.k3_bwd(g_li, x, hp)
    gp, ra1, ra2, ra3, rb = K.k2_bwd(proj, *p, gh, g_hq, g_H)
    dx, gW1 = K.k1_bwd(gp, x.view(T, NC), W, proj, inv)
    assert torch.equal(gW, gW1)
    for name, a, b in (("alpha_pre", ga1, ra1), ("alpha_post", ga2, ra2), ("alpha_res", ga3, ra3), ("bias", gb, rb)):
        assert torch.equal(a, b), name
    dx = dx.view(T, 4, C)
    for t0 in range(0, T, 16384):
        s = slice(t0, t0 + 16384)
        want = (g_in[s].float() + (gx3[s].float() + dx[s].float()).to(BF16).float()).to(BF16)
        assert torch.equal(gx[s], want), f"pre-map grad_x differs in tokens {t0}..{t0 + 16383}"
