"""Seeded random shapes through every kernel and the pre-map entry points.

Each case draws T (1 ... 70000) and C (multiples of 8 up to 4104, and ragged
widths that force the element-wise paths), scales every (T // 37)-th token by 50,
and may move operands 2 or 4 bytes off 16-byte alignment (the element-wise
fallbacks).  Per-token outputs of K1, K3 and K4 forward and backward are
checked on sampled tokens (random ones and the last 17) against the oracle;
K1's grad_W against the oracle where T allows; the pre-map forward against
K1 -> K2 -> K3 bit for bit, and the pre-map backward against the composition
of the separate backward kernels (bit for bit on the vector paths, to the bf16
chain bound where the element-wise paths sum in another order).
"""

from __future__ import annotations

import random

import pytest
import torch

from flash_mhc import build_permutation_matrices
from flash_mhc import kernels as K
from oracle import mhc_oracle as O
from parity import check_bf16, check_chain, check_fp32, check_rel

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16 = torch.bfloat16
N_CASES = 24


def _case(k: int):
    rng = random.Random(1000 + k)
    C = rng.choice([rng.randrange(8, 4097, 8), rng.randrange(1, 600),
                    rng.choice([8, 16, 64, 128, 256, 512, 1024, 2048, 4096, 4104])])
    T = rng.choice([rng.randrange(1, 70), rng.randrange(70, 3000), rng.randrange(3000, 70000)])
    if T * C > 40_000_000:
        T = max(1, 40_000_000 // C)
    return rng, T, C, rng.random() < 0.35


@pytest.mark.parametrize("k", range(N_CASES))
def test_random_shape(k):
    rng, T, C, misalign = _case(k)
    nC = 4 * C
    print(f"[random-shape] case {k}: T={T} C={C} misaligned={misalign}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(k)

    def rn(shape, scale=1.0):
        t = (torch.randn(shape, device=DEV, generator=g) * scale).to(BF16)
        if misalign and rng.random() < 0.5:
            buf = torch.empty(t.numel() + 8, device=DEV, dtype=BF16)
            view = buf[1:1 + t.numel()].view(t.shape)
            view.copy_(t)
            return view
        return t

    x = rn((T, 4, C))
    x[:: max(1, T // 37)] *= 50
    W = rn((32, nC), 0.02)
    p = [torch.tensor([0.8], device=DEV), torch.tensor([1.2], device=DEV), torch.tensor([1.7], device=DEV),
         torch.randn(32, device=DEV, generator=g) * 0.5, build_permutation_matrices(4)[0].to(DEV)]
    cg = torch.Generator().manual_seed(k)
    idx = torch.cat([torch.randint(0, T, (48,), generator=cg), torch.arange(max(0, T - 17), T)]).unique()
    i = idx.to(DEV)
    xs = x[i].cpu()

    proj, inv = K.k1_fwd(x.view(T, nC), W)
    R, S, invR = O.k1_fwd(xs.view(-1, nC), W.cpu())
    check_bf16("k1 proj", proj[i], R, S, nC)
    check_rel("k1 inv_rms", inv[i], invR, rtol=4 * nC ** 0.5 * 2.0**-24 + 4 * 2.0**-24)
    go1 = rn((T, 32))
    gx, gW = K.k1_bwd(go1, x.view(T, nC), W, proj, inv)
    R, S = O.k1_bwd_dx(go1[i].cpu(), xs.view(-1, nC), W.cpu(), proj[i].cpu(), inv[i].cpu())
    check_bf16("k1 grad_x", gx[i], R, S, 64)
    if T <= 20000:
        R, S = O.k1_grad_W(go1.cpu(), x.view(T, nC).cpu(), inv.cpu())
        check_bf16("k1 grad_W", gW, R, S, T)

    h = torch.rand(T, 4, device=DEV, generator=g)
    out3 = K.k3_fwd(x, h)
    R, S = O.k3_fwd(xs, h[i].cpu())
    check_bf16("k3 out", out3[i], R, S, 4)
    go3 = rn((T, C))
    gx3, gh3 = K.k3_bwd(go3, x, h)
    gxR, gxS, ghR, ghS = O.k3_bwd(go3[i].cpu(), xs, h[i].cpu())
    check_bf16("k3 grad_x", gx3[i], gxR, gxS, 1)
    check_fp32("k3 grad_h_pre", gh3[i], ghR, ghS, C)

    lo = rn((T, C))
    H = torch.randn(T, 4, 4, device=DEV, generator=g)
    hp = torch.rand(T, 4, device=DEV, generator=g)
    out4 = K.k4_fwd(x, lo, H, hp)
    R, S = O.k4_fwd(xs, lo[i].cpu(), H[i].cpu(), hp[i].cpu())
    check_bf16("k4 out", out4[i], R, S, 5)
    go4 = rn((T, 4, C))
    gx4, glo, gH, ghp = K.k4_bwd(go4, x, lo, H, hp)
    ref = O.k4_bwd(go4[i].cpu(), xs, lo[i].cpu(), H[i].cpu(), hp[i].cpu())
    check_bf16("k4 grad_x", gx4[i], *ref["grad_x"], 4)
    check_bf16("k4 grad_lo", glo[i], *ref["grad_lo"], 4)
    check_fp32("k4 grad_H", gH[i], *ref["grad_H"], C)
    check_fp32("k4 grad_hp", ghp[i], *ref["grad_hp"], C)

    li, Hm, hq, hpre, pj, iv = K.premap_fwd(x, W, *p)
    hp1, hq1, H1 = K.k2_fwd(pj, *p)
    assert torch.equal(hpre, hp1) and torch.equal(hq, hq1) and torch.equal(Hm, H1), "pre-map K2 outputs"
    assert torch.equal(li, K.k3_fwd(x, hp1)), "pre-map layer input"
    g_in = rn((T, 4, C))
    gxp, gWp, *pg = K.premap_bwd(x, W, *p, hpre, pj, iv, go3, hq, Hm, g_in)
    gx3b, gh = K.k3_bwd(go3, x, hpre)
    gp, *rpg = K.k2_bwd(pj, *p, gh, hq, Hm)
    dx, gW1 = K.k1_bwd(gp, x.view(T, nC), W, pj, iv)
    want = (g_in.float() + (gx3b.float() + dx.view(T, 4, C).float()).to(BF16).float()).to(BF16)
    for a, b in zip(pg, rpg):
        assert torch.equal(a, b), "pre-map parameter gradients"
    if C % 8 == 0 and not misalign:
        assert torch.equal(gWp, gW1), "pre-map grad_W"
        assert torch.equal(gxp, want), "pre-map grad_x"
    else:
        check_chain("pre-map grad_W (element-wise)", gWp.float().t(), gW1.float().t(), max_rate=1.0)
        check_chain("pre-map grad_x (element-wise)", gxp.float().reshape(T, -1), want.float().reshape(T, -1),
                    max_rate=1.0)
