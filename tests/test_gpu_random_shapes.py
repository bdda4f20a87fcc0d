"""Seeded random (T, C) for the six kernels against the float64 oracle.

The fixed shapes of test_gpu_kernels.py pick out the edges of each launch
policy (column split, 32- / 64-token tiles, backward run counts, lanes per
token, element-wise paths).  These draws add shapes nobody picked: token
counts around powers of two and tile sizes, widths with and without
C % 8 == 0, so that a policy boundary nobody thought of is still crossed.
Same tolerances as the fixed-shape tests (tests/parity.py).
"""

from __future__ import annotations

import random

import pytest
import torch

from flash_mhc import kernels as K
from oracle import mhc_oracle as O
from parity import check_bf16, check_fp32, check_rel

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16 = torch.bfloat16

_T = [1, 2, 3, 7, 15, 16, 17, 31, 33, 63, 65, 127, 129, 255, 257, 511, 513, 1023, 1025, 2047, 2049, 3000,
      4095, 4097]
_C = [8, 16, 24, 25, 40, 64, 72, 100, 120, 128, 136, 256, 264, 300, 504, 512, 520, 1000, 1001, 1016, 1024,
      1032, 2040, 2048, 2050, 4096]


def _draws(n=16, seed=20261201, max_elems=1 << 22):
    """C first, then a token count that keeps T x C within the oracle's budget."""
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        C = rng.choice(_C)
        T = rng.choice([t for t in _T if t * C <= max_elems])
        if (T, C) not in out:
            out.append((T, C))
    return out


SHAPES = _draws()


def randn(shape, seed, scale=1.0, dtype=BF16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * scale).to(dtype)


@pytest.mark.parametrize("T,C", SHAPES)
def test_random_shape_six_kernels(T, C):
    nC = 4 * C
    seed = 1000 + 7 * T + C
    x = randn((T, 4, C), seed)
    W = randn((32, nC), seed + 1, 0.02)
    xd, Wd = x.to(DEV), W.to(DEV)
    xf = x.view(T, nC)

    # K1 forward and the fused backward (grad_x and grad_W).
    proj, inv = K.k1_fwd(xd.view(T, nC), Wd)
    R, S, invR = O.k1_fwd(xf, W)
    check_bf16("k1 proj", proj, R, S, nC)
    check_rel("k1 inv_rms", inv, invR, rtol=4 * nC ** 0.5 * 2.0**-24 + 4 * 2.0**-24)
    go1 = randn((T, 32), seed + 2)
    gx, gW = K.k1_bwd(go1.to(DEV), xd.view(T, nC), Wd, proj, inv)
    R, S = O.k1_bwd_dx(go1, xf, W, proj.cpu(), inv.cpu())
    check_bf16("k1 grad_x", gx, R, S, 64)
    R, S = O.k1_grad_W(go1, xf, inv.cpu())
    check_bf16("k1 grad_W", gW, R, S, T)

    # K3 forward and backward.
    h = randn((T, 4), seed + 3, dtype=torch.float32)
    out = K.k3_fwd(xd, h.to(DEV))
    R, S = O.k3_fwd(x, h)
    check_bf16("k3 out", out, R, S, 4)
    go3 = randn((T, C), seed + 4)
    gx3, gh3 = K.k3_bwd(go3.to(DEV), xd, h.to(DEV))
    gxR, gxS, ghR, ghS = O.k3_bwd(go3, x, h)
    check_bf16("k3 grad_x", gx3, gxR, gxS, 1)
    check_fp32("k3 grad_h_pre", gh3, ghR, ghS, C)

    # K4 forward and backward.
    lo = randn((T, C), seed + 5)
    H = randn((T, 4, 4), seed + 6, dtype=torch.float32)
    hp = randn((T, 4), seed + 7, dtype=torch.float32)
    out4 = K.k4_fwd(xd, lo.to(DEV), H.to(DEV), hp.to(DEV))
    R, S = O.k4_fwd(x, lo, H, hp)
    check_bf16("k4 out", out4, R, S, 5)
    go4 = randn((T, 4, C), seed + 8)
    gx4, glo, gH, ghp = K.k4_bwd(go4.to(DEV), xd, lo.to(DEV), H.to(DEV), hp.to(DEV))
    ref = O.k4_bwd(go4, x, lo, H, hp)
    check_bf16("k4 grad_x", gx4, *ref["grad_x"], 4)
    check_bf16("k4 grad_lo", glo, *ref["grad_lo"], 4)
    check_fp32("k4 grad_H", gH, *ref["grad_H"], C)
    check_fp32("k4 grad_hp", ghp, *ref["grad_hp"], C)
