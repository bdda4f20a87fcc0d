"""GPU parity of the six HIP kernels against the float64 oracle.

Inputs are generated on the CPU from fixed seeds and copied to the GPU, so the
oracle sees exactly the kernels' inputs.  Tolerances: tests/parity.py.
Shapes cover the reference's own test size (T=2048, C=256), the edge shapes
of the eval config (T in {1, 64, 257} at C=4096), ragged C (tails of the
16-byte paths), C that forces the element-wise paths, base pointers that are
not 16-byte aligned, and the metric size T=65536, C=1024 (checked on a random
sample of tokens: every kernel is independent per token).
"""

from __future__ import annotations

import pytest
import torch

from flash_mhc import kernels as K
from oracle import mhc_oracle as O
from parity import check_bf16, check_fp32, check_rel

pytestmark = pytest.mark.gpu

DEV = "cuda"


def randn(shape, seed, scale=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * scale).to(dtype)


def stress_rows(x: torch.Tensor, seed: int, frac=0.01, factor=100.0) -> torch.Tensor:
    """Scale ~frac of the tokens (dim 0) by `factor` (the eval config's RMSNorm stress)."""
    g = torch.Generator().manual_seed(seed)
    T = x.shape[0]
    k = max(1, int(T * frac))
    idx = torch.randperm(T, generator=g)[:k]
    y = x.float().clone()
    y[idx] *= factor
    return y.to(x.dtype)


def misaligned(t: torch.Tensor) -> torch.Tensor:
    """Same values, on the GPU, at a base address that is 2 mod 16 bytes."""
    buf = torch.empty(t.numel() + 8, dtype=t.dtype, device=DEV)
    view = buf[1 : 1 + t.numel()].view(t.shape)
    view.copy_(t.to(DEV))
    assert view.data_ptr() % 16 != 0
    return view


# (T, C) pairs; nC = 4C.  C=24 / 100 / 1000 exercise ragged tails of the
# vector paths (K1: nC % 64 != 0; K3/K4: C/8 not a multiple of the lanes per
# token); C=25 forces the element-wise paths (C % 8 != 0, nC % 8 != 0).  C=300
# and 2050 run the element-wise K3/K4 paths with a workgroup per token (256
# lanes, the per-token sums finished across waves).  C=2560, 3072 and 3584 run
# the 16-byte K3/K4 paths with a workgroup of one group per lane (320, 384 and
# 448 lanes: five to seven waves).
SHAPES = [(2048, 256), (257, 1024), (1, 4096), (64, 4096), (333, 100), (129, 1000), (31, 24), (17, 25),
          (7, 300), (5, 2050), (33, 2560), (9, 3072), (5, 3584)]


# ---------------------------------------------------------------------------
# K1


def _k1_inputs(T, C, seed, w_scale=0.02, stress=False):
    nC = 4 * C
    x = randn((T, nC), seed)
    if stress:
        x = stress_rows(x, seed + 1)
    W = randn((32, nC), seed + 2, scale=w_scale)
    return x, W


@pytest.mark.parametrize("T,C", SHAPES)
def test_k1_fwd(T, C):
    x, W = _k1_inputs(T, C, seed=10 + T + C, stress=True)
    out, inv = K.k1_fwd(x.to(DEV), W.to(DEV))
    torch.cuda.synchronize()
    R, S, invR = O.k1_fwd(x, W)
    check_bf16("k1 proj", out, R, S, 4 * C)
    check_rel("k1 inv_rms", inv, invR, rtol=4 * (4 * C) ** 0.5 * 2.0**-24 + 4 * 2.0**-24)


@pytest.mark.parametrize("T,C", [(2048, 256), (17, 25), (257, 1024)])
def test_k1_fwd_misaligned(T, C):
    x, W = _k1_inputs(T, C, seed=77)
    out, inv = K.k1_fwd(misaligned(x), W.to(DEV))
    torch.cuda.synchronize()
    R, S, invR = O.k1_fwd(x, W)
    check_bf16("k1 proj (misaligned x)", out, R, S, 4 * C)
    check_rel("k1 inv_rms (misaligned x)", inv, invR, rtol=1e-5)


@pytest.mark.parametrize("T,C", [(1, 1024), (100, 4096), (2048, 1024), (4095, 1024), (8191, 256), (8192, 1024),
                                 (8193, 1024), (16417, 1024), (3, 16384)])
def test_k1_fwd_split_columns(T, C):
    """Few tokens: fmhc_k1_fwd_ws splits the nC axis over workgroups and adds
    the fp32 partials in a fixed order.  Both it and the one-pass fmhc_k1_fwd
    meet the oracle's bound; the split result is deterministic; where no split
    is planned (workspace size 0, always from T = 2721 on) the two entry
    points run the same kernel: 16-token workgroups up to T = 4096 (T = 4095:
    a ragged last one), 32-token tiles up to 8192, 48 up to 12288 (T = 8193:
    ragged), 64 beyond (T = 16417: ragged)."""
    from flash_mhc import _abi

    nC = 4 * C
    x, W = _k1_inputs(T, C, seed=90 + T, stress=True)
    xd, Wd = x.to(DEV), W.to(DEV)
    lib = _abi.load()
    nbytes = int(lib.fmhc_k1_fwd_workspace_bytes(T, nC))
    assert nbytes > 0 if T <= 256 else True  # few tokens always split
    assert nbytes == 0 if T > 2720 else True
    a = K.k1_fwd(xd, Wd)
    b = K.k1_fwd(xd, Wd)
    one = (torch.empty(T, 32, dtype=torch.bfloat16, device=DEV), torch.empty(T, device=DEV))
    st = lib.fmhc_k1_fwd(xd.data_ptr(), Wd.data_ptr(), one[0].data_ptr(), one[1].data_ptr(), T, nC, 32,
                         _abi.stream_of(xd))
    assert st == 0
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    R, S, invR = O.k1_fwd(x, W)
    for name, (out, inv) in (("split", a), ("one-pass", one)):
        check_bf16(f"k1 proj ({name})", out, R, S, nC)
        check_rel(f"k1 inv_rms ({name})", inv, invR, rtol=4 * nC ** 0.5 * 2.0**-24 + 4 * 2.0**-24)
    if nbytes == 0:
        assert torch.equal(a[0], one[0]) and torch.equal(a[1], one[1])
    else:  # a workspace one byte short is refused before any launch
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        st = lib.fmhc_k1_fwd_ws(xd.data_ptr(), Wd.data_ptr(), one[0].data_ptr(), one[1].data_ptr(),
                                ws.data_ptr(), nbytes - 1, T, nC, 32, _abi.stream_of(xd))
        assert st == 1  # FMHC_ERR_INVALID_ARGUMENT


def test_k1_fwd_unit_weights():
    # Reference test distribution: W ~ N(0, 1).
    x, W = _k1_inputs(2048, 256, seed=5, w_scale=1.0)
    out, _ = K.k1_fwd(x.to(DEV), W.to(DEV))
    R, S, _ = O.k1_fwd(x, W)
    check_bf16("k1 proj (W ~ N(0,1))", out, R, S, 1024)


@pytest.mark.parametrize("T,C", SHAPES)
def test_k1_bwd_dx(T, C):
    x, W = _k1_inputs(T, C, seed=20 + T + C, stress=True)
    go = randn((T, 32), seed=21 + T)
    xd, Wd = x.to(DEV), W.to(DEV)
    proj, inv = K.k1_fwd(xd, Wd)
    gx = K.k1_bwd_dx(go.to(DEV), xd, Wd, proj, inv)
    torch.cuda.synchronize()
    R, S = O.k1_bwd_dx(go, x, W, proj.cpu(), inv.cpu())
    check_bf16("k1 grad_x", gx, R, S, 64)


def test_k1_bwd_dx_misaligned():
    T, C = 300, 256
    x, W = _k1_inputs(T, C, seed=31)
    go = randn((T, 32), seed=32)
    proj, inv = K.k1_fwd(x.to(DEV), W.to(DEV))
    gx = K.k1_bwd_dx(misaligned(go), misaligned(x), W.to(DEV), misaligned(proj.cpu()), inv)
    R, S = O.k1_bwd_dx(go, x, W, proj.cpu(), inv.cpu())
    check_bf16("k1 grad_x (misaligned)", gx, R, S, 64)


def test_k1_bwd_inv_rms_off_16_bytes():
    """Every operand aligned but inv_rms (4 mod 16 bytes): the matrix-core
    backward reads inv_rms 16 bytes at a time, so this input takes the
    element-wise kernels, which must give the oracle's values too."""
    T, C = 320, 256
    x, W = _k1_inputs(T, C, seed=33)
    go = randn((T, 32), seed=34)
    xd, Wd, god = x.to(DEV), W.to(DEV), go.to(DEV)
    proj, inv = K.k1_fwd(xd, Wd)
    inv_off = misaligned(inv.cpu())
    assert inv_off.data_ptr() % 16 == 4
    gx = K.k1_bwd_dx(god, xd, Wd, proj, inv_off)
    gx2, gW = K.k1_bwd(god, xd, Wd, proj, inv_off)
    R, S = O.k1_bwd_dx(go, x, W, proj.cpu(), inv.cpu())
    check_bf16("k1 grad_x (inv_rms off 16)", gx, R, S, 64)
    check_bf16("k1 fused grad_x (inv_rms off 16)", gx2, R, S, 64)
    R, S = O.k1_grad_W(go, x, inv.cpu())
    check_bf16("k1 fused grad_W (inv_rms off 16)", gW, R, S, T)


@pytest.mark.parametrize(
    "T,C", [(2048, 256), (257, 1024), (1, 4096), (1500, 1024), (20000, 256), (333, 100), (31, 24), (17, 25)]
)
def test_k1_bwd_fused_dw(T, C):
    """grad_x and grad_W in one pass: grad_x as the dx kernel, grad_W against
    the oracle's bf16(bf16(go * inv_rms)^T @ x) with n = T terms.  T = 20000
    spans several workgroups along T, the last one with idle waves."""
    x, W = _k1_inputs(T, C, seed=200 + T + C, stress=True)
    go = randn((T, 32), seed=201 + T)
    xd, Wd = x.to(DEV), W.to(DEV)
    proj, inv = K.k1_fwd(xd, Wd)
    gx, gW = K.k1_bwd(go.to(DEV), xd, Wd, proj, inv)
    gx_ref = K.k1_bwd_dx(go.to(DEV), xd, Wd, proj, inv)
    torch.cuda.synchronize()
    R, S = O.k1_bwd_dx(go, x, W, proj.cpu(), inv.cpu())
    check_bf16("k1 fused grad_x", gx, R, S, 64)
    assert torch.equal(gx, gx_ref)  # same arithmetic as the dx-only kernel
    R, S = O.k1_grad_W(go, x, inv.cpu())
    check_bf16("k1 fused grad_W", gW, R, S, T)


def test_k1_bwd_fused_dw_misaligned_and_empty():
    T, C = 300, 256
    x, W = _k1_inputs(T, C, seed=210)
    go = randn((T, 32), seed=211)
    proj, inv = K.k1_fwd(x.to(DEV), W.to(DEV))
    gx, gW = K.k1_bwd(misaligned(go), misaligned(x), W.to(DEV), misaligned(proj.cpu()), inv)
    R, S = O.k1_grad_W(go, x, inv.cpu())
    check_bf16("k1 fused grad_W (element-wise path)", gW, R, S, T)
    e = torch.empty((0, 4 * C), dtype=torch.bfloat16, device=DEV)
    gx0, gW0 = K.k1_bwd(torch.empty((0, 32), dtype=torch.bfloat16, device=DEV), e, W.to(DEV),
                        torch.empty((0, 32), dtype=torch.bfloat16, device=DEV),
                        torch.empty((0,), device=DEV))
    assert gx0.shape == (0, 4 * C) and torch.count_nonzero(gW0) == 0


def test_k1_bwd_fused_dw_deterministic():
    T, C = 4096, 1024
    x, W = _k1_inputs(T, C, seed=220)
    go = randn((T, 32), seed=221)
    xd, Wd = x.to(DEV), W.to(DEV)
    proj, inv = K.k1_fwd(xd, Wd)
    a = K.k1_bwd(go.to(DEV), xd, Wd, proj, inv)
    b = K.k1_bwd(go.to(DEV), xd, Wd, proj, inv)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


# ---------------------------------------------------------------------------
# K3


def _streams(T, C, seed, stress=False):
    x = randn((T, 4, C), seed)
    return stress_rows(x, seed + 1) if stress else x


@pytest.mark.parametrize("T,C", SHAPES)
def test_k3_fwd(T, C):
    x = _streams(T, C, 40 + T + C, stress=True)
    h = randn((T, 4), 41 + T, dtype=torch.float32)
    out = K.k3_fwd(x.to(DEV), h.to(DEV))
    R, S = O.k3_fwd(x, h)
    check_bf16("k3 out", out, R, S, 4)


@pytest.mark.parametrize("T,C", SHAPES)
def test_k3_bwd(T, C):
    x = _streams(T, C, 50 + T + C)
    h = randn((T, 4), 51 + T, dtype=torch.float32)
    go = randn((T, C), 52 + T)
    gx, gh = K.k3_bwd(go.to(DEV), x.to(DEV), h.to(DEV))
    gxR, gxS, ghR, ghS = O.k3_bwd(go, x, h)
    check_bf16("k3 grad_x", gx, gxR, gxS, 1)
    check_fp32("k3 grad_h_pre", gh, ghR, ghS, C)


def test_k3_misaligned():
    T, C = 129, 1000
    x = _streams(T, C, 60)
    h = randn((T, 4), 61, dtype=torch.float32)
    go = randn((T, C), 62)
    out = K.k3_fwd(misaligned(x), h.to(DEV))
    R, S = O.k3_fwd(x, h)
    check_bf16("k3 out (misaligned)", out, R, S, 4)
    gx, gh = K.k3_bwd(misaligned(go), misaligned(x), h.to(DEV))
    gxR, gxS, ghR, ghS = O.k3_bwd(go, x, h)
    check_bf16("k3 grad_x (misaligned)", gx, gxR, gxS, 1)
    check_fp32("k3 grad_h_pre (misaligned)", gh, ghR, ghS, C)


# ---------------------------------------------------------------------------
# K4


def _k4_inputs(T, C, seed, stress=False):
    x = _streams(T, C, seed, stress)
    lo = randn((T, C), seed + 2)
    H = randn((T, 4, 4), seed + 3, dtype=torch.float32)
    hp = randn((T, 4), seed + 4, dtype=torch.float32)
    return x, lo, H, hp


@pytest.mark.parametrize("T,C", SHAPES)
def test_k4_fwd(T, C):
    x, lo, H, hp = _k4_inputs(T, C, 70 + T + C, stress=True)
    out = K.k4_fwd(x.to(DEV), lo.to(DEV), H.to(DEV), hp.to(DEV))
    R, S = O.k4_fwd(x, lo, H, hp)
    check_bf16("k4 out", out, R, S, 5)


@pytest.mark.parametrize("T,C", SHAPES)
def test_k4_bwd(T, C):
    x, lo, H, hp = _k4_inputs(T, C, 80 + T + C)
    go = randn((T, 4, C), 85 + T)
    gx, glo, gH, ghp = K.k4_bwd(go.to(DEV), x.to(DEV), lo.to(DEV), H.to(DEV), hp.to(DEV))
    ref = O.k4_bwd(go, x, lo, H, hp)
    check_bf16("k4 grad_x", gx, *ref["grad_x"], 4)
    check_bf16("k4 grad_lo", glo, *ref["grad_lo"], 4)
    check_fp32("k4 grad_H", gH, *ref["grad_H"], C)
    check_fp32("k4 grad_hp", ghp, *ref["grad_hp"], C)


@pytest.mark.parametrize("n,C", [(8192, 1024), (4096, 4096), (16384, 512)])
def test_k4_bwd_early_and_late_loads_agree(n, C):
    """K4's backward issues each iteration's loads before its stores up to
    16384 tokens x 64 lanes (n tokens x the lanes per token here: 128 at
    C = 1024, 256 at 4096, 64 at 512) and keeps the plain loop above: the
    same arithmetic in the same order, so the first n tokens of an
    (n + 1)-token call equal an n-token call bit for bit."""
    x, lo, H, hp = (t.to(DEV) for t in _k4_inputs(n + 1, C, 97))
    go = randn((n + 1, 4, C), 98).to(DEV)
    late = K.k4_bwd(go, x, lo, H, hp)
    early = K.k4_bwd(go[:n], x[:n], lo[:n], H[:n], hp[:n])
    for u, v in zip(early, late):
        assert torch.equal(u, v[:n])


def test_k4_misaligned():
    T, C = 129, 1000
    x, lo, H, hp = _k4_inputs(T, C, 90)
    go = randn((T, 4, C), 95)
    out = K.k4_fwd(misaligned(x), misaligned(lo), H.to(DEV), hp.to(DEV))
    R, S = O.k4_fwd(x, lo, H, hp)
    check_bf16("k4 out (misaligned)", out, R, S, 5)
    gx, glo, gH, ghp = K.k4_bwd(misaligned(go), x.to(DEV), misaligned(lo), H.to(DEV), hp.to(DEV))
    ref = O.k4_bwd(go, x, lo, H, hp)
    check_bf16("k4 grad_x (misaligned)", gx, *ref["grad_x"], 4)
    check_bf16("k4 grad_lo (misaligned)", glo, *ref["grad_lo"], 4)
    check_fp32("k4 grad_H (misaligned)", gH, *ref["grad_H"], C)
    check_fp32("k4 grad_hp (misaligned)", ghp, *ref["grad_hp"], C)


# ---------------------------------------------------------------------------
# Metric size T=65536, n=4, C=1024, and the same T at C=2560 (K3/K4 with 320
# lanes per token): all six kernels, checked on 512 sampled tokens (each
# kernel is independent per token, so the oracle runs on the sampled rows
# only).


@pytest.mark.parametrize("C", [1024, 2560])
def test_metric_size_sampled(C):
    T = 65536
    nC = 4 * C
    g = torch.Generator().manual_seed(1234)
    idx = torch.randperm(T, generator=g)[:512]
    # Besides the random tokens: a contiguous band (whole 64-token tiles of K1
    # forward and both halves of a 16-token block of K1 backward) and the
    # last tile.
    band = T - 40960
    idx = torch.cat([idx, torch.arange(band - 80, band + 80), torch.arange(T - 64, T)]).unique()
    x = randn((T, 4, C), 1)
    W = randn((32, nC), 2, scale=0.02)
    lo = randn((T, C), 3)
    H = randn((T, 4, 4), 4, dtype=torch.float32)
    hp = randn((T, 4), 5, dtype=torch.float32)
    hpre = randn((T, 4), 6, dtype=torch.float32)
    go1 = randn((T, 32), 7)
    go3 = randn((T, C), 8)
    go4 = randn((T, 4, C), 9)
    xd = x.to(DEV)
    xf = xd.view(T, nC)
    Wd = W.to(DEV)

    proj, inv = K.k1_fwd(xf, Wd)
    gx1 = K.k1_bwd_dx(go1.to(DEV), xf, Wd, proj, inv)
    out3 = K.k3_fwd(xd, hpre.to(DEV))
    gx3, gh3 = K.k3_bwd(go3.to(DEV), xd, hpre.to(DEV))
    out4 = K.k4_fwd(xd, lo.to(DEV), H.to(DEV), hp.to(DEV))
    gx4, glo4, gH4, ghp4 = K.k4_bwd(go4.to(DEV), xd, lo.to(DEV), H.to(DEV), hp.to(DEV))
    torch.cuda.synchronize()

    i = idx.to(DEV)
    xs = x[idx]
    R, S, invR = O.k1_fwd(xs.view(-1, nC), W)
    check_bf16("k1 proj @metric", proj[i], R, S, nC)
    check_rel("k1 inv_rms @metric", inv[i], invR, rtol=1e-5)
    R, S = O.k1_bwd_dx(go1[idx], xs.view(-1, nC), W, proj[i].cpu(), inv[i].cpu())
    check_bf16("k1 grad_x @metric", gx1[i], R, S, 64)
    R, S = O.k3_fwd(xs, hpre[idx])
    check_bf16("k3 out @metric", out3[i], R, S, 4)
    gxR, gxS, ghR, ghS = O.k3_bwd(go3[idx], xs, hpre[idx])
    check_bf16("k3 grad_x @metric", gx3[i], gxR, gxS, 1)
    check_fp32("k3 grad_h_pre @metric", gh3[i], ghR, ghS, C)
    R, S = O.k4_fwd(xs, lo[idx], H[idx], hp[idx])
    check_bf16("k4 out @metric", out4[i], R, S, 5)
    ref = O.k4_bwd(go4[idx], xs, lo[idx], H[idx], hp[idx])
    check_bf16("k4 grad_x @metric", gx4[i], *ref["grad_x"], 4)
    check_bf16("k4 grad_lo @metric", glo4[i], *ref["grad_lo"], 4)
    check_fp32("k4 grad_H @metric", gH4[i], *ref["grad_H"], C)
    check_fp32("k4 grad_hp @metric", ghp4[i], *ref["grad_hp"], C)


@pytest.mark.parametrize("T,sub,tile,C", [(4000, 3200, 16, 4096), (6150, 4352, 32, 4096), (12000, 8256, 48, 4096),
                                          (16000, 12352, 64, 4096), (40000, 30016, 64, 1024)])
def test_k1_fwd_tile_sizes(T, sub, tile, C):
    """K1 forward on each one-pass tile size (blocks of 16 tokens, as many per
    workgroup as keep the launch to one round of 256 workgroups, at most 4:
    16, 32, 48 and 64 tokens), at wide rows and with a ragged last tile.  Sampled tokens (random, and the last tile) against the
    oracle; the first `sub` rows computed alone (the same tile size) give the
    same bits: a tile's result depends on its own rows and its workgroup's
    place only (the chunk rotation starts at the workgroup id)."""
    nC = 4 * C
    g = torch.Generator().manual_seed(99)
    idx = torch.cat([torch.randperm(T, generator=g)[:192], torch.arange(T - 40, T)]).unique()
    x = randn((T, nC), 21)
    W = randn((32, nC), 22, scale=0.02)
    xd, Wd = x.to(DEV), W.to(DEV)
    proj, inv = K.k1_fwd(xd, Wd)
    i = idx.to(DEV)
    R, S, invR = O.k1_fwd(x[idx], W)
    check_bf16(f"k1 proj ({tile}-token tiles, wide rows)", proj[i], R, S, nC)
    check_rel(f"k1 inv_rms ({tile}-token tiles, wide rows)", inv[i], invR, rtol=1e-5)
    assert sub % tile == 0
    p2, i2 = K.k1_fwd(xd[:sub].contiguous(), Wd)
    torch.cuda.synchronize()
    assert torch.equal(p2, proj[:sub]) and torch.equal(i2, inv[:sub])


# ---------------------------------------------------------------------------
# Launch behaviour


def test_deterministic_and_stream_aware():
    """Bitwise-identical results run to run, and on a non-default stream."""
    T, C = 1024, 1024
    x, lo, H, hp = _k4_inputs(T, C, 100)
    go = randn((T, 4, C), 101)
    W = randn((32, 4 * C), 102, scale=0.02)
    args = [t.to(DEV) for t in (go, x, lo, H, hp)]
    a = K.k4_bwd(*args)
    b = K.k4_bwd(*args)
    p1 = K.k1_fwd(args[1].view(T, -1), W.to(DEV))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        from flash_mhc import _abi

        assert _abi.stream_of(args[0]) == s.cuda_stream  # launches go to the current stream
        c = K.k4_bwd(*args)
        p2 = K.k1_fwd(args[1].view(T, -1), W.to(DEV))
    assert _abi.stream_of(args[0]) == torch.cuda.current_stream().cuda_stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for u, v, w in zip(a, b, c):
        assert torch.equal(u, v) and torch.equal(u, w)
    assert torch.equal(p1[0], p2[0]) and torch.equal(p1[1], p2[1])


def test_empty_tokens():
    x = torch.empty((0, 4, 256), dtype=torch.bfloat16, device=DEV)
    h = torch.empty((0, 4), dtype=torch.float32, device=DEV)
    assert K.k3_fwd(x, h).shape == (0, 256)
    out, inv = K.k1_fwd(x.view(0, 1024), torch.zeros((32, 1024), dtype=torch.bfloat16, device=DEV))
    assert out.shape == (0, 32) and inv.shape == (0,)


def test_single_hip_runtime():
    """The extension shares torch's HIP runtime (one libamdhip64 mapped)."""
    from flash_mhc import _abi

    _abi.load()
    torch.zeros(1, device=DEV)
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            if "libamdhip64" in line:
                paths.add(line.split()[-1])
    assert len(paths) == 1, paths
