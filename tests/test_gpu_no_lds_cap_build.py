"""The product launches K1's backward dx (up to C = 2560), K3 forward, K3
backward (with grad_x, up to C = 2048) and K4 forward (from 16 workgroups per
CU on) with LDS reserved that the kernels do not use, which caps how many
workgroups share a CU.  The evidence build "no_lds_cap" launches them
without it.  Loaded beside the product library through the same C ABI, its
K1, K3 and K4 entry points must give the product's outputs bit for bit: the
cap changes residency, not arithmetic."""

from __future__ import annotations

import ctypes

import pytest
import torch

from flash_mhc import _abi, build

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16 = torch.bfloat16


@pytest.fixture(scope="module")
def nocap_lib():
    _abi.load()
    path = build.variant_path("no_lds_cap")
    if not path.exists():
        pytest.skip(f"evidence build not present: {path} (python -m flash_mhc.build --variants)")
    lib = ctypes.CDLL(str(path), mode=ctypes.RTLD_LOCAL)
    for name, argtypes in _abi.SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _abi.RESTYPES.get(name, ctypes.c_int)
    return lib


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16) if t.dtype == BF16 else t.view(torch.int32)


def _k134(lib, x, W, go1, lo, hp, hq, H, go3, go4):
    T, n, C = x.shape
    s = _abi.stream_of(x)
    proj = torch.empty(T, 32, dtype=BF16, device=DEV)
    inv = torch.empty(T, device=DEV)
    gx1 = torch.empty_like(x)
    assert lib.fmhc_k1_fwd(x.data_ptr(), W.data_ptr(), proj.data_ptr(), inv.data_ptr(), T, n * C, 32, s) == 0
    assert lib.fmhc_k1_bwd_dx(x.data_ptr(), W.data_ptr(), go1.data_ptr(), proj.data_ptr(), inv.data_ptr(),
                              gx1.data_ptr(), T, n * C, 32, s) == 0
    out = dict(proj=proj, inv=inv, gx1=gx1, li=torch.empty(T, C, dtype=BF16, device=DEV), gx3=torch.empty_like(x),
               gh3=torch.empty(T, n, device=DEV), out4=torch.empty_like(x), gx4=torch.empty_like(x),
               glo4=torch.empty(T, C, dtype=BF16, device=DEV), gH4=torch.empty(T, n, n, device=DEV),
               ghq4=torch.empty(T, n, device=DEV), gh3r=torch.empty(T, n, device=DEV))
    assert lib.fmhc_k3_fwd(x.data_ptr(), hp.data_ptr(), out["li"].data_ptr(), T, C, n, s) == 0
    assert lib.fmhc_k3_bwd(x.data_ptr(), hp.data_ptr(), go3.data_ptr(), out["gx3"].data_ptr(),
                           out["gh3"].data_ptr(), T, C, n, s) == 0
    assert lib.fmhc_k3_bwd(x.data_ptr(), hp.data_ptr(), go3.data_ptr(), None, out["gh3r"].data_ptr(),
                           T, C, n, s) == 0
    assert lib.fmhc_k4_fwd(x.data_ptr(), lo.data_ptr(), H.data_ptr(), hq.data_ptr(), out["out4"].data_ptr(),
                           T, C, n, s) == 0
    assert lib.fmhc_k4_bwd(x.data_ptr(), lo.data_ptr(), H.data_ptr(), hq.data_ptr(), go4.data_ptr(),
                           out["gx4"].data_ptr(), out["glo4"].data_ptr(), out["gH4"].data_ptr(),
                           out["ghq4"].data_ptr(), T, C, n, s) == 0
    torch.cuda.synchronize()
    return out


# The metric width and its neighbours at many tokens (the caps apply), a
# ragged token count, few tokens (K4 forward below the cap's threshold),
# C = 4096 (K1 and K3 backward uncapped) and the one-element path (C = 100).
@pytest.mark.parametrize("T,C", [(65536, 1024), (20001, 512), (16384, 2048), (4096, 1024), (16384, 4096),
                                 (3000, 2560), (777, 100)])
def test_capped_launches_equal_uncapped(nocap_lib, T, C):
    g = torch.Generator(device=DEV).manual_seed(T + C)
    x = torch.randn(T, 4, C, device=DEV, generator=g).to(BF16)
    W = (torch.randn(32, 4 * C, device=DEV, generator=g) * 0.02).to(BF16)
    go1 = torch.randn(T, 32, device=DEV, generator=g).to(BF16)
    lo = torch.randn(T, C, device=DEV, generator=g).to(BF16)
    go3 = torch.randn(T, C, device=DEV, generator=g).to(BF16)
    go4 = torch.randn(T, 4, C, device=DEV, generator=g).to(BF16)
    hp = torch.rand(T, 4, device=DEV, generator=g)
    hq = torch.rand(T, 4, device=DEV, generator=g) * 2
    H = torch.randn(T, 4, 4, device=DEV, generator=g)
    got = _k134(_abi.load(), x, W, go1, lo, hp, hq, H, go3, go4)
    want = _k134(nocap_lib, x, W, go1, lo, hp, hq, H, go3, go4)
    for k in want:
        a, b = _bits(got[k]), _bits(want[k])
        assert torch.equal(a, b), f"{k}: {int((a != b).sum())} of {a.numel()} differ"
