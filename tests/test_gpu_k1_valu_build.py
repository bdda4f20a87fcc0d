"""GPU parity of the K1 VALU evidence build (build.py variant "k1_valu": the
K1 forward and backward-dx contractions as fp32 FMAs on the VALU, timed
against the matrix-core build).  The library is loaded beside the product
library through the same C ABI and held to the same oracle bounds, so the
timing comparison is between two builds that compute the same values.

Shapes: T = 16417 (64-token tiles, ragged last tile), T = 4096 (32-token
tiles), C = 100 (nC % 64 != 0: the ragged last chunk), few tokens (the
column-split forward), and the backward's full and ragged token blocks.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from flash_mhc import _abi, build
from oracle import mhc_oracle as O
from parity import check_bf16, check_rel

pytestmark = pytest.mark.gpu

DEV = "cuda"


def randn(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


@pytest.fixture(scope="module")
def valu():
    _abi.load()  # torch's HIP runtime first, then the variant (same soname resolution)
    path = build.variant_path("k1_valu")
    if not path.exists():
        pytest.skip(f"evidence build not present: {path} (python -m flash_mhc.build --variants)")
    lib = ctypes.CDLL(str(path), mode=ctypes.RTLD_LOCAL)
    for name, argtypes in _abi.SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _abi.RESTYPES.get(name, ctypes.c_int)
    assert lib.fmhc_abi_version() == _abi.ABI_VERSION
    return lib


@pytest.mark.parametrize("T,C", [(16417, 1024), (4096, 1024), (300, 100), (37, 4096), (1, 1024)])
def test_valu_k1_fwd_matches_oracle(valu, T, C):
    nC = 4 * C
    x = randn((T, nC), 900 + T + C)
    x[:: max(1, T // 100)] *= 100
    W = randn((32, nC), 901 + C, 0.02)
    xd, Wd = x.to(DEV), W.to(DEV)
    out = torch.empty(T, 32, dtype=torch.bfloat16, device=DEV)
    inv = torch.empty(T, device=DEV)
    nbytes = int(valu.fmhc_k1_fwd_workspace_bytes(T, nC))
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=DEV)
    st = valu.fmhc_k1_fwd_ws(xd.data_ptr(), Wd.data_ptr(), out.data_ptr(), inv.data_ptr(), ws.data_ptr(), nbytes,
                             T, nC, 32, _abi.stream_of(xd))
    assert st == 0
    torch.cuda.synchronize()
    R, S, invR = O.k1_fwd(x, W)
    check_bf16("valu k1 proj", out, R, S, nC)
    check_rel("valu k1 inv_rms", inv, invR, rtol=4 * nC ** 0.5 * 2.0**-24 + 4 * 2.0**-24)


@pytest.mark.parametrize("T,C", [(4096, 1024), (257, 1024), (33, 4096)])
def test_valu_k1_bwd_dx_matches_oracle(valu, T, C):
    nC = 4 * C
    x = randn((T, nC), 910 + T)
    W = randn((32, nC), 911 + C, 0.02)
    go = randn((T, 32), 912 + T)
    xd, Wd, god = x.to(DEV), W.to(DEV), go.to(DEV)
    from flash_mhc import kernels as K

    proj, inv = K.k1_fwd(xd, Wd)  # the product library's forward
    gx = torch.empty_like(xd)
    st = valu.fmhc_k1_bwd_dx(xd.data_ptr(), Wd.data_ptr(), god.data_ptr(), proj.data_ptr(), inv.data_ptr(),
                             gx.data_ptr(), T, nC, 32, _abi.stream_of(xd))
    assert st == 0
    torch.cuda.synchronize()
    R, S = O.k1_bwd_dx(go, x, W, proj.cpu(), inv.cpu())
    check_bf16("valu k1 grad_x", gx, R, S, 64)
