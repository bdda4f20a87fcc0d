"""The product's pre-map forward is one kernel wherever K1 is not split over
the columns (K1 on a tile of 16 to 64 tokens, then K2 and K3 on it by the
same workgroup).  The evidence
builds of build.py time it against K1, K2, K3 as three kernels
("premap_three_kernels") and against the one kernel with nontemporal loads of
x ("premap_tile_nt").  Loaded beside the product library through the same C
ABI, each fmhc_premap_fwd must give the product's outputs bit for bit: the
same per-token arithmetic in the same order."""

from __future__ import annotations

import ctypes

import pytest
import torch

from flash_mhc import _abi, build, build_permutation_matrices

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", params=["premap_three_kernels", "premap_tile_nt"])
def three_lib(request):
    _abi.load()
    path = build.variant_path(request.param)
    if not path.exists():
        pytest.skip(f"evidence build not present: {path} (python -m flash_mhc.build --variants)")
    lib = ctypes.CDLL(str(path), mode=ctypes.RTLD_LOCAL)
    for name, argtypes in _abi.SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _abi.RESTYPES.get(name, ctypes.c_int)
    return lib


def _run(lib, x, W, params, T, C, with_li):
    f32 = torch.float32
    out = dict(li=torch.empty(T, C, dtype=torch.bfloat16, device=DEV) if with_li else None,
               proj=torch.empty(T, 32, dtype=torch.bfloat16, device=DEV), inv=torch.empty(T, device=DEV),
               hp=torch.empty(T, 4, device=DEV), hq=torch.empty(T, 4, device=DEV),
               H=torch.empty(T, 4, 4, device=DEV, dtype=f32))
    nbytes = int(lib.fmhc_premap_fwd_workspace_bytes(T, C))
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=DEV)
    st = lib.fmhc_premap_fwd(x.data_ptr(), W.data_ptr(), *[p.data_ptr() for p in params], 0,
                             None if out["li"] is None else out["li"].data_ptr(), out["proj"].data_ptr(),
                             out["inv"].data_ptr(), out["hp"].data_ptr(), out["hq"].data_ptr(), out["H"].data_ptr(),
                             None, None, ws.data_ptr(), nbytes, T, C, 4, _abi.stream_of(x))
    assert st == 0
    torch.cuda.synchronize()
    return out


# Rows of C = 512 or 1024 with a layer input and at least 16384 tokens take the
# single-read kernel instead (tests/test_gpu_premap_resident.py); the
# metric-size tile kernel is covered here without the layer input and at
# C = 2048, and against the three kernels in the premap_reread build there.
# (16390, 4096) runs the tile's K3 part with the next piece's loads ahead of
# each store (rows of 4096), a last block of 6 tokens included.
@pytest.mark.parametrize("T,C,with_li", [(3000, 1024, True), (5000, 512, True), (7000, 1024, False),
                                         (16000, 1024, True), (16383, 1024, True), (20000, 256, True),
                                         (16390, 4096, True), (65536, 1024, False), (32768, 2048, True)])
def test_tile_kernel_equals_three_kernels(three_lib, T, C, with_li):
    g = torch.Generator().manual_seed(T + C)
    x = torch.randn(T, 4, C, generator=g).to(torch.bfloat16)
    x[:: 97] *= 100
    W = (torch.randn(32, 4 * C, generator=g) * 0.02).to(torch.bfloat16)
    params = [torch.tensor([0.8]), torch.tensor([1.2]), torch.tensor([1.7]), torch.randn(32, generator=g) * 0.5,
              build_permutation_matrices(4)[0]]
    xd, Wd = x.to(DEV), W.to(DEV)
    pd = [p.to(DEV) for p in params]
    got = _run(_abi.load(), xd, Wd, pd, T, C, with_li)
    want = _run(three_lib, xd, Wd, pd, T, C, with_li)
    for k in want:
        if want[k] is None:
            assert got[k] is None
            continue
        a, b = got[k], want[k]
        ai = a.view(torch.int16) if a.dtype == torch.bfloat16 else a.view(torch.int32)
        bi = b.view(torch.int16) if b.dtype == torch.bfloat16 else b.view(torch.int32)
        assert torch.equal(ai, bi), f"{k}: {int((ai != bi).sum())} of {ai.numel()} differ"
