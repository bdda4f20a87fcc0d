"""GPU parity of the single-read pre-map forward (premap_resident.hip): rows of
C = 512 or 1024 per stream, at least 16384 tokens, with a layer input.

Each stage is checked against the oracle with the kernel's own upstream
outputs as the oracle's inputs (tests/parity.py): proj to K1's bf16 rule over
nC terms, inv_rms to a relative bound, K2's outputs to the chain rule, the
layer input to K3's bf16 rule.  K2 and K3 must moreover equal the separate K2
and K3 kernels run on the kernel's own projection bit for bit (the same
per-token arithmetic in the same order); only K1's fp32 summation order
differs from the K1 op's.  The re-read build (premap_reread, the tile kernel
at these shapes) must equal K1 -> K2 -> K3 launched separately, bit for bit.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from flash_mhc import _abi, build
from flash_mhc import kernels as K
from oracle import k2_oracle as K2O
from oracle import mhc_oracle as O
from parity import check_bf16, check_chain, check_rel

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16 = torch.bfloat16
PERM = O.permutation_matrices(4)[0]


def _inputs(T, C, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((T, 4, C), generator=g).to(BF16)
    idx = torch.randperm(T, generator=g)[: max(1, T // 100)]
    x[idx] = (x[idx].float() * 100).to(BF16)  # 1% of the tokens far from unit RMS
    W = (torch.randn((32, 4 * C), generator=g) * 0.02).to(BF16)
    p = [torch.tensor([0.8]), torch.tensor([1.2]), torch.tensor([1.7]), torch.randn(32, generator=g) * 0.5, PERM]
    return x, W, p


# The threshold itself, a ragged last block, block counts that are and are
# not multiples of the 256 workgroups, and both widths.
@pytest.mark.parametrize("T,C", [(16384, 1024), (32768, 1024), (32769, 1024), (65536, 1024), (20001, 512),
                                 (40001, 512), (70001, 512)])
def test_resident_stages(T, C):
    nC = 4 * C
    x, W, p = _inputs(T, C, 500 + T + C)
    xd, Wd, pd = x.to(DEV), W.to(DEV), [t.to(DEV) for t in p]
    li, H, hq, hp, proj, inv = K.premap_fwd(xd, Wd, *pd)
    torch.cuda.synchronize()
    R, S, invR = O.k1_fwd(x.view(T, nC), W)
    check_bf16("resident proj", proj, R, S, nC)
    check_rel("resident inv_rms", inv, invR, rtol=4 * nC ** 0.5 * 2.0 ** -24 + 4 * 2.0 ** -24)
    f = K2O.k2_fwd(proj.cpu(), *p)
    check_chain("resident h_pre", hp, f["h_pre"])
    check_chain("resident h_post", hq, f["h_post"])
    check_chain("resident H_merged", H, f["H_merged"])
    R3, S3 = O.k3_fwd(x, hp.cpu())
    check_bf16("resident layer_input", li, R3, S3, 4)
    # K2 and K3 kernels on this kernel's projection and h_pre: the same bits.
    hp1, hq1, H1 = K.k2_fwd(proj, *pd)
    li1 = K.k3_fwd(xd, hp1)
    for name, a, b in (("h_pre", hp, hp1), ("h_post", hq, hq1), ("H_merged", H, H1), ("layer_input", li, li1)):
        assert torch.equal(a, b), f"{name}: {int((a != b).sum())} of {a.numel()} differ"


def test_resident_repeatable():
    """Two launches on the same inputs give the same bits (fixed summation
    order over the waves; no atomics)."""
    T, C = 65537, 1024
    x, W, p = _inputs(T, C, 7)
    xd, Wd, pd = x.to(DEV), W.to(DEV), [t.to(DEV) for t in p]
    a = K.premap_fwd(xd, Wd, *pd)
    b = K.premap_fwd(xd, Wd, *pd)
    torch.cuda.synchronize()
    for u, v in zip(a, b):
        assert torch.equal(u, v)


@pytest.fixture(scope="module")
def reread_lib():
    _abi.load()
    path = build.variant_path("premap_reread")
    if not path.exists():
        pytest.skip(f"evidence build not present: {path} (python -m flash_mhc.build --variants)")
    lib = ctypes.CDLL(str(path), mode=ctypes.RTLD_LOCAL)
    for name, argtypes in _abi.SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _abi.RESTYPES.get(name, ctypes.c_int)
    return lib


@pytest.mark.parametrize("T,C", [(65536, 1024), (40001, 512)])
def test_reread_build_equals_three_kernels(reread_lib, T, C):
    """The tile kernel (K3's re-read of x from the memory-side cache) at the
    shapes the product now gives to the single-read kernel."""
    x, W, p = _inputs(T, C, 900 + C)
    xd, Wd, pd = x.to(DEV), W.to(DEV), [t.to(DEV) for t in p]
    out = dict(li=torch.empty(T, C, dtype=BF16, device=DEV), proj=torch.empty(T, 32, dtype=BF16, device=DEV),
               inv=torch.empty(T, device=DEV), hp=torch.empty(T, 4, device=DEV), hq=torch.empty(T, 4, device=DEV),
               H=torch.empty(T, 4, 4, device=DEV))
    nbytes = int(reread_lib.fmhc_premap_fwd_workspace_bytes(T, C))
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=DEV)
    st = reread_lib.fmhc_premap_fwd(xd.data_ptr(), Wd.data_ptr(), *[t.data_ptr() for t in pd], 0,
                                    out["li"].data_ptr(), out["proj"].data_ptr(), out["inv"].data_ptr(),
                                    out["hp"].data_ptr(), out["hq"].data_ptr(), out["H"].data_ptr(), None, None,
                                    ws.data_ptr(), nbytes, T, C, 4, _abi.stream_of(xd))
    assert st == 0
    proj1, inv1 = K.k1_fwd(xd.view(T, -1), Wd)
    hp1, hq1, H1 = K.k2_fwd(proj1, *pd)
    li1 = K.k3_fwd(xd, hp1)
    torch.cuda.synchronize()
    for name, a, b in (("proj", out["proj"], proj1), ("inv_rms", out["inv"], inv1), ("h_pre", out["hp"], hp1),
                       ("h_post", out["hq"], hq1), ("H_merged", out["H"], H1), ("layer_input", out["li"], li1)):
        assert torch.equal(a, b), f"{name}: {int((a != b).sum())} of {a.numel()} differ"
