"""GPU parity of the pre-map backward with one read of x (premap_split.hip,
the evidence build premap_bwd_split), at the token counts and widths where it
runs (T >= 16384, C a multiple of 128).

Its outputs must equal K3's backward -> K2's backward -> K1's backward (the
separate kernels, each reading x) bit for bit: grad_x (with and without x's
incoming gradient), grad_W and the four parameter gradients.  The same holds
when every wave computes every exchanged value itself instead of waiting for
the team (FLASH_MHC_SPLIT_SPIN=-1: the bounded waits' fallback), on repeated
calls, and against the product's pre-map backward (two reads of x).  The
separate kernels are pinned to the oracle by tests/test_gpu_kernels.py and
tests/test_gpu_k2.py.
"""

from __future__ import annotations

import ctypes
import os

import pytest
import torch

from flash_mhc import _abi, build
from flash_mhc import kernels as K
from oracle import mhc_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16 = torch.bfloat16
PERM = O.permutation_matrices(4)[0]


def _case(T, C, seed, gi):
    g = torch.Generator(device=DEV).manual_seed(seed)
    nC = 4 * C
    x = torch.randn((T, 4, C), generator=g, device=DEV).to(BF16)
    rows = torch.randperm(T, generator=g, device=DEV)[: max(1, T // 100)]
    x[rows] = (x[rows].float() * 100).to(BF16)  # 1% of the tokens far from unit RMS
    W = (torch.randn((32, nC), generator=g, device=DEV) * 0.02).to(BF16)
    p = [torch.tensor([0.8], device=DEV), torch.tensor([1.2], device=DEV), torch.tensor([1.7], device=DEV),
         torch.randn(32, generator=g, device=DEV) * 0.5, PERM.to(DEV)]
    _, _, _, hp, proj, inv = K.premap_fwd(x, W, *p)
    g_li = torch.randn((T, C), generator=g, device=DEV).to(BF16)
    g_hq = torch.randn((T, 4), generator=g, device=DEV)
    g_H = torch.randn((T, 4, 4), generator=g, device=DEV)
    g_in = torch.randn((T, 4, C), generator=g, device=DEV).to(BF16) if gi else None
    return x, W, p, hp, proj, inv, g_li, g_hq, g_H, g_in


def _composed(x, W, p, hp, proj, inv, g_li, g_hq, g_H, g_in):
    T, _, C = x.shape
    gx3, gh = K.k3_bwd(g_li, x, hp)
    gp, ra1, ra2, ra3, rb_ = K.k2_bwd(proj, *p, gh, g_hq, g_H)
    gx1, rW = K.k1_bwd(gp, x.view(T, 4 * C), W, proj, inv)
    gx = gx3 + gx1.view(T, 4, C)
    if g_in is not None:
        gx = g_in + gx
    return gx, rW, ra1, ra2, ra3, rb_


@pytest.fixture(scope="module")
def split_lib():
    _abi.load()
    path = build.variant_path("premap_bwd_split")
    if not path.exists():
        pytest.skip(f"evidence build not present: {path} (python -m flash_mhc.build --variants)")
    lib = ctypes.CDLL(str(path), mode=ctypes.RTLD_LOCAL)
    for name, argtypes in _abi.SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _abi.RESTYPES.get(name, ctypes.c_int)
    return lib


def _split(lib, x, W, p, hp, proj, inv, g_li, g_hq, g_H, g_in):
    """fmhc_premap_bwd of the evidence build."""
    T, _, C = x.shape
    gx = torch.empty_like(x)
    gW = torch.empty((32, 4 * C), dtype=BF16, device=DEV)
    ga = [torch.empty(1, device=DEV) for _ in range(3)]
    gb = torch.empty(32, device=DEV)
    nbytes = int(lib.fmhc_premap_bwd_workspace_bytes(T, C))
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=DEV)
    st = lib.fmhc_premap_bwd(x.data_ptr(), W.data_ptr(), *[t.data_ptr() for t in p], 0, hp.data_ptr(),
                             proj.data_ptr(), inv.data_ptr(), g_li.data_ptr(), g_hq.data_ptr(), g_H.data_ptr(),
                             None if g_in is None else g_in.data_ptr(), gx.data_ptr(), gW.data_ptr(),
                             ga[0].data_ptr(), ga[1].data_ptr(), ga[2].data_ptr(), gb.data_ptr(), ws.data_ptr(),
                             nbytes, T, C, 4, _abi.stream_of(x))
    assert st == 0
    return gx, gW, *ga, gb


def _assert_same(got, want):
    for name, a, b in zip(("grad_x", "grad_W", "grad_alpha_pre", "grad_alpha_post", "grad_alpha_res", "grad_bias"),
                          got, want):
        assert torch.equal(a, b), f"{name}: {int((a != b).sum())} of {a.numel()} differ"


# The threshold, a ragged last block, the metric width and its neighbours,
# C = 2560 (20 slices per stream, a team of 20 workgroups, 240 in all), and
# the narrowest rows (one and two slices per stream).
SHAPES = [(16384, 1024), (16390, 1024), (65536, 1024), (20000, 512), (16384, 2048), (16400, 4096),
          (32768, 2560), (16384, 128), (16387, 256)]


@pytest.mark.parametrize("gi", [False, True])
@pytest.mark.parametrize("T,C", SHAPES)
def test_split_equals_composed(split_lib, T, C, gi):
    case = _case(T, C, 7000 + T + C, gi)
    got = _split(split_lib, *case)
    want = _composed(*case)
    torch.cuda.synchronize()
    _assert_same(got, want)


@pytest.mark.parametrize("T,C", [(16390, 1024), (16400, 2048)])
def test_split_fallback_equals_composed(split_lib, T, C):
    """Every wave computes every block's grad_h_pre and grad_proj itself from
    HBM (no waiting on the team): the bounded waits' fallback gives the same
    bits."""
    case = _case(T, C, 7100 + T + C, True)
    old = os.environ.get("FLASH_MHC_SPLIT_SPIN")
    os.environ["FLASH_MHC_SPLIT_SPIN"] = "-1"
    try:
        got = _split(split_lib, *case)
        torch.cuda.synchronize()
    finally:
        if old is None:
            os.environ.pop("FLASH_MHC_SPLIT_SPIN", None)
        else:
            os.environ["FLASH_MHC_SPLIT_SPIN"] = old
    _assert_same(got, _composed(*case))


def test_split_repeatable_across_shapes(split_lib):
    """Calls of different sizes in a row (the exchange ring is zeroed by every
    call) and the same call twice give the same bits."""
    first = None
    for T, C in ((65536, 1024), (16390, 1024), (65536, 1024)):
        case = _case(T, C, 7200 + C, True)
        out = _split(split_lib, *case)
        torch.cuda.synchronize()
        if T == 65536:
            if first is None:
                first = [t.clone() for t in out]
            else:
                for a, b in zip(out, first):
                    assert torch.equal(a, b)


@pytest.mark.parametrize("T,C", [(65536, 1024), (16400, 4096)])
def test_product_equals_split(split_lib, T, C):
    """The product's pre-map backward (K3's reduce pass, K2, K1: two reads of
    x) gives the split kernel's bits."""
    case = _case(T, C, 7300 + C, True)
    x, W, p, hp, proj, inv, g_li, g_hq, g_H, g_in = case
    got = K.premap_bwd(x, W, *p, hp, proj, inv, g_li, g_hq, g_H, g_in)
    torch.cuda.synchronize()
    _assert_same(got, _split(split_lib, *case))
