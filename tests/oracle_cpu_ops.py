"""Test-only CPU kernels for the flash_mhc ops, computed by the oracle.

The product registers device ("CUDA"-key) implementations only.  To test the
op *contract* without a GPU (schemas, fakes, autograd registration,
torch.library.opcheck, torch.compile tracing), these helpers temporarily
register CPU kernels that evaluate the oracle's float64 formulas and round
once to the op's output dtype.  The registration lives in a context manager
and is removed on exit; GPU tensors never dispatch to it.
"""

from __future__ import annotations

from contextlib import contextmanager

import numpy as np
import torch

from oracle import k2_oracle as K2O
from oracle import mhc_oracle as O

BF16 = torch.bfloat16


def _k1(x_flat, W):
    R, _, inv = O.k1_fwd(x_flat, W)
    return R.to(x_flat.dtype), inv.to(torch.float32)


def _k1_bwd_dx(grad_out, x_flat, W, proj_out, inv_rms):
    R, _ = O.k1_bwd_dx(grad_out, x_flat, W, proj_out, inv_rms)
    return R.to(x_flat.dtype)


def _k1_bwd(grad_out, x_flat, W, proj_out, inv_rms):
    gx, _ = O.k1_bwd_dx(grad_out, x_flat, W, proj_out, inv_rms)
    gW, _ = O.k1_grad_W(grad_out, x_flat, inv_rms)
    return gx.to(x_flat.dtype), gW.to(x_flat.dtype)


def _k2(proj, ap, apo, ar, b, perm):
    f = K2O.k2_fwd(proj, ap, apo, ar, b, perm)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    return t(f["h_pre"]), t(f["h_post"]), t(f["H_merged"])


def _k2_bwd(g_hpre, g_hpost, g_H, proj, ap, apo, ar, b, perm):
    r = K2O.k2_bwd(proj, ap, apo, ar, b, perm, g_hpre, g_hpost, g_H)
    gp = torch.from_numpy(np.ascontiguousarray(r["grad_proj"])).to(proj.dtype)

    def par(key, like):
        R = torch.as_tensor(r[key][0], dtype=torch.float64).reshape(like.shape)
        return R.float().to(torch.bfloat16).to(like.dtype)

    return (gp, par("grad_alpha_pre", ap), par("grad_alpha_post", apo), par("grad_alpha_res", ar),
            par("grad_bias", b))


def _pre_map(x, W, ap, apo, ar, b, perm):
    T, n, C = x.shape
    proj, inv = _k1(x.reshape(T, n * C), W.to(x.dtype))
    h_pre, h_post, H = _k2(proj, ap, apo, ar, b, perm)
    sink = x.new_empty_strided(tuple(x.shape), (0,) * x.dim())  # mhc_pre_map's x_sink
    if sink.numel() > 0:
        sink.as_strided((1,), (1,)).zero_()
    return _k3(x, h_pre), H, h_post, h_pre, proj, inv, sink


def _pre_map_coeffs(x, W, ap, apo, ar, b, perm):
    T, n, C = x.shape
    proj, inv = _k1(x.reshape(T, n * C), W.to(x.dtype))
    h_pre, h_post, H = _k2(proj, ap, apo, ar, b, perm)
    sinks = [x.new_empty_strided(shape, (0,) * len(shape)) for shape in (tuple(x.shape), (T, C))]
    for sink in sinks:  # x_sink and li_sink, one zeroed element each
        if sink.numel() > 0:
            sink.as_strided((1,), (1,)).zero_()
    return H, h_post, h_pre, proj, inv, sinks[0], sinks[1]


def _pre_map_mix(x, h_pre, li_sink):
    return _k3(x, h_pre)


def _pre_map_bwd(g_li, g_H, g_hp, g_hpre, g_proj, g_sink, x, W, ap, apo, ar, b, perm, h_pre, proj, inv):
    T, n, C = x.shape
    if g_li is None:
        g_li = torch.zeros(T, C, dtype=x.dtype)
    gx3, gh = _k3_bwd(g_li, x, h_pre)
    if g_hpre is not None:
        gh = gh + g_hpre.float()
    gp, ga1, ga2, ga3, gb = _k2_bwd(gh, g_hp, g_H, proj, ap, apo, ar, b, perm)
    if g_proj is not None:
        gp = (gp.float() + g_proj.float()).to(gp.dtype)
    gx1, gW = _k1_bwd(gp, x.reshape(T, n * C), W.to(x.dtype), proj, inv)
    gx = gx3 + gx1.view(T, n, C)
    if g_sink is not None:
        gx = g_sink.to(gx.dtype) + gx
    return gx, gW.to(W.dtype), ga1, ga2, ga3, gb


def _k3(x, h):
    if x.shape[1] != 4:
        raise ValueError("flash_mhc::fused_pre_map currently supports n=4 only")
    R, _ = O.k3_fwd(x, h)
    return R.to(x.dtype)


def _k3_bwd(go, x, h):
    gx, _, gh, _ = O.k3_bwd(go, x, h)
    return gx.to(x.dtype), gh.to(torch.float32)


def _k4(x, lo, H, hp):
    R, _ = O.k4_fwd(x, lo, H, hp)
    return R.to(x.dtype)


def _post_res_sink(x, sink, lo, H, hp):
    return _k4(x, lo, H, hp)


def _k4_bwd(go, x, lo, H, hp):
    r = O.k4_bwd(go, x, lo, H, hp)
    return (r["grad_x"][0].to(x.dtype), r["grad_lo"][0].to(lo.dtype),
            r["grad_H"][0].to(torch.float32), r["grad_hp"][0].to(torch.float32))


IMPLS = {
    "fused_rmsnorm_project": _k1,
    "fused_rmsnorm_project_bwd_dx": _k1_bwd_dx,
    "fused_rmsnorm_project_bwd": _k1_bwd,
    "mhc_coefficients": _k2,
    "mhc_coefficients_backward": _k2_bwd,
    "mhc_pre_map": _pre_map,
    "mhc_pre_map_backward": _pre_map_bwd,
    "mhc_pre_map_coeffs": _pre_map_coeffs,
    "mhc_pre_map_mix": _pre_map_mix,
    "fused_pre_map": _k3,
    "fused_pre_map_backward": _k3_bwd,
    "fused_post_res": _k4,
    "mhc_post_res": _post_res_sink,
    "fused_post_res_backward": _k4_bwd,
}


@contextmanager
def oracle_cpu_kernels():
    import flash_mhc  # noqa: F401  # the op schemas must exist first

    lib = torch.library.Library("flash_mhc", "IMPL")
    try:
        for name, fn in IMPLS.items():
            lib.impl(name, fn, "CPU")
        yield
    finally:
        lib._destroy()
