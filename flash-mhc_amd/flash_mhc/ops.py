"""torch.library custom ops for the mHC-lite fused path, backed by gfx950 HIP.

The op namespace, names, schemas, FakeTensor behaviour and autograd formulas
are those of the reference (alint77/flash-mHC ``src/flash_mhc/ops.py``), so
``torch.ops.flash_mhc.*`` callers and ``torch.compile`` (which sees the ops as
opaque through their fakes) work unchanged.  Only the device implementation
differs: each "CUDA"-key impl validates its inputs and launches one HIP kernel
through the C ABI (:mod:`flash_mhc.kernels`).  There is no other backend: on a
tensor that is not on a GPU, or without the built extension, the ops raise.

Reference map:
  schemas                              ops.py:22-41
  fakes                                ops.py:145-202
  device impls                         ops.py:205-667
  autograd (setup_context + backward)  ops.py:670-714
  disable_autotune_temporarily         ops.py:44-58

Additions (not in the reference):
  fused_rmsnorm_project_bwd   grad_x and grad_W of K1 in one pass over x; the K1
                              autograd rule uses it unless FLASH_MHC_FUSED_DW=0,
                              which runs the reference's two-step rule (bwd_dx,
                              then a matmul for grad_W).
  mhc_coefficients (+ _backward)
                              K2, the coefficient math of block.py:161-170 and
                              the .float() casts of :176-177, as one kernel each
                              way, with the reference's bf16 rounding points.
                              MHCLiteBlock uses it unless FLASH_MHC_FUSED_K2=0.
  mhc_pre_map (+ _backward)   the pre-map region (K1, K2, K3 of block.py:157-177)
                              as one op: the forward runs the K1, K2 and K3
                              kernels; the backward runs K3's reduction, K2 and
                              K1 (with grad_W) and returns one grad_x.  MHCLiteBlock uses it unless
                              FLASH_MHC_FUSED_PREMAP=0 (or FLASH_MHC_FUSED_K2=0).
"""

from __future__ import annotations

import os
from contextlib import contextmanager

import torch
import torch.library

from . import kernels as _k

_lib = torch.library.Library("flash_mhc", "DEF")

_lib.define(
    "fused_rmsnorm_project(Tensor x_flat, Tensor W) -> (Tensor out, Tensor inv_rms)"
)
_lib.define(
    "fused_rmsnorm_project_bwd_dx(Tensor grad_out, Tensor x_flat, Tensor W, Tensor proj_out, Tensor inv_rms) -> Tensor grad_x"
)

# Not in the reference: K1's x- and W-gradient in one pass over x (the
# reference's autograd rule computes grad_W with a second matmul over x).
_lib.define(
    "fused_rmsnorm_project_bwd(Tensor grad_out, Tensor x_flat, Tensor W, Tensor proj_out, Tensor inv_rms) -> (Tensor grad_x, Tensor grad_W)"
)

# Not in the reference: K2 as one op (block.py:161-170 of the reference is a
# chain of ~15 PyTorch ops).  Outputs are the fp32 casts K3/K4 consume.
_lib.define(
    "mhc_coefficients(Tensor proj, Tensor alpha_pre, Tensor alpha_post, Tensor alpha_res, Tensor bias, Tensor perm_mat) -> (Tensor h_pre, Tensor h_post, Tensor H_merged)"
)
_lib.define(
    "mhc_coefficients_backward(Tensor? grad_h_pre, Tensor? grad_h_post, Tensor? grad_H_merged, Tensor proj, Tensor alpha_pre, Tensor alpha_post, Tensor alpha_res, Tensor bias, Tensor perm_mat) -> (Tensor grad_proj, Tensor grad_alpha_pre, Tensor grad_alpha_post, Tensor grad_alpha_res, Tensor grad_bias)"
)

# Not in the reference: the pre-map region (K1 + K2 + K3) as one op.
# x_sink is a (T, n, C) placeholder with zero strides (one element of storage)
# that stands for x: passed to mhc_post_res in place of a second use of x, it
# brings post-res's x-gradient back into this op's backward, which adds it in
# K1's store instead of leaving autograd a separate accumulation pass.
_lib.define(
    "mhc_pre_map(Tensor x_streams, Tensor W, Tensor alpha_pre, Tensor alpha_post, Tensor alpha_res, Tensor bias, Tensor perm_mat) -> (Tensor layer_input, Tensor H_merged, Tensor h_post, Tensor h_pre, Tensor proj, Tensor inv_rms, Tensor x_sink)"
)
_lib.define(
    "mhc_pre_map_backward(Tensor? grad_layer_input, Tensor? grad_H_merged, Tensor? grad_h_post, Tensor? grad_h_pre, Tensor? grad_proj, Tensor? grad_x_sink, Tensor x_streams, Tensor W, Tensor alpha_pre, Tensor alpha_post, Tensor alpha_res, Tensor bias, Tensor perm_mat, Tensor h_pre, Tensor proj, Tensor inv_rms) -> (Tensor grad_x, Tensor grad_W, Tensor grad_alpha_pre, Tensor grad_alpha_post, Tensor grad_alpha_res, Tensor grad_bias)"
)
# Not in the reference: mhc_pre_map in two ops, so that activation
# checkpointing can recompute K3 alone (the layer input is the one large
# tensor of the region; K1's and K2's outputs are 84 bytes per token).
# mhc_pre_map_coeffs runs K1 + K2 and returns, besides x_sink, li_sink: a
# zero-stride (T, C) placeholder passed to mhc_pre_map_mix (K3).  mix's
# backward hands the layer input's gradient to li_sink unchanged, and
# mhc_pre_map_coeffs's backward is mhc_pre_map's fused backward.
_lib.define(
    "mhc_pre_map_coeffs(Tensor x_streams, Tensor W, Tensor alpha_pre, Tensor alpha_post, Tensor alpha_res, Tensor bias, Tensor perm_mat) -> (Tensor H_merged, Tensor h_post, Tensor h_pre, Tensor proj, Tensor inv_rms, Tensor x_sink, Tensor li_sink)"
)
_lib.define("mhc_pre_map_mix(Tensor x_streams, Tensor h_pre, Tensor li_sink) -> Tensor layer_input")
# Not in the reference: fused_post_res whose x-gradient goes to x_sink (an
# output of mhc_pre_map for the same x) instead of x.  Same forward.
_lib.define(
    "mhc_post_res(Tensor x_streams, Tensor x_sink, Tensor layer_output, Tensor H_merged, Tensor h_post) -> Tensor out"
)

_lib.define("fused_pre_map(Tensor x_streams, Tensor h_pre) -> Tensor out")
_lib.define(
    "fused_pre_map_backward(Tensor grad_out, Tensor x_streams, Tensor h_pre) -> (Tensor grad_x, Tensor grad_h_pre)"
)

_lib.define(
    "fused_post_res(Tensor x_streams, Tensor layer_output, Tensor H_merged, Tensor h_post) -> Tensor out"
)
_lib.define(
    "fused_post_res_backward(Tensor grad_out, Tensor x_streams, Tensor layer_output, Tensor H_merged, Tensor h_post) -> (Tensor grad_x, Tensor grad_layer_output, Tensor grad_H_merged, Tensor grad_h_post)"
)


# ---------------------------------------------------------------------------
# Launch-configuration control.  The reference switches Triton autotuning off
# inside this context manager (ops.py:44-63); the HIP kernels have one fixed
# gfx950 configuration per shape class, so here it does nothing.  It stays
# for callers that enter it (MHCLiteBlock does in eval mode).


@contextmanager
def disable_autotune_temporarily():
    """Kept for API compatibility; launch configurations are fixed."""
    yield


# ---------------------------------------------------------------------------
# Fake (meta) implementations: output shapes/dtypes only (ops.py:145-202).

@torch.library.register_fake("flash_mhc::fused_rmsnorm_project")
def _fused_rmsnorm_project_fake(x_flat: torch.Tensor, W: torch.Tensor):
    T = x_flat.shape[0]
    D_out = W.shape[0]
    out = torch.empty((T, D_out), device=x_flat.device, dtype=x_flat.dtype)
    inv_rms = torch.empty((T,), device=x_flat.device, dtype=torch.float32)
    return out, inv_rms


@torch.library.register_fake("flash_mhc::fused_rmsnorm_project_bwd_dx")
def _fused_rmsnorm_project_bwd_dx_fake(grad_out, x_flat, W, proj_out, inv_rms):
    return torch.empty_like(x_flat)


@torch.library.register_fake("flash_mhc::fused_rmsnorm_project_bwd")
def _fused_rmsnorm_project_bwd_fake(grad_out, x_flat, W, proj_out, inv_rms):
    return torch.empty_like(x_flat), torch.empty_like(W, dtype=x_flat.dtype)


@torch.library.register_fake("flash_mhc::mhc_coefficients")
def _mhc_coefficients_fake(proj, alpha_pre, alpha_post, alpha_res, bias, perm_mat):
    T = proj.shape[0]
    n = int(round(perm_mat.shape[1] ** 0.5))
    h_pre = proj.new_empty((T, n), dtype=torch.float32)
    h_post = proj.new_empty((T, n), dtype=torch.float32)
    H_merged = proj.new_empty((T, n, n), dtype=torch.float32)
    return h_pre, h_post, H_merged


@torch.library.register_fake("flash_mhc::mhc_coefficients_backward")
def _mhc_coefficients_backward_fake(grad_h_pre, grad_h_post, grad_H_merged, proj, alpha_pre,
                                    alpha_post, alpha_res, bias, perm_mat):
    return (torch.empty_like(proj), torch.empty_like(alpha_pre), torch.empty_like(alpha_post),
            torch.empty_like(alpha_res), torch.empty_like(bias))


def x_sink_like(x_streams: torch.Tensor) -> torch.Tensor:
    """mhc_pre_map's x_sink: x's shape and dtype, zero strides, one element of storage."""
    return x_streams.new_empty_strided(tuple(x_streams.shape), (0,) * x_streams.dim())


@torch.library.register_fake("flash_mhc::mhc_pre_map")
def _mhc_pre_map_fake(x_streams, W, alpha_pre, alpha_post, alpha_res, bias, perm_mat):
    T, n, C = x_streams.shape
    f32 = torch.float32
    return (x_streams.new_empty((T, C)), x_streams.new_empty((T, n, n), dtype=f32),
            x_streams.new_empty((T, n), dtype=f32), x_streams.new_empty((T, n), dtype=f32),
            x_streams.new_empty((T, W.shape[0])), x_streams.new_empty((T,), dtype=f32),
            x_sink_like(x_streams))


@torch.library.register_fake("flash_mhc::mhc_pre_map_coeffs")
def _mhc_pre_map_coeffs_fake(x_streams, W, alpha_pre, alpha_post, alpha_res, bias, perm_mat):
    T, n, C = x_streams.shape
    f32 = torch.float32
    return (x_streams.new_empty((T, n, n), dtype=f32), x_streams.new_empty((T, n), dtype=f32),
            x_streams.new_empty((T, n), dtype=f32), x_streams.new_empty((T, W.shape[0])),
            x_streams.new_empty((T,), dtype=f32), x_sink_like(x_streams),
            x_streams.new_empty_strided((T, C), (0, 0)))


@torch.library.register_fake("flash_mhc::mhc_pre_map_mix")
def _mhc_pre_map_mix_fake(x_streams, h_pre, li_sink):
    T, n, C = x_streams.shape
    return x_streams.new_empty((T, C))


@torch.library.register_fake("flash_mhc::mhc_pre_map_backward")
def _mhc_pre_map_backward_fake(grad_layer_input, grad_H_merged, grad_h_post, grad_h_pre, grad_proj,
                               grad_x_sink, x_streams, W, alpha_pre, alpha_post, alpha_res, bias,
                               perm_mat, h_pre, proj, inv_rms):
    return (torch.empty_like(x_streams), torch.empty_like(W), torch.empty_like(alpha_pre),
            torch.empty_like(alpha_post), torch.empty_like(alpha_res), torch.empty_like(bias))


@torch.library.register_fake("flash_mhc::fused_pre_map")
def _fused_pre_map_fake(x_streams: torch.Tensor, h_pre: torch.Tensor):
    T, _, C = x_streams.shape
    return torch.empty((T, C), device=x_streams.device, dtype=x_streams.dtype)


@torch.library.register_fake("flash_mhc::fused_pre_map_backward")
def _fused_pre_map_backward_fake(grad_out, x_streams, h_pre):
    grad_x = torch.empty_like(x_streams)
    grad_h_pre = torch.empty_like(h_pre, dtype=torch.float32)
    return grad_x, grad_h_pre


@torch.library.register_fake("flash_mhc::mhc_post_res")
def _mhc_post_res_fake(x_streams, x_sink, layer_output, H_merged, h_post):
    return torch.empty_like(x_streams)


@torch.library.register_fake("flash_mhc::fused_post_res")
def _fused_post_res_fake(x_streams, layer_output, H_merged, h_post):
    return torch.empty_like(x_streams)


@torch.library.register_fake("flash_mhc::fused_post_res_backward")
def _fused_post_res_backward_fake(grad_out, x_streams, layer_output, H_merged, h_post):
    grad_x = torch.empty_like(x_streams)
    grad_layer_output = torch.empty_like(layer_output)
    grad_H_merged = torch.empty_like(H_merged, dtype=torch.float32)
    grad_h_post = torch.empty_like(h_post, dtype=torch.float32)
    return grad_x, grad_layer_output, grad_H_merged, grad_h_post


# ---------------------------------------------------------------------------
# Device implementations (GPU tensors -> HIP kernels).


def _check_n4(x_streams: torch.Tensor, message: str) -> None:
    # Same errors as the reference (ops.py:352-353, 424-425, 506-507, 581-582).
    if x_streams.dim() != 3:
        raise ValueError(f"x_streams must have shape (T, n, C), got {tuple(x_streams.shape)}")
    if x_streams.shape[1] != 4:
        raise ValueError(message)


def _coeff(t: torch.Tensor) -> torch.Tensor:
    # The reference kernels upcast whatever coefficient dtype they receive.
    return t.to(torch.float32).contiguous()


def _params(*ts: torch.Tensor):
    """K2's parameters (alphas, bias, perm) as the kernels take them: in their
    own dtype when all are fp32 or all bf16 (no conversion launches), else fp32."""
    dt = ts[0].dtype
    if dt is torch.float32 or dt is torch.bfloat16:
        if all(t.dtype is dt and t.is_contiguous() for t in ts):
            return ts
        if all(t.dtype is dt for t in ts):
            return [t.contiguous() for t in ts]
    return [_coeff(t) for t in ts]


@torch.library.impl(_lib, "fused_rmsnorm_project", "CUDA")
def _fused_rmsnorm_project_cuda(x_flat: torch.Tensor, W: torch.Tensor):
    return _k.k1_fwd(x_flat.contiguous(), W.contiguous())


@torch.library.impl(_lib, "fused_rmsnorm_project_bwd_dx", "CUDA")
def _fused_rmsnorm_project_bwd_dx_cuda(grad_out, x_flat, W, proj_out, inv_rms):
    return _k.k1_bwd_dx(grad_out.contiguous(), x_flat.contiguous(), W.contiguous(),
                        proj_out.contiguous(), inv_rms.contiguous())


@torch.library.impl(_lib, "fused_rmsnorm_project_bwd", "CUDA")
def _fused_rmsnorm_project_bwd_cuda(grad_out, x_flat, W, proj_out, inv_rms):
    return _k.k1_bwd(grad_out.contiguous(), x_flat.contiguous(), W.to(x_flat.dtype).contiguous(),
                     proj_out.contiguous(), inv_rms.contiguous())


def _check_k2(proj: torch.Tensor, perm_mat: torch.Tensor) -> None:
    _check_k2_shapes(tuple(proj.shape), perm_mat)


def _check_k2_shapes(proj_shape: tuple, perm_mat: torch.Tensor) -> None:
    if len(proj_shape) != 2 or proj_shape[1] != 32 or tuple(perm_mat.shape) != (24, 16):
        raise ValueError(
            "flash_mhc::mhc_coefficients supports n=4 only: proj must be (T, 32) and "
            f"perm_mat (24, 16), got {tuple(proj_shape)} and {tuple(perm_mat.shape)}"
        )


@torch.library.impl(_lib, "mhc_coefficients", "CUDA")
def _mhc_coefficients_cuda(proj, alpha_pre, alpha_post, alpha_res, bias, perm_mat):
    _check_k2(proj, perm_mat)
    return _k.k2_fwd(proj.contiguous(), *_params(alpha_pre, alpha_post, alpha_res, bias, perm_mat))


@torch.library.impl(_lib, "mhc_coefficients_backward", "CUDA")
def _mhc_coefficients_backward_cuda(grad_h_pre, grad_h_post, grad_H_merged, proj, alpha_pre,
                                    alpha_post, alpha_res, bias, perm_mat):
    _check_k2(proj, perm_mat)
    g = [None if t is None else _coeff(t) for t in (grad_h_pre, grad_h_post, grad_H_merged)]
    gp, ga1, ga2, ga3, gb = _k.k2_bwd(proj.contiguous(), *_params(alpha_pre, alpha_post, alpha_res, bias,
                                                                 perm_mat), *g)
    # Parameter gradients in the parameters' dtype (exact: the values are bf16).
    return (gp, ga1.to(alpha_pre.dtype), ga2.to(alpha_post.dtype), ga3.to(alpha_res.dtype),
            gb.to(bias.dtype))


@torch.library.impl(_lib, "mhc_pre_map", "CUDA")
def _mhc_pre_map_cuda(x_streams, W, alpha_pre, alpha_post, alpha_res, bias, perm_mat):
    _check_n4(x_streams, "flash_mhc::mhc_pre_map supports n=4 only")
    _check_k2_shapes((0, W.shape[0]), perm_mat)
    # The sink's one element is zeroed by the same launches (no fill kernel).
    x_sink = x_sink_like(x_streams)
    outs = _k.premap_fwd(x_streams.contiguous(), W.to(x_streams.dtype).contiguous(),
                         *_params(alpha_pre, alpha_post, alpha_res, bias, perm_mat), zero=(x_sink,))
    return (*outs, x_sink)


def pre_map_nograd(x_streams, W, alpha_pre, alpha_post, alpha_res, bias, perm_mat):
    """(layer_input, coeffs) of mhc_pre_map without the op's dispatch, for
    forwards that record no autograd graph: the same kernels and conversions
    as the op's device implementation, so the same values; coeffs holds
    H_merged and h_post for post_res_nograd (kernels.premap_fwd_eval)."""
    if x_streams.dim() != 3 or x_streams.shape[1] != 4:
        _check_n4(x_streams, "flash_mhc::mhc_pre_map supports n=4 only")
    if W.dim() != 2 or W.shape[0] != 32 or perm_mat.shape != (24, 16):
        _check_k2_shapes((0, W.shape[0]), perm_mat)
    # The op's conversions, skipped where they would return the tensor itself.
    if not x_streams.is_contiguous():
        x_streams = x_streams.contiguous()
    if W.dtype is not x_streams.dtype:
        W = W.to(x_streams.dtype)
    if not W.is_contiguous():
        W = W.contiguous()
    return _k.premap_fwd_eval(x_streams, W, *_params(alpha_pre, alpha_post, alpha_res, bias, perm_mat))


def post_res_nograd(x_streams, layer_output, coeffs):
    """fused_post_res's device implementation without the op's dispatch, for
    the coeffs of pre_map_nograd of the same x_streams."""
    if x_streams.dim() != 3 or x_streams.shape[1] != 4:
        _check_n4(x_streams, "flash_mhc::fused_post_res currently supports n=4 only")
    if not x_streams.is_contiguous():
        x_streams = x_streams.contiguous()
    if not layer_output.is_contiguous():
        layer_output = layer_output.contiguous()
    return _k.k4_fwd_eval(x_streams, layer_output, coeffs)


@torch.library.impl(_lib, "mhc_pre_map_coeffs", "CUDA")
def _mhc_pre_map_coeffs_cuda(x_streams, W, alpha_pre, alpha_post, alpha_res, bias, perm_mat):
    _check_n4(x_streams, "flash_mhc::mhc_pre_map_coeffs supports n=4 only")
    _check_k2_shapes((0, W.shape[0]), perm_mat)
    T, n, C = x_streams.shape
    x_sink = x_sink_like(x_streams)
    li_sink = x_streams.new_empty_strided((T, C), (0, 0))
    _li, H, h_post, h_pre, proj, inv = _k.premap_fwd(
        x_streams.contiguous(), W.to(x_streams.dtype).contiguous(),
        *_params(alpha_pre, alpha_post, alpha_res, bias, perm_mat), layer_input=False, zero=(x_sink, li_sink))
    return H, h_post, h_pre, proj, inv, x_sink, li_sink


@torch.library.impl(_lib, "mhc_pre_map_mix", "CUDA")
def _mhc_pre_map_mix_cuda(x_streams, h_pre, li_sink):
    _check_n4(x_streams, "flash_mhc::mhc_pre_map_mix supports n=4 only")
    return _k.k3_fwd(x_streams.contiguous(), _coeff(h_pre))


@torch.library.impl(_lib, "mhc_pre_map_backward", "CUDA")
def _mhc_pre_map_backward_cuda(grad_layer_input, grad_H_merged, grad_h_post, grad_h_pre, grad_proj,
                               grad_x_sink, x_streams, W, alpha_pre, alpha_post, alpha_res, bias,
                               perm_mat, h_pre, proj, inv_rms):
    _check_n4(x_streams, "flash_mhc::mhc_pre_map_backward supports n=4 only")
    x = x_streams.contiguous()
    T, n, C = x.shape
    Wc = W.to(x.dtype).contiguous()
    coeffs = _params(alpha_pre, alpha_post, alpha_res, bias, perm_mat)
    g_li = (torch.zeros((T, C), device=x.device, dtype=x.dtype) if grad_layer_input is None
            else grad_layer_input.to(x.dtype).contiguous())
    g_hp = None if grad_h_post is None else _coeff(grad_h_post)
    g_H = None if grad_H_merged is None else _coeff(grad_H_merged)
    g_sink = None if grad_x_sink is None else grad_x_sink.to(x.dtype).contiguous()
    if grad_h_pre is None and grad_proj is None:
        # One launch sequence: K3's reduction, K2, K1 with K3's term (and the
        # sink's gradient) in its store.
        gx, gW, ga1, ga2, ga3, gb = _k.premap_bwd(x, Wc, *coeffs, h_pre.contiguous(), proj.contiguous(),
                                                  inv_rms.contiguous(), g_li, g_hp, g_H, g_sink)
    else:
        # Gradients also flow into the h_pre / proj outputs: compose the ops.
        gx3, gh = _k.k3_bwd(g_li, x, h_pre.contiguous())
        if grad_h_pre is not None:
            gh = gh + grad_h_pre.float()
        gp, ga1, ga2, ga3, gb = _k.k2_bwd(proj.contiguous(), *coeffs, gh, g_hp, g_H)
        if grad_proj is not None:
            gp = (gp.float() + grad_proj.float()).to(gp.dtype)
        gx1, gW = _k.k1_bwd(gp, x.view(T, n * C), Wc, proj.contiguous(), inv_rms.contiguous())
        gx = gx3 + gx1.view(T, n, C)
        if g_sink is not None:
            gx = g_sink + gx
    return (gx, gW.to(W.dtype), ga1.to(alpha_pre.dtype), ga2.to(alpha_post.dtype),
            ga3.to(alpha_res.dtype), gb.to(bias.dtype))


@torch.library.impl(_lib, "fused_pre_map", "CUDA")
def _fused_pre_map_cuda(x_streams: torch.Tensor, h_pre: torch.Tensor):
    _check_n4(x_streams, "flash_mhc::fused_pre_map currently supports n=4 only")
    return _k.k3_fwd(x_streams.contiguous(), _coeff(h_pre))


@torch.library.impl(_lib, "fused_pre_map_backward", "CUDA")
def _fused_pre_map_backward_cuda(grad_out, x_streams, h_pre):
    _check_n4(x_streams, "flash_mhc::fused_pre_map_backward supports n=4 only")
    return _k.k3_bwd(grad_out.contiguous(), x_streams.contiguous(), _coeff(h_pre))


@torch.library.impl(_lib, "fused_post_res", "CUDA")
def _fused_post_res_cuda(x_streams, layer_output, H_merged, h_post):
    _check_n4(x_streams, "flash_mhc::fused_post_res currently supports n=4 only")
    return _k.k4_fwd(x_streams.contiguous(), layer_output.contiguous(), _coeff(H_merged),
                     _coeff(h_post))


@torch.library.impl(_lib, "mhc_post_res", "CUDA")
def _mhc_post_res_cuda(x_streams, x_sink, layer_output, H_merged, h_post):
    _check_n4(x_streams, "flash_mhc::mhc_post_res supports n=4 only")
    return _k.k4_fwd(x_streams.contiguous(), layer_output.contiguous(), _coeff(H_merged),
                     _coeff(h_post))


@torch.library.impl(_lib, "fused_post_res_backward", "CUDA")
def _fused_post_res_backward_cuda(grad_out, x_streams, layer_output, H_merged, h_post):
    _check_n4(x_streams, "flash_mhc::fused_post_res_backward supports n=4 only")
    return _k.k4_bwd(grad_out.contiguous(), x_streams.contiguous(), layer_output.contiguous(),
                     _coeff(H_merged), _coeff(h_post))


# ---------------------------------------------------------------------------
# Autograd (ops.py:670-714).  The formulas are the reference's; each op saves
# only the tensors its backward reads (the reference also saves the K3/K4
# outputs, which its backward never uses).


def _setup_k1(ctx, inputs, output):
    x_flat, W = inputs
    out, inv_rms = output
    ctx.save_for_backward(x_flat, W, out, inv_rms)


_OFF = frozenset({"0", "false", "off", "no"})


def _env_flag(name: str) -> bool:
    v = os.environ.get(name)
    return v is None or v.strip().lower() not in _OFF


def _fused_dw_enabled() -> bool:
    return _env_flag("FLASH_MHC_FUSED_DW")


def fused_k2_enabled() -> bool:
    """MHCLiteBlock runs K2 as flash_mhc::mhc_coefficients unless FLASH_MHC_FUSED_K2=0."""
    return _env_flag("FLASH_MHC_FUSED_K2")


def fused_premap_enabled() -> bool:
    """MHCLiteBlock runs K1 + K2 + K3 as flash_mhc::mhc_pre_map unless
    FLASH_MHC_FUSED_PREMAP=0 or FLASH_MHC_FUSED_K2=0."""
    return _env_flag("FLASH_MHC_FUSED_PREMAP") and fused_k2_enabled()


def fused_xgrad_flag() -> bool:
    """FLASH_MHC_FUSED_XGRAD alone (callers that already know the pre-map op is on)."""
    return _env_flag("FLASH_MHC_FUSED_XGRAD")


def fused_xgrad_enabled() -> bool:
    """With the pre-map op, MHCLiteBlock sends post-res's x-gradient through
    mhc_pre_map's x_sink (added in K1's store) unless FLASH_MHC_FUSED_XGRAD=0."""
    return fused_xgrad_flag() and fused_premap_enabled()


def _fused_rmsnorm_project_backward(ctx, grad_out, grad_inv_rms):
    # inv_rms is treated as non-differentiable, as in the reference.
    x_flat, W, proj_out, inv_rms = ctx.saved_tensors
    if _fused_dw_enabled():
        # Same gradients as the two-step rule below, computed in one pass over x.
        grad_x, grad_W = torch.ops.flash_mhc.fused_rmsnorm_project_bwd(
            grad_out, x_flat, W, proj_out, inv_rms
        )
        return grad_x, grad_W
    grad_x = torch.ops.flash_mhc.fused_rmsnorm_project_bwd_dx(
        grad_out, x_flat, W, proj_out, inv_rms
    )
    grad_out_scaled = (grad_out * inv_rms[:, None]).to(x_flat.dtype)
    grad_W = torch.matmul(grad_out_scaled.transpose(0, 1).contiguous(), x_flat)
    return grad_x, grad_W


def _setup_inputs(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _mhc_coefficients_backward(ctx, grad_h_pre, grad_h_post, grad_H_merged):
    # The backward recomputes the chain from proj (64 bytes per token).
    proj, alpha_pre, alpha_post, alpha_res, bias, perm_mat = ctx.saved_tensors
    grads = torch.ops.flash_mhc.mhc_coefficients_backward(
        grad_h_pre, grad_h_post, grad_H_merged, proj, alpha_pre, alpha_post, alpha_res, bias, perm_mat
    )
    return (*grads, None)


def _fused_pre_map_backward(ctx, grad_out):
    x_streams, h_pre = ctx.saved_tensors
    return torch.ops.flash_mhc.fused_pre_map_backward(grad_out, x_streams, h_pre)


def _fused_post_res_backward(ctx, grad_out):
    x_streams, layer_output, H_merged, h_post = ctx.saved_tensors
    return torch.ops.flash_mhc.fused_post_res_backward(
        grad_out, x_streams, layer_output, H_merged, h_post
    )


torch.library.register_autograd(
    "flash_mhc::fused_rmsnorm_project",
    _fused_rmsnorm_project_backward,
    setup_context=_setup_k1,
)
torch.library.register_autograd(
    "flash_mhc::mhc_coefficients",
    _mhc_coefficients_backward,
    setup_context=_setup_inputs,
)
def _setup_pre_map(ctx, inputs, output):
    _li, _H, _hp, h_pre, proj, inv_rms, _sink = output
    ctx.save_for_backward(*inputs, h_pre, proj, inv_rms)
    # Outputs nobody differentiates (h_pre, proj, inv_rms in the block) arrive
    # as None rather than as zero tensors.
    ctx.set_materialize_grads(False)


def _mhc_pre_map_backward(ctx, g_li, g_H, g_hp, g_hpre, g_proj, _g_inv_rms, g_sink):
    # inv_rms is not differentiable, as K1's in the reference.
    x, W, ap, apo, ar, b, perm, h_pre, proj, inv_rms = ctx.saved_tensors
    grads = torch.ops.flash_mhc.mhc_pre_map_backward(
        g_li, g_H, g_hp, g_hpre, g_proj, g_sink, x, W, ap, apo, ar, b, perm, h_pre, proj, inv_rms
    )
    return (*grads, None)


def _mhc_post_res_backward(ctx, grad_out):
    x_streams, _sink, layer_output, H_merged, h_post = ctx.saved_tensors
    g_x, g_lo, g_H, g_hp = torch.ops.flash_mhc.fused_post_res_backward(
        grad_out, x_streams, layer_output, H_merged, h_post
    )
    # x's gradient goes to the sink; mhc_pre_map's backward adds it to x's.
    return None, g_x, g_lo, g_H, g_hp


torch.library.register_autograd(
    "flash_mhc::mhc_pre_map",
    _mhc_pre_map_backward,
    setup_context=_setup_pre_map,
)


class _PreMapEager(torch.autograd.Function):
    """mhc_pre_map with its registered autograd, without the op's dispatch,
    for eager forwards that record an autograd graph: forward and backward
    call the op's device implementations (_mhc_pre_map_cuda,
    _mhc_pre_map_backward_cuda), so the values, the saved tensors and the
    x_sink contract are the op's.  Returns (layer_input, H_merged, h_post,
    x_sink); h_pre, proj and inv_rms stay internal (the block does not
    differentiate them)."""

    @staticmethod
    def forward(ctx, x_streams, W, alpha_pre, alpha_post, alpha_res, bias, perm_mat):
        li, H, hq, h_pre, proj, inv_rms, x_sink = _mhc_pre_map_cuda(x_streams, W, alpha_pre, alpha_post,
                                                                     alpha_res, bias, perm_mat)
        ctx.save_for_backward(x_streams, W, alpha_pre, alpha_post, alpha_res, bias, perm_mat, h_pre, proj, inv_rms)
        ctx.set_materialize_grads(False)
        return li, H, hq, x_sink

    @staticmethod
    def backward(ctx, g_li, g_H, g_hp, g_sink):
        x, W, ap, apo, ar, b, perm, h_pre, proj, inv_rms = ctx.saved_tensors
        grads = _mhc_pre_map_backward_cuda(g_li, g_H, g_hp, None, None, g_sink, x, W, ap, apo, ar, b, perm,
                                           h_pre, proj, inv_rms)
        return (*grads, None)


class _PostResEager(torch.autograd.Function):
    """mhc_post_res with its registered autograd, without the op's dispatch
    (see _PreMapEager): x's gradient goes to x_sink."""

    @staticmethod
    def forward(ctx, x_streams, x_sink, layer_output, H_merged, h_post):
        out = _mhc_post_res_cuda(x_streams, x_sink, layer_output, H_merged, h_post)
        ctx.save_for_backward(x_streams, layer_output, H_merged, h_post)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x_streams, layer_output, H_merged, h_post = ctx.saved_tensors
        g_x, g_lo, g_H, g_hp = _fused_post_res_backward_cuda(grad_out, x_streams, layer_output, H_merged, h_post)
        return None, g_x, g_lo, g_H, g_hp


def pre_map_eager(x_streams, W, alpha_pre, alpha_post, alpha_res, bias, perm_mat):
    """(layer_input, H_merged, h_post, x_sink) of mhc_pre_map, recorded for
    autograd without the op's dispatch (eager training forwards)."""
    return _PreMapEager.apply(x_streams, W, alpha_pre, alpha_post, alpha_res, bias, perm_mat)


def post_res_eager(x_streams, x_sink, layer_output, H_merged, h_post):
    """mhc_post_res, recorded for autograd without the op's dispatch."""
    return _PostResEager.apply(x_streams, x_sink, layer_output, H_merged, h_post)


def _setup_pre_map_coeffs(ctx, inputs, output):
    _H, _hp, h_pre, proj, inv_rms, _xs, _ls = output
    ctx.save_for_backward(*inputs, h_pre, proj, inv_rms)
    ctx.set_materialize_grads(False)


def _mhc_pre_map_coeffs_backward(ctx, g_H, g_hp, g_hpre, g_proj, _g_inv_rms, g_xsink, g_lisink):
    # g_lisink is the layer input's gradient, handed over by mhc_pre_map_mix.
    x, W, ap, apo, ar, b, perm, h_pre, proj, inv_rms = ctx.saved_tensors
    grads = torch.ops.flash_mhc.mhc_pre_map_backward(
        g_lisink, g_H, g_hp, g_hpre, g_proj, g_xsink, x, W, ap, apo, ar, b, perm, h_pre, proj, inv_rms
    )
    return (*grads, None)


def _mhc_pre_map_mix_backward(ctx, g_li):
    # K3's gradients with respect to x and h_pre are formed in
    # mhc_pre_map_coeffs's backward from the layer input's gradient.
    return None, None, g_li


torch.library.register_autograd(
    "flash_mhc::mhc_pre_map_coeffs",
    _mhc_pre_map_coeffs_backward,
    setup_context=_setup_pre_map_coeffs,
)
torch.library.register_autograd(
    "flash_mhc::mhc_pre_map_mix",
    _mhc_pre_map_mix_backward,
    setup_context=lambda ctx, inputs, output: None,
)
torch.library.register_autograd(
    "flash_mhc::fused_pre_map",
    _fused_pre_map_backward,
    setup_context=_setup_inputs,
)
torch.library.register_autograd(
    "flash_mhc::fused_post_res",
    _fused_post_res_backward,
    setup_context=_setup_inputs,
)
torch.library.register_autograd(
    "flash_mhc::mhc_post_res",
    _mhc_post_res_backward,
    setup_context=_setup_inputs,
)
