"""mHC-lite residual wrapper with the gfx950 HIP fused path.

``MHCLiteBlock`` keeps the reference's public surface
(alint77/flash-mHC ``src/flash_mhc/block.py``): constructor arguments,
attribute / parameter / buffer names and their registration order (hence the
``state_dict`` keys and the RNG draws at construction), the fused-path
predicate (``block.py:221-231``), the activation-checkpoint predicate
(``block.py:74-80``) and the method names ``_forward_pytorch`` /
``_forward_triton`` that callers use directly.

Per layer, with x of shape (T, n, C):
  K1  proj, inv_rms = rmsnorm-project(x.reshape(T, nC), W_all.weight)   HIP kernel
  K2  h_pre = sigmoid(a_pre * proj[:, :n] + b), h_post = 2 sigmoid(...),
      H_res = softmax(a_res * proj[:, 2n:] + b) @ perm, H_merged = H_res - h_post h_pre^T
                                                 HIP kernel (the reference's bf16 ops
                                                 with FLASH_MHC_FUSED_K2=0)
  K3  layer_input = sum_j h_pre[:, j] x[:, j]                             HIP kernel
      layer_output = layer(layer_input)                                  user module
  K4  out = H_merged @ x + h_post (x) layer_output                       HIP kernel

The fused path runs for GPU bf16 inputs of shape (T, 4, C); every other input
(other n, other dtypes, CPU tensors, extra leading dims) takes the plain
PyTorch formulation of the same block, as in the reference.
"""

from __future__ import annotations

import itertools
import math
from contextlib import nullcontext

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint as _checkpoint

from . import ops as _ops


def build_permutation_matrices(n: int) -> tuple[torch.Tensor, int]:
    """All n x n permutation matrices, flattened: shape (n!, n*n), values {0, 1}.

    Row m is the permutation number m of ``itertools.permutations(range(n))``
    (lexicographic order), with entry ``[m, i*n + j] = 1`` iff that permutation
    maps i to j.  Index 0 is the identity.  Same layout as the reference's
    ``build_permutation_matrices`` (block.py:21-32).
    """
    if n < 1:
        raise ValueError(f"n must be >= 1, got {n}")
    images = torch.tensor(list(itertools.permutations(range(n))), dtype=torch.long)
    mats = torch.zeros(images.shape[0], n, n)
    mats.scatter_(2, images.unsqueeze(-1), 1.0)
    return mats.reshape(images.shape[0], n * n), 0


def _private_probe(get):
    """A private torch query, or None where this torch build lacks it."""
    try:
        return get()
    except (AttributeError, ImportError):
        return None


# Two private torch queries the eager fast paths rely on.  Where a torch
# build lacks either, _plain_eager is always False and every forward takes the
# torch.library ops (the same kernels, through the dispatcher).
def _dispatch_mode_query():
    from torch.utils._python_dispatch import _get_current_dispatch_mode

    return _get_current_dispatch_mode


_dispatch_mode = _private_probe(_dispatch_mode_query)
_functorch_active = _private_probe(lambda: torch._C._are_functorch_transforms_active)


def _plain_eager(x: torch.Tensor) -> bool:
    """x is an ordinary GPU tensor in eager mode: not traced or compiled, no
    Python dispatch mode (fake tensors, functionalization) and no functorch
    transform is active, so the ops' device implementations can be called
    without going through the ops."""
    if _dispatch_mode is None or _functorch_active is None:
        return False
    return (type(x) is torch.Tensor and x.is_cuda and not torch.compiler.is_compiling()
            and not torch.jit.is_tracing() and _dispatch_mode() is None and not _functorch_active())


class MHCLiteBlock(nn.Module):
    """mHC-lite wrapper for a residual layer mapping (T, C) -> (T, C).

    Args:
        n_streams: number of residual streams n (the fused path needs n == 4).
        hidden_size: C.
        layer: module applied to the pre-mixed (T, C) input.
        triton_fused: use the fused device path when the input qualifies (the
            name is the reference's; here the fused path is HIP, not Triton).
        activation_checkpointing: recompute the pre-map and post-res regions
            in backward instead of keeping their activations.
        rmsnorm_weight: give the RMSNorm over the n*C stream a learnable
            per-channel weight ``rms_weight`` (initialised to ones).  Off by
            default, which is the reference's block (no RMSNorm weight) with
            an identical state_dict.  The fused path folds it into the
            projection: rmsnorm(x) * g @ W^T == rmsnorm(x) @ (W * g)^T.
    """

    def __init__(
        self,
        n_streams: int,
        hidden_size: int,
        layer: nn.Module,
        triton_fused: bool = True,
        activation_checkpointing: bool = False,
        rmsnorm_weight: bool = False,
    ) -> None:
        super().__init__()
        self.n = n_streams
        self.C = hidden_size
        self.nC = n_streams * hidden_size
        self.layer = layer
        self.triton_fused = triton_fused
        self.activation_checkpointing = activation_checkpointing

        self.n_fact = math.factorial(n_streams)

        self.alpha_pre = nn.Parameter(torch.tensor([0.01]))
        self.alpha_post = nn.Parameter(torch.tensor([0.01]))
        self.alpha_res = nn.Parameter(torch.tensor([0.01]))

        self.W_all = nn.Linear(self.nC, 2 * n_streams + self.n_fact, bias=True)

        perm_flat, self.identity_idx = build_permutation_matrices(n_streams)
        self.register_buffer("perm_mat", perm_flat)

        if rmsnorm_weight:
            self.rms_weight = nn.Parameter(torch.ones(self.nC))
        else:
            self.rms_weight = None

    # -- shared pieces ------------------------------------------------------

    def _use_activation_checkpointing(self, x_streams: torch.Tensor) -> bool:
        return (
            self.activation_checkpointing
            and self.training
            and torch.is_grad_enabled()
            and x_streams.requires_grad
        )

    def _coefficients(
        self, proj: torch.Tensor, dt: torch.dtype
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """K2: mixing coefficients from the (..., 2n + n!) projection, in dtype dt.

        Same operations, in the same order and precision, as the reference's
        block.py:93-105 (fallback) and :162-170 (fused path).
        """
        n = self.n
        pre, post, res = proj.split([n, n, self.n_fact], dim=-1)
        bias = self.W_all.bias.to(dt)
        h_pre = torch.sigmoid(self.alpha_pre.to(dt) * pre + bias[:n])
        h_post = 2.0 * torch.sigmoid(self.alpha_post.to(dt) * post + bias[n : 2 * n])
        a_res = F.softmax(self.alpha_res.to(dt) * res + bias[2 * n :], dim=-1)
        H_res = torch.matmul(a_res, self.perm_mat.to(dt)).unflatten(-1, (n, n))
        H_merged = H_res - h_post.unsqueeze(-1) * h_pre.unsqueeze(-2)
        return h_pre, h_post, H_merged

    # -- plain PyTorch formulation (block.py:82-148) ------------------------

    def _mhc_coeffs_pytorch(self, x_streams: torch.Tensor):
        dt = x_streams.dtype
        x_flat = x_streams.reshape(*x_streams.shape[:-2], self.nC)
        g = None if self.rms_weight is None else self.rms_weight.to(dt)
        x_norm = F.rms_norm(x_flat, (self.nC,), weight=g)
        proj = F.linear(x_norm, self.W_all.weight.to(dt), None)
        return self._coefficients(proj, dt)

    def _mhc_pre_map_pytorch(self, x_streams: torch.Tensor):
        h_pre, h_post, H_merged = self._mhc_coeffs_pytorch(x_streams)
        layer_input = torch.matmul(h_pre.unsqueeze(-2), x_streams).squeeze(-2)
        return layer_input, H_merged, h_post

    def _mhc_post_res_pytorch(self, x_streams, layer_output, H_merged, h_post):
        return (
            torch.matmul(H_merged, x_streams)
            + h_post.unsqueeze(-1) * layer_output.unsqueeze(-2)
        )

    def _forward_pytorch(self, x_streams: torch.Tensor, **kwargs) -> torch.Tensor:
        def pre_map(x, use_ckpt):
            return self._pre_map_region(self._mhc_pre_map_pytorch, x, use_ckpt)

        return self._run(x_streams, pre_map, self._mhc_post_res_pytorch, nullcontext(), kwargs)

    @staticmethod
    def _pre_map_region(fn, x_streams: torch.Tensor, use_ckpt: bool):
        """fn(x_streams), recomputed in the backward under activation checkpointing."""
        if use_ckpt:
            return _checkpoint(fn, x_streams, use_reentrant=False)
        return fn(x_streams)

    # -- fused HIP path (block.py:150-219) ------------------------------------

    def _projection_weight(self, dt: torch.dtype) -> torch.Tensor:
        """K1's W in dtype dt, with the optional RMSNorm weight folded in."""
        if self.rms_weight is None:
            w = self.W_all.weight
            return w if w.dtype is dt else w.to(dt)
        return (self.W_all.weight.float() * self.rms_weight.float()).to(dt)

    def _project_triton(self, x_streams: torch.Tensor) -> torch.Tensor:
        """K1: the (T, 2n + n!) projection of the RMS-normalised streams."""
        T = x_streams.shape[0]
        proj, _inv_rms = torch.ops.flash_mhc.fused_rmsnorm_project(
            x_streams.reshape(T, self.nC), self._projection_weight(x_streams.dtype)
        )
        return proj

    def _mhc_coeffs_triton(self, x_streams: torch.Tensor):
        """K1 + K2 as the reference's PyTorch ops: bf16 (h_pre, h_post, H_merged)."""
        return self._coefficients(self._project_triton(x_streams), x_streams.dtype)

    def _mhc_pre_map_triton(self, x_streams: torch.Tensor, use_ckpt: bool = False):
        if _ops.fused_premap_enabled():
            xgrad = _ops.fused_xgrad_flag()  # the pre-map op is on: only its own switch left
            # With x_sink, post-res's x-gradient is added in K1's backward
            # store rather than by autograd.
            args = (x_streams, self._projection_weight(x_streams.dtype), self.alpha_pre, self.alpha_post,
                    self.alpha_res, self.W_all.bias, self.perm_mat)
            if use_ckpt:
                # K1 + K2 as one op, K3 as a second one whose backward hands
                # the layer input's gradient to the first (the fused pre-map
                # backward); the checkpoint recomputes K3 alone, the layer
                # input being the one large tensor of the region.
                H_merged, h_post, h_pre, _proj, _inv, x_sink, li_sink = torch.ops.flash_mhc.mhc_pre_map_coeffs(*args)
                layer_input = _checkpoint(torch.ops.flash_mhc.mhc_pre_map_mix, x_streams, h_pre, li_sink,
                                          use_reentrant=False)
            else:
                layer_input, H_merged, h_post, _h_pre, _proj, _inv, x_sink = torch.ops.flash_mhc.mhc_pre_map(*args)
            if xgrad:
                return layer_input, H_merged, h_post, x_sink
            return layer_input, H_merged, h_post
        return self._pre_map_region(self._mhc_pre_map_triton_ops, x_streams, use_ckpt)

    def _mhc_pre_map_triton_ops(self, x_streams: torch.Tensor):
        if _ops.fused_k2_enabled():
            # One kernel for K2, same values as the ops below (fp32 outputs).
            h_pre, h_post, H_merged = torch.ops.flash_mhc.mhc_coefficients(
                self._project_triton(x_streams), self.alpha_pre, self.alpha_post,
                self.alpha_res, self.W_all.bias, self.perm_mat,
            )
            layer_input = torch.ops.flash_mhc.fused_pre_map(x_streams, h_pre)
            return layer_input, H_merged, h_post
        h_pre, h_post, H_merged = self._mhc_coeffs_triton(x_streams)
        layer_input = torch.ops.flash_mhc.fused_pre_map(x_streams, h_pre.float())
        return layer_input, H_merged.float(), h_post.float()

    def _mhc_post_res_triton(self, x_streams, layer_output, H_merged, h_post, x_sink=None):
        if x_sink is not None:
            return torch.ops.flash_mhc.mhc_post_res(x_streams, x_sink, layer_output, H_merged, h_post)
        return torch.ops.flash_mhc.fused_post_res(x_streams, layer_output, H_merged, h_post)

    def _forward_triton(self, x_streams: torch.Tensor, **kwargs) -> torch.Tensor:
        """Fused path: K1/K2/K3/K4 on the HIP kernels."""
        if _ops.fused_premap_enabled() and _plain_eager(x_streams):
            if not torch.is_grad_enabled():
                return self._forward_nograd(x_streams, **kwargs)
            if _ops.fused_xgrad_flag():
                # Also under activation checkpointing: in eager mode the
                # checkpointed K3 op saves nothing, so nothing is ever
                # recomputed, and the layer keeps the layer input if its
                # backward needs it.  The single pre-map op saves the same
                # tensors as the two ops and reads x once where the
                # single-read forward applies.
                return self._forward_eager(x_streams, **kwargs)
        ctx = nullcontext() if self.training else _ops.disable_autotune_temporarily()
        # Only the pre-map region is checkpointed: post-res's backward needs
        # exactly the inputs a checkpoint would keep (x, layer_output,
        # H_merged, h_post), so recomputing its forward would only cost time.
        return self._run(x_streams, self._mhc_pre_map_triton, self._mhc_post_res_triton, ctx, kwargs,
                         checkpoint_post_res=False)

    def _forward_eager(self, x_streams: torch.Tensor, **kwargs) -> torch.Tensor:
        """The fused forward in eager mode with autograd (training at few
        tokens is bound by the host): mhc_pre_map and mhc_post_res with their
        registered autograd, applied as autograd Functions around the ops'
        device implementations instead of through the dispatcher.  Same
        kernels, same values, same x-gradient sink."""
        p = self._parameters
        layer_input, H_merged, h_post, x_sink = _ops.pre_map_eager(
            x_streams, self._projection_weight(x_streams.dtype), p["alpha_pre"], p["alpha_post"], p["alpha_res"],
            self.W_all.bias, self._buffers["perm_mat"])
        layer_output = self.layer(layer_input, **kwargs)
        return _ops.post_res_eager(x_streams, x_sink, layer_output, H_merged, h_post)

    def _forward_nograd(self, x_streams: torch.Tensor, **kwargs) -> torch.Tensor:
        """The fused forward when no autograd graph is recorded (inference):
        the pre-map and post-res kernels are launched as the ops' device
        implementations launch them, without the custom-op dispatch around
        each call (tens of microseconds per call at few tokens).  Same
        kernels, same values."""
        p = self._parameters
        layer_input, coeffs = _ops.pre_map_nograd(
            x_streams, self._projection_weight(x_streams.dtype), p["alpha_pre"], p["alpha_post"], p["alpha_res"],
            self.W_all.bias, self._buffers["perm_mat"])
        layer_output = self.layer(layer_input, **kwargs)
        return _ops.post_res_nograd(x_streams, layer_output, coeffs)

    # -- common driver ------------------------------------------------------

    def _run(self, x_streams, pre_map, post_res, ctx, kwargs, checkpoint_post_res=True) -> torch.Tensor:
        use_ckpt = self._use_activation_checkpointing(x_streams)
        with ctx:
            # pre_map(x, use_ckpt) returns (layer_input, H_merged, h_post, *extra)
            # and applies the checkpointing of its region itself; post_res
            # takes (x_streams, layer_output, H_merged, h_post, *extra).
            layer_input, *coeffs = pre_map(x_streams, use_ckpt)

            layer_output = self.layer(layer_input, **kwargs)

            if use_ckpt and checkpoint_post_res:
                return _checkpoint(post_res, x_streams, layer_output, *coeffs, use_reentrant=False)
            return post_res(x_streams, layer_output, *coeffs)

    def forward(self, x_streams: torch.Tensor, **kwargs) -> torch.Tensor:
        use_fused = (
            self.triton_fused
            and x_streams.is_cuda
            and x_streams.dtype == torch.bfloat16
            and x_streams.dim() == 3
            and self.n == 4
        )
        if use_fused:
            return self._forward_triton(x_streams, **kwargs)
        return self._forward_pytorch(x_streams, **kwargs)
