"""Oracle for K2, the mHC-lite coefficient math, with the bf16 rounding points
of the reference's fused path (alint77/flash-mHC src/flash_mhc/block.py:161-170).

TEST INFRASTRUCTURE ONLY (same rules as mhc_oracle.py): the ``flash_mhc``
package never imports it; only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may.

The reference computes K2 as a chain of PyTorch ops on bf16 tensors.  Each op
evaluates in fp32 from its bf16 inputs and rounds its output to bf16
(round-to-nearest-even), and autograd does the same for every backward op.
This module restates that chain step by step in numpy float32, with an
explicit RNE rounding ``rb`` wherever a bf16 tensor is produced:

forward (per token; p = proj (32,), a_* = bf16(alpha_*), b = bf16(bias)):
    z_pre  = rb(rb(a_pre * p[0:4]) + b[0:4]);    h_pre  = rb(sigmoid(z_pre))
    z_post = rb(rb(a_post * p[4:8]) + b[4:8]);   s_post = rb(sigmoid(z_post));  h_post = rb(2 s_post)
    z_res  = rb(rb(a_res * p[8:32]) + b[8:32]);  a      = rb(softmax(z_res))
    H_res  = rb(a @ perm);  P = rb(h_post[:, None] * h_pre[None, :]);  H_merged = rb(H_res - P)
  (block.py:164-170), with sigmoid(z) = 1 / (1 + exp(-z)) and
  softmax = exp(z - max) / sum exp(z - max), fp32 arithmetic.

backward (what autograd does for that chain, given the fp32 gradients of the
fp32 casts h_pre.float(), h_post.float(), H_merged.float() of block.py:176-177,
which autograd first rounds to bf16):
    gH = rb(g_H); gP = -gH
    h_post <- rb(sum_j rb(gP[i, j] h_pre[j])) + rb(g_hpost);  h_pre <- rb(sum_i rb(gP[i, j] h_post[i])) + rb(g_hpre)
    g_a = rb(gH_flat @ perm^T);  g_zres = softmax_bwd(g_a, a)
    g_zpre = sigmoid_bwd(g_hpre, h_pre);  g_zpost = sigmoid_bwd(rb(2 g_hpost), s_post)
    g_proj = rb(g_z * a_*);  g_alpha = rb(sum over tokens and lanes of rb(g_z * p));  g_bias = rb(sum over tokens of g_z)
  Sums over the (at most 24) terms of one token run in index order in fp32;
  the sums over tokens (alpha and bias gradients) are returned in float64 with
  S = sum |terms|, the magnitude that bounds any fp32 summation order.

The two backward ops with internal arithmetic round differently on torch's
GPU and CPU kernels, and the reference's fused path runs on the GPU:
  rounding="gpu" (default, the reference's device semantics: PyTorch's CUDA /
  HIP kernels for bf16 do c10::BFloat16 arithmetic, which rounds every step)
      sigmoid_bwd(g, y) = rb(rb(g * rb(1 - y)) * y)
      softmax_bwd(g, y) = rb(gy - y * s),  gy = rb(g * y),  s = sum gy   (fp32 sum)
  rounding="cpu" (torch's CPU kernels: fp32 inside, one rounding)
      sigmoid_bwd(g, y) = rb(g * (1 - y) * y)
      softmax_bwd(g, y) = rb(gy - y * s),  gy = g * y,      s = sum gy

Pinning: the forward and the rounding="cpu" backward equal, up to rare
last-bit flips of exp and of fp32 summation order, torch's own bf16 CPU
forward and autograd through the same op sequence (mhc_oracle.coefficients,
tests/test_oracle.py); the two rounding="gpu" steps equal torch's GPU
aten.sigmoid_backward / aten._softmax_backward_data (tests/test_gpu_k2.py);
planted mistakes (a dropped rounding, a transposed permutation, a wrong
sigmoid derivative) break the CPU agreement.
"""

from __future__ import annotations

import numpy as np
import torch

N = 4
NF = 24
D = 2 * N + NF  # 32 projection columns
F32 = np.float32


def rb(a) -> np.ndarray:
    """Round float32 values to bf16 (nearest, ties to even); returns float32."""
    a = np.asarray(a, dtype=F32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(F32)


def _np(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        return t.detach().to("cpu", torch.float32).numpy()
    return np.asarray(t, dtype=F32)


def _exp(x: np.ndarray) -> np.ndarray:
    # exp correctly rounded to fp32.
    with np.errstate(over="ignore"):  # exp overflows to inf, as in fp32
        return np.exp(x.astype(np.float64)).astype(F32)


def _sigmoid(z: np.ndarray) -> np.ndarray:
    # fp32: 1 / (1 + exp(-z)), each operation rounded to fp32.
    d = (F32(1) + _exp(-z)).astype(F32)
    return (F32(1) / d).astype(F32)


def _seqsum(terms, axis: int) -> np.ndarray:
    """fp32 sum in index order along ``axis``."""
    terms = np.moveaxis(np.asarray(terms, dtype=F32), axis, 0)
    acc = np.zeros(terms.shape[1:], dtype=F32)
    for k in range(terms.shape[0]):
        acc = (acc + terms[k]).astype(F32)
    return acc


def sigmoid_bwd(g, y, rounding: str = "gpu") -> np.ndarray:
    """Gradient of z for y = rb(sigmoid(z)), given the bf16 gradient g of y."""
    g, y = np.asarray(g, F32), np.asarray(y, F32)
    if rounding == "gpu":
        return rb(rb(g * rb(F32(1) - y)) * y)
    return rb(((g * (F32(1) - y)).astype(F32) * y).astype(F32))


def softmax_bwd(g, y, rounding: str = "gpu") -> np.ndarray:
    """Gradient of z (rows along the last axis) for y = rb(softmax(z))."""
    g, y = np.asarray(g, F32), np.asarray(y, F32)
    gy = (g * y).astype(F32)
    if rounding == "gpu":
        gy = rb(gy)
    s = _seqsum(gy, gy.ndim - 1)[..., None]
    return rb(gy - (y * s).astype(F32))


def _params(alpha_pre, alpha_post, alpha_res, bias, perm):
    a = [rb(_np(v).reshape(-1)[:1])[0] for v in (alpha_pre, alpha_post, alpha_res)]
    b = rb(_np(bias).reshape(-1))
    P = rb(_np(perm).reshape(NF, N * N))
    return a[0], a[1], a[2], b, P


def k2_fwd(proj, alpha_pre, alpha_post, alpha_res, bias, perm, _plant: str | None = None) -> dict:
    """Forward chain; returns h_pre (T,4), h_post (T,4), H_merged (T,4,4) as
    bf16-exact float32 arrays, plus the intermediates the backward uses.
    ``_plant`` is a test hook that introduces a named mistake."""
    p = _np(proj).reshape(-1, D)
    ap, apo, ar, b, P = _params(alpha_pre, alpha_post, alpha_res, bias, perm)
    if _plant == "transpose_perm":
        P = P.reshape(NF, N, N).transpose(0, 2, 1).reshape(NF, N * N)
    scale = (lambda v: (v).astype(F32)) if _plant == "no_round_scale" else rb
    z_pre = rb(scale(ap * p[:, :N]) + b[:N])
    h_pre = rb(_sigmoid(z_pre))
    z_post = rb(scale(apo * p[:, N : 2 * N]) + b[N : 2 * N])
    s_post = rb(_sigmoid(z_post))
    h_post = rb(F32(2) * s_post)
    z_res = rb(scale(ar * p[:, 2 * N :]) + b[2 * N :])
    e = _exp((z_res - z_res.max(axis=1, keepdims=True)).astype(F32))
    a = rb((e / _seqsum(e, 1)[:, None]).astype(F32))
    H_res = rb(_seqsum(a[:, :, None] * P[None, :, :], 1))  # (T, 16)
    Pm = rb(h_post[:, :, None] * h_pre[:, None, :])
    H = rb(H_res.reshape(-1, N, N) - Pm)
    return dict(h_pre=h_pre, h_post=h_post, H_merged=H, s_post=s_post, a_res=a, H_res=H_res,
                P=Pm, p=p, ap=ap, apo=apo, ar=ar, perm=P)


def k2_bwd(proj, alpha_pre, alpha_post, alpha_res, bias, perm, g_hpre, g_hpost, g_H,
           rounding: str = "gpu", _plant: str | None = None) -> dict:
    """Backward chain.  Gradients of the fp32 outputs may be None (zero).
    ``rounding`` selects the GPU or CPU semantics of the sigmoid and softmax
    backward steps (module docstring).

    Returns grad_proj (T,32) bf16-exact float32 and, for alpha_pre,
    alpha_post, alpha_res (scalars) and bias (32,), float64 sums R with their
    magnitudes S (keys ``grad_alpha_pre`` -> (R, S), ...)."""
    f = k2_fwd(proj, alpha_pre, alpha_post, alpha_res, bias, perm)
    p, ap, apo, ar, P = f["p"], f["ap"], f["apo"], f["ar"], f["perm"]
    h_pre, h_post, s_post, a = f["h_pre"], f["h_post"], f["s_post"], f["a_res"]
    T = p.shape[0]
    zero = lambda *s: np.zeros((T,) + s, dtype=F32)
    gH = rb(zero(N, N) if g_H is None else _np(g_H).reshape(T, N, N))
    ghp_in = rb(zero(N) if g_hpre is None else _np(g_hpre).reshape(T, N))
    ghq_in = rb(zero(N) if g_hpost is None else _np(g_hpost).reshape(T, N))

    gP = -gH
    ghq = rb(ghq_in + rb(_seqsum(rb(gP * h_pre[:, None, :]), 2)))
    ghp = rb(ghp_in + rb(_seqsum(rb(gP * h_post[:, :, None]), 1)))

    gHf = gH.reshape(T, N * N)
    ga = rb(_seqsum(gHf[:, None, :] * P[None, :, :], 2))  # (T, 24)
    gz_res = softmax_bwd(ga, a, rounding)

    if _plant == "sigmoid_derivative":
        gz_pre = rb((ghp * h_pre).astype(F32))
    else:
        gz_pre = sigmoid_bwd(ghp, h_pre, rounding)
    gs = rb(ghq * F32(2))
    gz_post = sigmoid_bwd(gs, s_post, rounding)

    grad_proj = np.concatenate([rb(gz_pre * ap), rb(gz_post * apo), rb(gz_res * ar)], axis=1)

    def total(terms):
        t = terms.astype(np.float64)
        return t.sum(), np.abs(t).sum()

    out = dict(grad_proj=grad_proj)
    out["grad_alpha_pre"] = total(rb(gz_pre * p[:, :N]))
    out["grad_alpha_post"] = total(rb(gz_post * p[:, N : 2 * N]))
    out["grad_alpha_res"] = total(rb(gz_res * p[:, 2 * N :]))
    gz = np.concatenate([gz_pre, gz_post, gz_res], axis=1).astype(np.float64)
    out["grad_bias"] = (gz.sum(axis=0), np.abs(gz).sum(axis=0))
    return out
