"""Parity tolerances for the bf16 / fp32 outputs of the HIP kernels.

Every check compares a device result ``o`` with the oracle value ``R``
computed in float64 from the *same* bf16/fp32 inputs, and with
``S = sum |terms|`` of the same formula.

bf16 outputs (the path's tolerance: equal to the fp32 value rounded to
bf16 within 1 bf16 ulp):
    |o - R| <= ulp_bf16(R) + 4 * sqrt(n) * 2^-24 * S
The second term is the probabilistic bound of an n-term fp32 sum in any
order (Higham's sqrt(n) rule with a 4-sigma margin).  It only matters where
the terms cancel (|R| << S), i.e. where "1 ulp of the fp32 reference" is
itself ill-defined.

fp32 outputs (reductions): |o - R| <= 4 * sqrt(n) * 2^-24 * S + 2^-23 * |R|.
"""

from __future__ import annotations

import math

import torch

U32 = 2.0 ** -24


def bf16_ulp(R: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |R| (normal range; 2^-133 below it)."""
    _, e = torch.frexp(R.abs().clamp_min(2.0 ** -126))
    return torch.ldexp(torch.ones_like(R), (e - 8).to(torch.int32))


def _stats(err: torch.Tensor, tol: torch.Tensor) -> str:
    ratio = err / tol
    idx = int(torch.argmax(ratio))
    return (f"max err {float(err.max()):.3e}, worst err/tol {float(ratio.flatten()[idx]):.3f} "
            f"at flat index {idx}")


def check_bf16(name: str, out: torch.Tensor, R: torch.Tensor, S: torch.Tensor, n_terms: int) -> dict:
    o = out.detach().to("cpu", torch.float64)
    assert o.shape == R.shape, f"{name}: shape {tuple(o.shape)} != {tuple(R.shape)}"
    assert out.dtype == torch.bfloat16, f"{name}: dtype {out.dtype}"
    err = (o - R).abs()
    tol = bf16_ulp(R) + 4.0 * math.sqrt(n_terms) * U32 * S
    bad = ~(err <= tol)  # also catches NaN
    assert not bool(bad.any()), f"{name}: {int(bad.sum())} of {err.numel()} elements out of tolerance; {_stats(err, tol)}"
    exact = (o == R.to(torch.bfloat16).double()).double().mean().item()
    return {"max_err": float(err.max()) if err.numel() else 0.0, "frac_equal_rn": exact}


def check_fp32(name: str, out: torch.Tensor, R: torch.Tensor, S: torch.Tensor, n_terms: int) -> dict:
    o = out.detach().to("cpu", torch.float64)
    assert o.shape == R.shape, f"{name}: shape {tuple(o.shape)} != {tuple(R.shape)}"
    assert out.dtype == torch.float32, f"{name}: dtype {out.dtype}"
    err = (o - R).abs()
    tol = 4.0 * math.sqrt(n_terms) * U32 * S + 2.0 * U32 * R.abs() + 1e-30
    bad = ~(err <= tol)
    assert not bool(bad.any()), f"{name}: {int(bad.sum())} of {err.numel()} elements out of tolerance; {_stats(err, tol)}"
    return {"max_err": float(err.max()) if err.numel() else 0.0}


def check_rel(name: str, out: torch.Tensor, R: torch.Tensor, rtol: float) -> None:
    """|o - R| <= rtol * |R| elementwise (positive quantities such as inv_rms)."""
    o = out.detach().to("cpu", torch.float64)
    err = (o - R).abs()
    tol = rtol * R.abs()
    bad = ~(err <= tol)
    assert not bool(bad.any()), f"{name}: {int(bad.sum())} elements out of tolerance; {_stats(err, tol)}"


def block_close(name: str, out: torch.Tensor, ref: torch.Tensor, rtol: float = 2e-2, atol: float = 5e-2) -> dict:
    """Block-level check of the bf16 fused pipeline against an fp32 reference:
        |o - ref| <= rtol * |ref| + atol * rms_t(ref)
    elementwise, where rms_t is the RMS of the reference over token t (dim 0).
    rtol/atol default to the reference's own end-to-end forward tolerances
    (tests/test_correctness.py:284; 5e-2 / 1e-1 for gradients, :296, :317),
    with the absolute term scaled by each token's magnitude so that tokens
    scaled x100 are held to the same relative standard.  The bf16 pipeline
    rounds the K2 coefficients to bf16 by design (block.py:163-169 of the
    reference); the per-kernel checks above are the tight ones."""
    o = out.detach().to("cpu", torch.float64)
    r = ref.detach().to("cpu", torch.float64)
    assert o.shape == r.shape, f"{name}: shape {tuple(o.shape)} != {tuple(r.shape)}"
    if r.dim() >= 2:
        rms_t = r.reshape(r.shape[0], -1).pow(2).mean(dim=1).sqrt().reshape(-1, *([1] * (r.dim() - 1)))
    else:
        rms_t = r.pow(2).mean().sqrt()
    err = (o - r).abs()
    tol = rtol * r.abs() + atol * rms_t + 1e-30
    bad = ~(err <= tol)
    assert not bool(bad.any()), f"{name}: {int(bad.sum())} of {err.numel()} out of tolerance; {_stats(err, tol)}"
    rel = float(err.norm() / max(float(r.norm()), 1e-30))
    return {"rel_l2": rel, "max_err_over_tol": float((err / tol).max()) if err.numel() else 0.0}


def check_chain(name: str, out, ref, max_rate: float = 1e-3) -> dict:
    """bf16 op chains (K2): ``out`` and ``ref`` are both bf16-exact, ``ref``
    from the oracle's step-by-step rounding of the same chain.  The two can
    only differ through last-bit flips of exp or of an fp32 summation order
    that a later rounding carries on, so at most ``max_rate`` of the elements
    may differ, and each by at most ulp_bf16(ref) + 4 ulp_bf16(max |ref| of
    its token).  Dim 0 indexes tokens."""
    o = torch.as_tensor(out).detach().to("cpu", torch.float64)
    r = torch.as_tensor(ref).detach().to("cpu", torch.float64)
    assert o.numel() == r.numel(), f"{name}: {o.numel()} != {r.numel()} elements"
    T = r.shape[0] if r.dim() else 1
    o, r = o.reshape(T, -1), r.reshape(T, -1)
    err = (o - r).abs()
    rowmax = r.abs().amax(dim=1, keepdim=True).expand_as(r)
    tol = bf16_ulp(r) + 4.0 * bf16_ulp(rowmax)
    bad = ~(err <= tol)
    assert not bool(bad.any()), f"{name}: {int(bad.sum())} of {err.numel()} elements out of tolerance; {_stats(err, tol)}"
    rate = float((err != 0).double().mean()) if err.numel() else 0.0
    assert rate <= max_rate, f"{name}: {rate:.2e} of the elements differ (allowed {max_rate:.0e})"
    return {"frac_differ": rate}
