"""Oracle: a CPU restatement of the reference's mHC-lite math (alint77/flash-mHC).

TEST INFRASTRUCTURE ONLY.  The ``flash_mhc`` package never imports this
module.  Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may use it, to check results or as the timed CPU baseline,
never as an implementation of the product path.

Contents
  * per-op formulas of the six device kernels, computed in float64 from the
    kernels' own (bf16 / fp32) inputs, each returning the value ``R`` and the
    magnitude ``S = sum |terms|`` that bounds the summation-order error of any
    fp32 evaluation (used by the parity tolerance in tests/parity.py);
  * the K1 weight-gradient formula of the autograd rule;
  * the block's coefficient math (K2) and the block's plain-PyTorch
    formulation, in any float dtype;
  * differentiable fp32 per-op formulas (the CPU baseline that bench.py times);
  * pure-Python loop versions for tiny shapes, used to pin the vectorised
    formulas above.

Pinning status (what checks each function; see tests/test_oracle.py):
  permutation_matrices   brute force over itertools + doubly-stochastic invariants
  k1_fwd                 loops, F.rms_norm(eps=1e-6) @ W^T in fp64, selector rows,
                         constant rows, scale invariance
  k1_bwd_dx              fp64 autograd of k1_fwd's formula (gradcheck)
  k1_grad_W              fp64 autograd + the bf16 rounding of go*inv_rms
  k3_fwd / k3_bwd        loops, one-hot h_pre, fp64 gradcheck
  k4_fwd / k4_bwd        loops, identity / permutation H, fp64 gradcheck
  coefficients, block    fp64 gradcheck, doubly-stochastic H_res,
                         out = H_res x + h_post (lo - h_pre^T x),
                         fixture written by the reference's own fallback
"""

from __future__ import annotations

import itertools
import math

import torch
import torch.nn.functional as F

EPS_K1 = 1e-6  # src/flash_mhc/kernels.py:296
F64 = torch.float64


def _f64(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to("cpu", F64)


# ---------------------------------------------------------------------------
# Permutation matrices (block.py:21-32)


def permutation_matrices(n: int) -> tuple[torch.Tensor, int]:
    """(n!, n*n) float32, row m = flattened matrix of the m-th permutation of
    itertools.permutations(range(n)); entry [i*n + j] = 1 iff perm(i) == j."""
    perms = list(itertools.permutations(range(n)))
    out = torch.zeros(len(perms), n * n)
    for m, p in enumerate(perms):
        for i in range(n):
            out[m, i * n + p[i]] = 1.0
    return out, 0


# ---------------------------------------------------------------------------
# K1 (kernels.py:250-303 forward, :306-376 dx; ops.py:678-685 autograd)


def k1_fwd(x_flat: torch.Tensor, W: torch.Tensor):
    """Returns (proj R, proj S, inv_rms R) in float64.

    inv_rms = (sum_k x^2 / nC + 1e-6)^-1/2 ; proj[t,d] = inv_rms[t] * sum_k x[t,k] W[d,k]
    (project first, then scale: kernels.py:264-303)."""
    x = _f64(x_flat)
    w = _f64(W)
    nC = x.shape[1]
    ss = (x * x).sum(dim=1)
    inv = (ss / nC + EPS_K1).rsqrt()
    raw = x @ w.T
    proj = raw * inv[:, None]
    proj_s = (x.abs() @ w.abs().T) * inv[:, None]
    return proj, proj_s, inv


def k1_bwd_dx(grad_out, x_flat, W, proj_out, inv_rms):
    """grad_x R and S (float64) following kernels.py:313-376:
    scale = (sum_d go*proj) * inv^2 / nC ; gx = inv * (go @ W) - scale * x."""
    go = _f64(grad_out)
    x = _f64(x_flat)
    w = _f64(W)
    p = _f64(proj_out)
    inv = _f64(inv_rms)
    nC = x.shape[1]
    dot = (go * p).sum(dim=1)
    scale = dot * inv * inv / nC
    gx = inv[:, None] * (go @ w) - scale[:, None] * x
    dot_s = (go * p).abs().sum(dim=1)
    gx_s = inv[:, None] * (go.abs() @ w.abs()) + (dot_s * inv * inv / nC)[:, None] * x.abs()
    return gx, gx_s


def k1_grad_W(grad_out, x_flat, inv_rms):
    """grad_W R and S (float64) of ops.py:683-684: bf16(go * inv)^T @ x."""
    go = grad_out.detach().cpu()
    scaled = (go.float() * inv_rms.detach().cpu().float()[:, None]).to(torch.bfloat16)
    s = _f64(scaled)
    x = _f64(x_flat)
    return s.T @ x, s.abs().T @ x.abs()


# ---------------------------------------------------------------------------
# K3 (kernels.py:673-717 forward, :720-853 backward)


def k3_fwd(x_streams, h_pre):
    x = _f64(x_streams)
    h = _f64(h_pre)
    return (h[:, :, None] * x).sum(dim=1), (h.abs()[:, :, None] * x.abs()).sum(dim=1)


def k3_bwd(grad_out, x_streams, h_pre):
    """(grad_x R, grad_x S, grad_h_pre R, grad_h_pre S)."""
    go = _f64(grad_out)
    x = _f64(x_streams)
    h = _f64(h_pre)
    gx = h[:, :, None] * go[:, None, :]
    gh = (x * go[:, None, :]).sum(dim=2)
    gh_s = (x.abs() * go.abs()[:, None, :]).sum(dim=2)
    return gx, gx.abs(), gh, gh_s


# ---------------------------------------------------------------------------
# K4 (kernels.py:384-481 forward, :487-665 backward)


def k4_fwd(x_streams, layer_output, H_merged, h_post):
    x = _f64(x_streams)
    lo = _f64(layer_output)
    H = _f64(H_merged)
    hp = _f64(h_post)
    out = H @ x + hp[:, :, None] * lo[:, None, :]
    s = H.abs() @ x.abs() + hp.abs()[:, :, None] * lo.abs()[:, None, :]
    return out, s


def k4_bwd(grad_out, x_streams, layer_output, H_merged, h_post):
    """Dict of name -> (R, S) for grad_x, grad_lo, grad_H, grad_hp."""
    go = _f64(grad_out)
    x = _f64(x_streams)
    lo = _f64(layer_output)
    H = _f64(H_merged)
    hp = _f64(h_post)
    res = {
        "grad_x": (H.transpose(1, 2) @ go, H.abs().transpose(1, 2) @ go.abs()),
        "grad_lo": ((hp[:, :, None] * go).sum(dim=1), (hp.abs()[:, :, None] * go.abs()).sum(dim=1)),
        "grad_H": (go @ x.transpose(1, 2), go.abs() @ x.abs().transpose(1, 2)),
        "grad_hp": ((go * lo[:, None, :]).sum(dim=2), (go.abs() * lo.abs()[:, None, :]).sum(dim=2)),
    }
    return res


# ---------------------------------------------------------------------------
# Differentiable per-op formulas in any float dtype (the reference's
# pure-PyTorch math for each op; bench.py times these in fp32 on the host).


def k1_torch(x_flat, W, eps: float = EPS_K1):
    nC = x_flat.shape[-1]
    inv = torch.rsqrt((x_flat * x_flat).sum(-1, keepdim=True) / nC + eps)
    return (x_flat @ W.T) * inv


def k3_torch(x_streams, h_pre):
    return (h_pre.unsqueeze(-1) * x_streams).sum(dim=-2)


def k4_torch(x_streams, layer_output, H_merged, h_post):
    return torch.matmul(H_merged, x_streams) + h_post.unsqueeze(-1) * layer_output.unsqueeze(-2)


# ---------------------------------------------------------------------------
# K2 coefficient math and the whole block (block.py:82-148, :150-177)


def coefficients(proj, bias, alpha_pre, alpha_post, alpha_res, perm, n: int, taps: dict | None = None):
    """(h_pre, h_post, H_merged, H_res) from the (.., 2n+n!) projection, in proj's dtype.

    If ``taps`` is a dict, the logits z = alpha * proj_part + bias and the
    projection parts are stored in it (tests use them to bound the rounding
    error of the alpha gradients, which are sums over all tokens)."""
    dt = proj.dtype
    nf = math.factorial(n)
    pre, post, res = proj[..., :n], proj[..., n : 2 * n], proj[..., 2 * n : 2 * n + nf]
    b = bias.to(dt)
    z_pre = alpha_pre.to(dt) * pre + b[:n]
    z_post = alpha_post.to(dt) * post + b[n : 2 * n]
    z_res = alpha_res.to(dt) * res + b[2 * n :]
    if taps is not None:
        for name, z, part in (("pre", z_pre, pre), ("post", z_post, post), ("res", z_res, res)):
            if z.requires_grad:
                z.retain_grad()
            taps["z_" + name] = z
            taps["p_" + name] = part
    h_pre = torch.sigmoid(z_pre)
    h_post = 2.0 * torch.sigmoid(z_post)
    a_res = torch.softmax(z_res, dim=-1)
    if taps is not None:
        if a_res.requires_grad:
            a_res.retain_grad()
        taps["a_res"] = a_res
    H_res = (a_res @ perm.to(dt)).reshape(*a_res.shape[:-1], n, n)
    H_merged = H_res - h_post[..., :, None] * h_pre[..., None, :]
    return h_pre, h_post, H_merged, H_res


def block_forward(x_streams, params: dict, layer, n: int, taps: dict | None = None):
    """The block's plain-PyTorch formulation (block.py:82-148).

    params: W (2n+n!, nC), b, alpha_pre, alpha_post, alpha_res, perm, and
    optionally g (nC,), an RMSNorm weight (block option, absent in the reference)."""
    dt = x_streams.dtype
    nC = x_streams.shape[-1] * n
    x_flat = x_streams.reshape(*x_streams.shape[:-2], nC)
    # F.rms_norm with eps=None uses finfo(float32).eps for fp32 and bf16
    # (bf16 is upcast), and finfo(float64).eps for fp64.
    g = params.get("g")
    x_norm = F.rms_norm(x_flat, (nC,), weight=None if g is None else g.to(dt))
    proj = x_norm @ params["W"].to(dt).T
    h_pre, h_post, H_merged, _ = coefficients(
        proj, params["b"], params["alpha_pre"], params["alpha_post"], params["alpha_res"],
        params["perm"], n, taps,
    )
    layer_input = (h_pre.unsqueeze(-1) * x_streams).sum(dim=-2)
    layer_output = layer(layer_input)
    return H_merged @ x_streams + h_post.unsqueeze(-1) * layer_output.unsqueeze(-2)


# ---------------------------------------------------------------------------
# Pure-Python loops for tiny shapes (pin the vectorised formulas)


def k1_fwd_loops(x_flat, W):
    x = x_flat.tolist()
    w = W.tolist()
    T, nC, D = len(x), len(x[0]), len(w)
    proj = [[0.0] * D for _ in range(T)]
    inv = [0.0] * T
    for t in range(T):
        ss = 0.0
        for k in range(nC):
            ss += float(x[t][k]) ** 2
        inv[t] = 1.0 / math.sqrt(ss / nC + EPS_K1)
        for d in range(D):
            acc = 0.0
            for k in range(nC):
                acc += float(x[t][k]) * float(w[d][k])
            proj[t][d] = acc * inv[t]
    return torch.tensor(proj, dtype=F64), torch.tensor(inv, dtype=F64)


def k3_fwd_loops(x_streams, h_pre):
    x = x_streams.tolist()
    h = h_pre.tolist()
    T, n, C = len(x), len(x[0]), len(x[0][0])
    out = [[sum(float(h[t][j]) * float(x[t][j][c]) for j in range(n)) for c in range(C)] for t in range(T)]
    return torch.tensor(out, dtype=F64)


def k4_fwd_loops(x_streams, layer_output, H_merged, h_post):
    x = x_streams.tolist()
    lo = layer_output.tolist()
    H = H_merged.tolist()
    hp = h_post.tolist()
    T, n, C = len(x), len(x[0]), len(x[0][0])
    out = [
        [
            [float(hp[t][i]) * float(lo[t][c]) + sum(float(H[t][i][j]) * float(x[t][j][c]) for j in range(n))
             for c in range(C)]
            for i in range(n)
        ]
        for t in range(T)
    ]
    return torch.tensor(out, dtype=F64)


def k4_bwd_loops(grad_out, x_streams, layer_output, H_merged, h_post):
    go = grad_out.tolist()
    x = x_streams.tolist()
    lo = layer_output.tolist()
    H = H_merged.tolist()
    hp = h_post.tolist()
    T, n, C = len(x), len(x[0]), len(x[0][0])
    gx = [[[sum(H[t][i][j] * go[t][i][c] for i in range(n)) for c in range(C)] for j in range(n)] for t in range(T)]
    glo = [[sum(hp[t][i] * go[t][i][c] for i in range(n)) for c in range(C)] for t in range(T)]
    gH = [[[sum(go[t][i][c] * x[t][j][c] for c in range(C)) for j in range(n)] for i in range(n)] for t in range(T)]
    ghp = [[sum(go[t][i][c] * lo[t][c] for c in range(C)) for i in range(n)] for t in range(T)]
    f = lambda v: torch.tensor(v, dtype=F64)  # noqa: E731
    return {"grad_x": f(gx), "grad_lo": f(glo), "grad_H": f(gH), "grad_hp": f(ghp)}
