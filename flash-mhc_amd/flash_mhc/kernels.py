"""Launchers for the gfx950 HIP kernels (drop-in for the reference's Triton
``kernels.py``).

Each function validates its tensors, allocates any output that was not passed
in, and enqueues one kernel through the C ABI on torch's current stream of
the tensors' device.  Nothing here falls back to another implementation: a
missing extension or a bad argument raises.

Reference counterparts (alint77/flash-mHC):
  k1_fwd     <- src/flash_mhc/kernels.py:250-303  _fused_rmsnorm_project_fwd_kernel
  k1_bwd_dx  <- src/flash_mhc/kernels.py:306-376  _fused_rmsnorm_project_bwd_dx_kernel
  k1_bwd     <- the above plus the grad_W matmul of src/flash_mhc/ops.py:683-684, fused
  k2_fwd     <- src/flash_mhc/block.py:161-170 (PyTorch ops) and the .float() casts of :176-177
  k2_bwd     <- autograd through the same ops
  premap_fwd <- K1 + K2 + K3 of src/flash_mhc/block.py:157-177 (one entry point)
  premap_bwd <- autograd through the same, x's two gradients summed in K1's store
  k3_fwd     <- src/flash_mhc/kernels.py:673-717  _fused_pre_map_fwd_kernel
  k3_bwd     <- src/flash_mhc/kernels.py:720-853  _fused_pre_map_bwd_fused_kernel_n4
  k4_fwd     <- src/flash_mhc/kernels.py:384-481  _fused_post_res_fwd_kernel_n4
  k4_bwd     <- src/flash_mhc/kernels.py:487-665  _fused_post_res_bwd_fused_kernel_n4
"""

from __future__ import annotations

import torch

from . import _abi

N_STREAMS = 4
D_OUT = 32  # 2n + n! at n = 4

_BF16 = torch.bfloat16
_F32 = torch.float32


def _require(t: torch.Tensor, name: str, dtype: torch.dtype, shape: tuple[int, ...], device) -> None:
    # One compound test on the common path; the messages come from _reject.
    if (not isinstance(t, torch.Tensor) or t.dtype is not dtype or t.shape != shape or t.device != device
            or not t.is_contiguous()):
        _reject(t, name, dtype, shape, device)


def _reject(t, name: str, dtype: torch.dtype, shape: tuple[int, ...], device) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.shape != shape:  # torch.Size compares equal to a tuple of the same ints
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    raise ValueError(f"{name} must be contiguous")


def _device_of(x: torch.Tensor) -> torch.device:
    if not isinstance(x, torch.Tensor):
        raise TypeError("expected a torch.Tensor")
    if x.device.type != "cuda":
        raise ValueError(f"flash_mhc HIP kernels need a GPU tensor, got device {x.device}")
    return x.device


class _OnDevice:
    """Make ``device`` current for the launch (cheap when it already is)."""

    __slots__ = ("idx", "prev")

    def __init__(self, device: torch.device):
        idx = device.index
        self.idx = torch.cuda.current_device() if idx is None else idx
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.idx:
            self.prev = cur
            torch.cuda.set_device(self.idx)

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)


def k1_fwd(x_flat: torch.Tensor, W: torch.Tensor, out: torch.Tensor | None = None,
           inv_rms: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """proj (T, 32) bf16 and inv_rms (T,) fp32 from x_flat (T, nC) bf16, W (32, nC) bf16
    (fmhc_k1_fwd_ws: few tokens split the nC axis over workgroups)."""
    dev = _device_of(x_flat)
    if x_flat.dim() != 2:
        raise ValueError(f"x_flat must be 2-D (T, nC), got shape {tuple(x_flat.shape)}")
    T, nC = x_flat.shape
    _require(x_flat, "x_flat", _BF16, (T, nC), dev)
    if W.dim() != 2 or W.shape[0] != D_OUT:
        raise ValueError(f"W must have shape ({D_OUT}, nC); got {tuple(W.shape)}")
    _require(W, "W", _BF16, (D_OUT, nC), dev)
    if out is None:
        out = torch.empty((T, D_OUT), device=dev, dtype=_BF16)
    if inv_rms is None:
        inv_rms = torch.empty((T,), device=dev, dtype=_F32)
    _require(out, "out", _BF16, (T, D_OUT), dev)
    _require(inv_rms, "inv_rms", _F32, (T,), dev)
    lib = _abi.load()
    ws = _workspace(int(lib.fmhc_k1_fwd_workspace_bytes(T, nC)), dev)
    with _OnDevice(dev):
        st = lib.fmhc_k1_fwd_ws(x_flat.data_ptr(), W.data_ptr(), out.data_ptr(), inv_rms.data_ptr(),
                                _ptr_or_none(ws), 0 if ws is None else ws.numel(), T, nC, D_OUT,
                                _abi.stream_of(x_flat))
    _abi.check(st, "k1_fwd")
    return out, inv_rms


def k1_bwd_dx(grad_out: torch.Tensor, x_flat: torch.Tensor, W: torch.Tensor,
              proj_out: torch.Tensor, inv_rms: torch.Tensor,
              grad_x: torch.Tensor | None = None) -> torch.Tensor:
    """grad of x_flat for K1, from the stored bf16 projection and inv_rms."""
    dev = _device_of(x_flat)
    if x_flat.dim() != 2:
        raise ValueError(f"x_flat must be 2-D (T, nC), got shape {tuple(x_flat.shape)}")
    T, nC = x_flat.shape
    _require(x_flat, "x_flat", _BF16, (T, nC), dev)
    _require(W, "W", _BF16, (D_OUT, nC), dev)
    _require(grad_out, "grad_out", _BF16, (T, D_OUT), dev)
    _require(proj_out, "proj_out", _BF16, (T, D_OUT), dev)
    _require(inv_rms, "inv_rms", _F32, (T,), dev)
    if grad_x is None:
        grad_x = torch.empty_like(x_flat)
    _require(grad_x, "grad_x", _BF16, (T, nC), dev)
    lib = _abi.load()
    with _OnDevice(dev):
        st = lib.fmhc_k1_bwd_dx(x_flat.data_ptr(), W.data_ptr(), grad_out.data_ptr(),
                                proj_out.data_ptr(), inv_rms.data_ptr(), grad_x.data_ptr(),
                                T, nC, D_OUT, _abi.stream_of(x_flat))
    _abi.check(st, "k1_bwd_dx")
    return grad_x


def k1_bwd(grad_out: torch.Tensor, x_flat: torch.Tensor, W: torch.Tensor,
           proj_out: torch.Tensor, inv_rms: torch.Tensor,
           grad_x: torch.Tensor | None = None,
           grad_W: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(grad_x, grad_W) of K1 in one pass over x; grad_W is (32, nC) bf16 and
    equals bf16(bf16(grad_out * inv_rms)^T @ x_flat) up to fp32 summation order."""
    dev = _device_of(x_flat)
    if x_flat.dim() != 2:
        raise ValueError(f"x_flat must be 2-D (T, nC), got shape {tuple(x_flat.shape)}")
    T, nC = x_flat.shape
    _require(x_flat, "x_flat", _BF16, (T, nC), dev)
    _require(W, "W", _BF16, (D_OUT, nC), dev)
    _require(grad_out, "grad_out", _BF16, (T, D_OUT), dev)
    _require(proj_out, "proj_out", _BF16, (T, D_OUT), dev)
    _require(inv_rms, "inv_rms", _F32, (T,), dev)
    if grad_x is None:
        grad_x = torch.empty_like(x_flat)
    if grad_W is None:
        grad_W = torch.empty((D_OUT, nC), device=dev, dtype=_BF16)
    _require(grad_x, "grad_x", _BF16, (T, nC), dev)
    _require(grad_W, "grad_W", _BF16, (D_OUT, nC), dev)
    lib = _abi.load()
    nbytes = int(lib.fmhc_k1_bwd_workspace_bytes(T, nC))
    ws = torch.empty((max(nbytes, 16),), device=dev, dtype=torch.uint8)
    with _OnDevice(dev):
        st = lib.fmhc_k1_bwd(x_flat.data_ptr(), W.data_ptr(), grad_out.data_ptr(), proj_out.data_ptr(),
                             inv_rms.data_ptr(), grad_x.data_ptr(), grad_W.data_ptr(), ws.data_ptr(),
                             ws.numel(), T, nC, D_OUT, _abi.stream_of(x_flat))
    _abi.check(st, "k1_bwd")
    return grad_x, grad_W


N_PERM = 24  # n! at n = 4


PARAM_DTYPES = {_F32: 0, _BF16: 1}  # FMHC_PARAM_F32, FMHC_PARAM_BF16


_K2_NAMES = ("alpha_pre", "alpha_post", "alpha_res", "bias", "perm")
_K2_SHAPES = ((1,), (1,), (1,), (D_OUT,), (N_PERM, N_STREAMS * N_STREAMS))


def _k2_params(alpha_pre, alpha_post, alpha_res, bias, perm, dev) -> int:
    """Check K2's parameters (all fp32 or all bf16) and return the ABI's dtype code."""
    dt = alpha_pre.dtype if isinstance(alpha_pre, torch.Tensor) else None
    code = PARAM_DTYPES.get(dt)
    if code is None:
        raise TypeError(f"K2 parameters must be float32 or bfloat16, got {dt}")
    ps = (alpha_pre, alpha_post, alpha_res, bias, perm)
    for t, shape in zip(ps, _K2_SHAPES):
        if (not isinstance(t, torch.Tensor) or t.dtype is not dt or t.shape != shape or t.device != dev
                or not t.is_contiguous()):
            break
    else:
        return code
    for t, name, shape in zip(ps, _K2_NAMES, _K2_SHAPES):
        _require(t, name, dt, shape, dev)
    return code


def k2_fwd(proj: torch.Tensor, alpha_pre: torch.Tensor, alpha_post: torch.Tensor,
           alpha_res: torch.Tensor, bias: torch.Tensor, perm: torch.Tensor
           ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(h_pre (T,4), h_post (T,4), H_merged (T,4,4)) fp32 from proj (T,32) bf16,
    with the bf16 rounding points of the reference's coefficient ops.
    Parameters: alphas (1,), bias (32,), perm (24,16), all fp32 or all bf16."""
    dev = _device_of(proj)
    if proj.dim() != 2:
        raise ValueError(f"proj must be 2-D (T, 32), got shape {tuple(proj.shape)}")
    T = proj.shape[0]
    _require(proj, "proj", _BF16, (T, D_OUT), dev)
    pdt = _k2_params(alpha_pre, alpha_post, alpha_res, bias, perm, dev)
    h_pre = torch.empty((T, N_STREAMS), device=dev, dtype=_F32)
    h_post = torch.empty((T, N_STREAMS), device=dev, dtype=_F32)
    H = torch.empty((T, N_STREAMS, N_STREAMS), device=dev, dtype=_F32)
    lib = _abi.load()
    with _OnDevice(dev):
        st = lib.fmhc_k2_fwd(proj.data_ptr(), alpha_pre.data_ptr(), alpha_post.data_ptr(),
                             alpha_res.data_ptr(), bias.data_ptr(), perm.data_ptr(), pdt, h_pre.data_ptr(),
                             h_post.data_ptr(), H.data_ptr(), T, N_STREAMS, _abi.stream_of(proj))
    _abi.check(st, "k2_fwd")
    return h_pre, h_post, H


def k2_bwd(proj: torch.Tensor, alpha_pre: torch.Tensor, alpha_post: torch.Tensor,
           alpha_res: torch.Tensor, bias: torch.Tensor, perm: torch.Tensor,
           grad_h_pre: torch.Tensor | None, grad_h_post: torch.Tensor | None,
           grad_H: torch.Tensor | None):
    """Gradients of k2_fwd: (grad_proj (T,32) bf16, grad_alpha_pre (1,),
    grad_alpha_post (1,), grad_alpha_res (1,), grad_bias (32,)), parameter
    gradients in the parameters' dtype.  A None output gradient counts as zero."""
    dev = _device_of(proj)
    if proj.dim() != 2:
        raise ValueError(f"proj must be 2-D (T, 32), got shape {tuple(proj.shape)}")
    T = proj.shape[0]
    _require(proj, "proj", _BF16, (T, D_OUT), dev)
    pdt = _k2_params(alpha_pre, alpha_post, alpha_res, bias, perm, dev)
    for t, name, shape in ((grad_h_pre, "grad_h_pre", (T, N_STREAMS)),
                           (grad_h_post, "grad_h_post", (T, N_STREAMS)),
                           (grad_H, "grad_H_merged", (T, N_STREAMS, N_STREAMS))):
        if t is not None:
            _require(t, name, _F32, shape, dev)
    grad_proj = torch.empty((T, D_OUT), device=dev, dtype=_BF16)
    g_ap = torch.empty((1,), device=dev, dtype=alpha_pre.dtype)
    g_apo = torch.empty((1,), device=dev, dtype=alpha_pre.dtype)
    g_ar = torch.empty((1,), device=dev, dtype=alpha_pre.dtype)
    g_b = torch.empty((D_OUT,), device=dev, dtype=alpha_pre.dtype)
    lib = _abi.load()
    nbytes = int(lib.fmhc_k2_bwd_workspace_bytes(T))
    ws = torch.empty((max(nbytes, 16),), device=dev, dtype=torch.uint8)
    ptr = lambda t: None if t is None else t.data_ptr()
    with _OnDevice(dev):
        st = lib.fmhc_k2_bwd(proj.data_ptr(), alpha_pre.data_ptr(), alpha_post.data_ptr(),
                             alpha_res.data_ptr(), bias.data_ptr(), perm.data_ptr(), pdt, ptr(grad_h_pre),
                             ptr(grad_h_post), ptr(grad_H), grad_proj.data_ptr(), g_ap.data_ptr(),
                             g_apo.data_ptr(), g_ar.data_ptr(), g_b.data_ptr(), ws.data_ptr(), ws.numel(),
                             T, N_STREAMS, _abi.stream_of(proj))
    _abi.check(st, "k2_bwd")
    return grad_proj, g_ap, g_apo, g_ar, g_b


def premap_fwd(x_streams: torch.Tensor, W: torch.Tensor, alpha_pre: torch.Tensor,
               alpha_post: torch.Tensor, alpha_res: torch.Tensor, bias: torch.Tensor,
               perm: torch.Tensor, layer_input: bool = True, zero: tuple = ()):
    """K1 + K2 + K3: (layer_input (T,C) bf16, H_merged (T,4,4), h_post (T,4),
    h_pre (T,4) fp32, proj (T,32) bf16, inv_rms (T,) fp32).  layer_input=False:
    K1 + K2 only, the first output is None.  zero: up to two 16-bit tensors
    whose first stored element the same launches set to zero (zero-stride
    placeholders; empty ones are skipped)."""
    if len(zero) > 2 or any(z.element_size() != 2 for z in zero):
        raise ValueError("premap_fwd: zero takes up to two 16-bit tensors")
    zw = [z.data_ptr() if z.numel() > 0 else None for z in zero] + [None, None]
    T, n, C = _streams_shape(x_streams)
    dev = _device_of(x_streams)
    _require(x_streams, "x_streams", _BF16, (T, n, C), dev)
    _require(W, "W", _BF16, (D_OUT, n * C), dev)
    pdt = _k2_params(alpha_pre, alpha_post, alpha_res, bias, perm, dev)
    li = torch.empty((T, C), device=dev, dtype=_BF16) if layer_input else None
    proj = torch.empty((T, D_OUT), device=dev, dtype=_BF16)
    inv = torch.empty((T,), device=dev, dtype=_F32)
    h_pre = torch.empty((T, n), device=dev, dtype=_F32)
    h_post = torch.empty((T, n), device=dev, dtype=_F32)
    H = torch.empty((T, n, n), device=dev, dtype=_F32)
    lib = _abi.load()
    ws = _workspace(int(lib.fmhc_premap_fwd_workspace_bytes(T, C)), dev)
    with _OnDevice(dev):
        st = lib.fmhc_premap_fwd(x_streams.data_ptr(), W.data_ptr(), alpha_pre.data_ptr(),
                                 alpha_post.data_ptr(), alpha_res.data_ptr(), bias.data_ptr(),
                                 perm.data_ptr(), pdt, _ptr_or_none(li), proj.data_ptr(), inv.data_ptr(),
                                 h_pre.data_ptr(), h_post.data_ptr(), H.data_ptr(), zw[0], zw[1],
                                 _ptr_or_none(ws), 0 if ws is None else ws.numel(), T, C, n,
                                 _abi.stream_of(x_streams))
    _abi.check(st, "premap_fwd")
    return li, H, h_post, h_pre, proj, inv


_PREMAP_WS_BYTES: dict[tuple[int, int], int] = {}


def _premap_ws_bytes(lib, T: int, C: int) -> int:
    key = (T, C)
    n = _PREMAP_WS_BYTES.get(key)
    if n is None:
        if len(_PREMAP_WS_BYTES) > 4096:
            _PREMAP_WS_BYTES.clear()
        n = _PREMAP_WS_BYTES[key] = int(lib.fmhc_premap_fwd_workspace_bytes(T, C))
    return n


def premap_fwd_eval(x_streams: torch.Tensor, W: torch.Tensor, alpha_pre: torch.Tensor,
                    alpha_post: torch.Tensor, alpha_res: torch.Tensor, bias: torch.Tensor,
                    perm: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """premap_fwd for a forward that records no autograd graph: the same
    launch, returning (layer_input, coeffs).  coeffs is one uint8 scratch
    buffer that holds H_merged (T, 4, 4) fp32 at byte 0 and h_post (T, 4)
    fp32 at byte 64 T, the inputs k4_fwd_eval reads, followed by h_pre, proj,
    inv_rms and the workspace, which nothing reads after the call: one
    allocation instead of six."""
    dev = x_streams.device
    shape = x_streams.shape
    if (len(shape) != 3 or shape[1] != N_STREAMS or dev.type != "cuda" or x_streams.dtype is not _BF16
            or not x_streams.is_contiguous() or W.dtype is not _BF16 or W.device != dev
            or W.shape != (D_OUT, N_STREAMS * shape[2]) or not W.is_contiguous()):
        T, n, C = _streams_shape(x_streams)
        dev = _device_of(x_streams)
        _require(x_streams, "x_streams", _BF16, (T, n, C), dev)
        _require(W, "W", _BF16, (D_OUT, n * C), dev)
    T, n, C = shape
    pdt = _k2_params(alpha_pre, alpha_post, alpha_res, bias, perm, dev)
    lib = _abi.load()
    ws_bytes = _premap_ws_bytes(lib, T, C)
    li = torch.empty((T, C), device=dev, dtype=_BF16)
    # H_merged | h_post | h_pre | inv_rms | proj | workspace, 16-byte aligned pieces
    o_hq, o_hp, o_inv = 64 * T, 80 * T, 96 * T
    o_proj = (o_inv + 4 * T + 15) // 16 * 16
    o_ws = (o_proj + 2 * D_OUT * T + 255) // 256 * 256
    coeffs = torch.empty((o_ws + ws_bytes,), device=dev, dtype=torch.uint8)
    base = coeffs.data_ptr()
    with _OnDevice(dev):
        st = lib.fmhc_premap_fwd(x_streams.data_ptr(), W.data_ptr(), alpha_pre.data_ptr(),
                                 alpha_post.data_ptr(), alpha_res.data_ptr(), bias.data_ptr(),
                                 perm.data_ptr(), pdt, li.data_ptr(), base + o_proj, base + o_inv, base + o_hp,
                                 base + o_hq, base, None, None,
                                 base + o_ws if ws_bytes else None, ws_bytes, T, C, n, _abi.stream_of(x_streams))
    _abi.check(st, "premap_fwd")
    return li, coeffs


def premap_bwd(x_streams: torch.Tensor, W: torch.Tensor, alpha_pre: torch.Tensor,
               alpha_post: torch.Tensor, alpha_res: torch.Tensor, bias: torch.Tensor,
               perm: torch.Tensor, h_pre: torch.Tensor, proj: torch.Tensor, inv_rms: torch.Tensor,
               grad_layer_input: torch.Tensor, grad_h_post: torch.Tensor | None,
               grad_H: torch.Tensor | None, grad_x_in: torch.Tensor | None = None):
    """Gradients of premap_fwd's inputs: (grad_x (T,4,C) bf16, grad_W (32,4C) bf16,
    grad_alpha_pre, grad_alpha_post, grad_alpha_res (1,), grad_bias (32,) in the parameters' dtype).
    grad_x_in (T,4,C) bf16, optional: a further gradient of x, added (bf16) into grad_x."""
    T, n, C = _streams_shape(x_streams)
    dev = _device_of(x_streams)
    _require(x_streams, "x_streams", _BF16, (T, n, C), dev)
    _require(W, "W", _BF16, (D_OUT, n * C), dev)
    pdt = _k2_params(alpha_pre, alpha_post, alpha_res, bias, perm, dev)
    _require(h_pre, "h_pre", _F32, (T, n), dev)
    _require(proj, "proj", _BF16, (T, D_OUT), dev)
    _require(inv_rms, "inv_rms", _F32, (T,), dev)
    _require(grad_layer_input, "grad_layer_input", _BF16, (T, C), dev)
    if grad_h_post is not None:
        _require(grad_h_post, "grad_h_post", _F32, (T, n), dev)
    if grad_H is not None:
        _require(grad_H, "grad_H_merged", _F32, (T, n, n), dev)
    if grad_x_in is not None:
        _require(grad_x_in, "grad_x_in", _BF16, (T, n, C), dev)
    gx = torch.empty_like(x_streams)
    gW = torch.empty((D_OUT, n * C), device=dev, dtype=_BF16)
    ga = [torch.empty((1,), device=dev, dtype=alpha_pre.dtype) for _ in range(3)]
    gb = torch.empty((D_OUT,), device=dev, dtype=alpha_pre.dtype)
    lib = _abi.load()
    nbytes = int(lib.fmhc_premap_bwd_workspace_bytes(T, C))
    ws = torch.empty((max(nbytes, 16),), device=dev, dtype=torch.uint8)
    ptr = lambda t: None if t is None else t.data_ptr()
    with _OnDevice(dev):
        st = lib.fmhc_premap_bwd(x_streams.data_ptr(), W.data_ptr(), alpha_pre.data_ptr(),
                                 alpha_post.data_ptr(), alpha_res.data_ptr(), bias.data_ptr(),
                                 perm.data_ptr(), pdt, h_pre.data_ptr(), proj.data_ptr(), inv_rms.data_ptr(),
                                 grad_layer_input.data_ptr(), ptr(grad_h_post), ptr(grad_H), ptr(grad_x_in),
                                 gx.data_ptr(),
                                 gW.data_ptr(), ga[0].data_ptr(), ga[1].data_ptr(), ga[2].data_ptr(),
                                 gb.data_ptr(), ws.data_ptr(), ws.numel(), T, C, n, _abi.stream_of(x_streams))
    _abi.check(st, "premap_bwd")
    return gx, gW, ga[0], ga[1], ga[2], gb


def _workspace(nbytes: int, dev) -> torch.Tensor | None:
    """A uint8 device buffer of nbytes (16-byte aligned: torch's allocations are), or None for 0."""
    return torch.empty((nbytes,), device=dev, dtype=torch.uint8) if nbytes > 0 else None


def _ptr_or_none(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def _streams_shape(x: torch.Tensor) -> tuple[int, int, int]:
    if x.dim() != 3:
        raise ValueError(f"x_streams must be 3-D (T, n, C), got shape {tuple(x.shape)}")
    T, n, C = x.shape
    if n != N_STREAMS:
        raise ValueError(f"flash_mhc HIP kernels support n={N_STREAMS} only, got n={n}")
    return T, n, C


def k3_fwd(x_streams: torch.Tensor, h_pre: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """layer_input (T, C) bf16 = sum_j h_pre[:, j] * x_streams[:, j, :]."""
    dev = _device_of(x_streams)
    T, n, C = _streams_shape(x_streams)
    _require(x_streams, "x_streams", _BF16, (T, n, C), dev)
    _require(h_pre, "h_pre", _F32, (T, n), dev)
    if out is None:
        out = torch.empty((T, C), device=dev, dtype=_BF16)
    _require(out, "out", _BF16, (T, C), dev)
    lib = _abi.load()
    with _OnDevice(dev):
        st = lib.fmhc_k3_fwd(x_streams.data_ptr(), h_pre.data_ptr(), out.data_ptr(), T, C, n,
                             _abi.stream_of(x_streams))
    _abi.check(st, "k3_fwd")
    return out


def k3_bwd(grad_out: torch.Tensor, x_streams: torch.Tensor, h_pre: torch.Tensor,
           grad_x: torch.Tensor | None = None,
           grad_h_pre: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(grad_x (T, n, C) bf16, grad_h_pre (T, n) fp32) of K3."""
    dev = _device_of(x_streams)
    T, n, C = _streams_shape(x_streams)
    _require(x_streams, "x_streams", _BF16, (T, n, C), dev)
    _require(h_pre, "h_pre", _F32, (T, n), dev)
    _require(grad_out, "grad_out", _BF16, (T, C), dev)
    if grad_x is None:
        grad_x = torch.empty_like(x_streams)
    if grad_h_pre is None:
        grad_h_pre = torch.empty((T, n), device=dev, dtype=_F32)
    _require(grad_x, "grad_x", _BF16, (T, n, C), dev)
    _require(grad_h_pre, "grad_h_pre", _F32, (T, n), dev)
    lib = _abi.load()
    with _OnDevice(dev):
        st = lib.fmhc_k3_bwd(x_streams.data_ptr(), h_pre.data_ptr(), grad_out.data_ptr(),
                             grad_x.data_ptr(), grad_h_pre.data_ptr(), T, C, n,
                             _abi.stream_of(x_streams))
    _abi.check(st, "k3_bwd")
    return grad_x, grad_h_pre


def k4_fwd(x_streams: torch.Tensor, layer_output: torch.Tensor, H_merged: torch.Tensor,
           h_post: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """out (T, n, C) bf16 = H_merged @ x_streams + h_post (x) layer_output."""
    dev = _device_of(x_streams)
    T, n, C = _streams_shape(x_streams)
    _require(x_streams, "x_streams", _BF16, (T, n, C), dev)
    _require(layer_output, "layer_output", _BF16, (T, C), dev)
    _require(H_merged, "H_merged", _F32, (T, n, n), dev)
    _require(h_post, "h_post", _F32, (T, n), dev)
    if out is None:
        out = torch.empty_like(x_streams)
    _require(out, "out", _BF16, (T, n, C), dev)
    lib = _abi.load()
    with _OnDevice(dev):
        st = lib.fmhc_k4_fwd(x_streams.data_ptr(), layer_output.data_ptr(), H_merged.data_ptr(),
                             h_post.data_ptr(), out.data_ptr(), T, C, n, _abi.stream_of(x_streams))
    _abi.check(st, "k4_fwd")
    return out


def k4_fwd_eval(x_streams: torch.Tensor, layer_output: torch.Tensor, coeffs: torch.Tensor) -> torch.Tensor:
    """k4_fwd with H_merged and h_post read from premap_fwd_eval's coeffs
    buffer for the same x_streams."""
    dev = x_streams.device
    shape = x_streams.shape
    if (len(shape) != 3 or shape[1] != N_STREAMS or dev.type != "cuda" or x_streams.dtype is not _BF16
            or not x_streams.is_contiguous() or layer_output.dtype is not _BF16 or layer_output.device != dev
            or layer_output.shape != (shape[0], shape[2]) or not layer_output.is_contiguous()):
        T, n, C = _streams_shape(x_streams)
        dev = _device_of(x_streams)
        _require(x_streams, "x_streams", _BF16, (T, n, C), dev)
        _require(layer_output, "layer_output", _BF16, (T, C), dev)
    T, n, C = shape
    if coeffs.dtype is not torch.uint8 or coeffs.numel() < 80 * T or coeffs.device != dev:
        raise ValueError("coeffs is not premap_fwd_eval's buffer for these tokens")
    out = torch.empty_like(x_streams)
    lib = _abi.load()
    base = coeffs.data_ptr()
    with _OnDevice(dev):
        st = lib.fmhc_k4_fwd(x_streams.data_ptr(), layer_output.data_ptr(), base, base + 64 * T,
                             out.data_ptr(), T, C, n, _abi.stream_of(x_streams))
    _abi.check(st, "k4_fwd")
    return out


def k4_bwd(grad_out: torch.Tensor, x_streams: torch.Tensor, layer_output: torch.Tensor,
           H_merged: torch.Tensor, h_post: torch.Tensor,
           grad_x: torch.Tensor | None = None, grad_layer_output: torch.Tensor | None = None,
           grad_H: torch.Tensor | None = None, grad_h_post: torch.Tensor | None = None):
    """(grad_x, grad_layer_output, grad_H_merged, grad_h_post) of K4."""
    dev = _device_of(x_streams)
    T, n, C = _streams_shape(x_streams)
    _require(x_streams, "x_streams", _BF16, (T, n, C), dev)
    _require(layer_output, "layer_output", _BF16, (T, C), dev)
    _require(H_merged, "H_merged", _F32, (T, n, n), dev)
    _require(h_post, "h_post", _F32, (T, n), dev)
    _require(grad_out, "grad_out", _BF16, (T, n, C), dev)
    if grad_x is None:
        grad_x = torch.empty_like(x_streams)
    if grad_layer_output is None:
        grad_layer_output = torch.empty((T, C), device=dev, dtype=_BF16)
    if grad_H is None:
        grad_H = torch.empty((T, n, n), device=dev, dtype=_F32)
    if grad_h_post is None:
        grad_h_post = torch.empty((T, n), device=dev, dtype=_F32)
    _require(grad_x, "grad_x", _BF16, (T, n, C), dev)
    _require(grad_layer_output, "grad_layer_output", _BF16, (T, C), dev)
    _require(grad_H, "grad_H", _F32, (T, n, n), dev)
    _require(grad_h_post, "grad_h_post", _F32, (T, n), dev)
    lib = _abi.load()
    with _OnDevice(dev):
        st = lib.fmhc_k4_bwd(x_streams.data_ptr(), layer_output.data_ptr(), H_merged.data_ptr(),
                             h_post.data_ptr(), grad_out.data_ptr(), grad_x.data_ptr(),
                             grad_layer_output.data_ptr(), grad_H.data_ptr(), grad_h_post.data_ptr(),
                             T, C, n, _abi.stream_of(x_streams))
    _abi.check(st, "k4_bwd")
    return grad_x, grad_layer_output, grad_H, grad_h_post
