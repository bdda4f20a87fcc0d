"""ctypes binding of the C ABI in ``include/flash_mhc_hip.h``.

The shared library is built in-tree by :mod:`flash_mhc.build` into
``flash_mhc/_lib/libflash_mhc_hip.so``.  It is loaded after ``import torch`` so
that its ``libamdhip64.so.7`` dependency resolves (by soname) to the HIP
runtime torch already loaded: torch's streams and the library's kernels then
belong to one runtime.

There is no fallback: if the library is missing, every fused op raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  # load torch's HIP runtime before the extension

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libflash_mhc_hip.so"

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int

# name -> argtypes, following include/flash_mhc_hip.h
SIGNATURES: dict[str, list] = {
    "fmhc_k1_fwd": [_P, _P, _P, _P, _I64, _I64, _I64, _P],
    "fmhc_k1_fwd_ws": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "fmhc_k1_fwd_workspace_bytes": [_I64, _I64],
    "fmhc_k1_bwd_dx": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "fmhc_k1_bwd": [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "fmhc_k1_bwd_workspace_bytes": [_I64, _I64],
    "fmhc_k2_fwd": [_P] * 6 + [_INT] + [_P] * 3 + [_I64, _I64, _P],
    "fmhc_k2_bwd": [_P] * 6 + [_INT] + [_P] * 9 + [_I64, _I64, _I64, _P],
    "fmhc_k2_bwd_workspace_bytes": [_I64],
    "fmhc_premap_fwd": [_P] * 7 + [_INT] + [_P] * 9 + [_I64, _I64, _I64, _I64, _P],
    "fmhc_premap_fwd_workspace_bytes": [_I64, _I64],
    "fmhc_premap_fwd_noalloc": [_P] * 7 + [_INT] + [_P] * 8 + [_I64, _I64, _I64, _P],
    "fmhc_premap_bwd": [_P] * 7 + [_INT] + [_P] * 14 + [_I64, _I64, _I64, _I64, _P],
    "fmhc_premap_bwd_workspace_bytes": [_I64, _I64],
    "fmhc_k3_fwd": [_P, _P, _P, _I64, _I64, _I64, _P],
    "fmhc_k3_bwd": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "fmhc_k4_fwd": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "fmhc_k4_bwd": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "fmhc_error_string": [ctypes.c_int],
    "fmhc_abi_version": [],
}
RESTYPES = {
    "fmhc_error_string": ctypes.c_char_p,
    "fmhc_k1_bwd_workspace_bytes": ctypes.c_int64,
    "fmhc_k1_fwd_workspace_bytes": ctypes.c_int64,
    "fmhc_premap_fwd_workspace_bytes": ctypes.c_int64,
    "fmhc_k2_bwd_workspace_bytes": ctypes.c_int64,
    "fmhc_premap_bwd_workspace_bytes": ctypes.c_int64,
}

ABI_VERSION = 7

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class ExtensionMissingError(RuntimeError):
    """The HIP extension has not been built (or failed to load)."""


def lib_path() -> Path:
    override = os.environ.get("FLASH_MHC_HIP_LIB")
    return Path(override) if override else LIB_PATH


def load() -> ctypes.CDLL:
    """Load (once) and return the extension; raise if it is unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = lib_path()
        if not path.exists():
            raise ExtensionMissingError(
                f"flash_mhc HIP extension not found at {path}. Build it with "
                "`python -m flash_mhc.build` (hipcc, --offload-arch=gfx950)."
            )
        try:
            lib = ctypes.CDLL(str(path), mode=ctypes.RTLD_LOCAL)
        except OSError as e:
            raise ExtensionMissingError(f"failed to load {path}: {e}") from e
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, ctypes.c_int)
        version = lib.fmhc_abi_version()
        if version != ABI_VERSION:
            raise ExtensionMissingError(
                f"{path} has ABI version {version}, expected {ABI_VERSION}; rebuild it"
            )
        _lib = lib
        return lib


def is_available() -> bool:
    try:
        load()
        return True
    except ExtensionMissingError:
        return False


def check(status: int, what: str) -> None:
    """Turn a non-zero C status into a RuntimeError."""
    if status != 0:
        msg = load().fmhc_error_string(status).decode("utf-8", "replace")
        raise RuntimeError(f"flash_mhc {what} failed with status {status}: {msg}")


def ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t of torch's current stream on ``t``'s device (the raw handle
    query avoids building a Stream object per launch)."""
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream
