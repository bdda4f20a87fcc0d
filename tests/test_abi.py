"""CPU tests of the C ABI library: it loads without a GPU, exports every
function include/flash_mhc_hip.h declares, and rejects bad arguments on the
host before any launch.  No kernel is launched here."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from flash_mhc import _abi

ROOT = Path(__file__).resolve().parents[1]
HEADERS = [ROOT / "include" / "flash_mhc_hip.h"]  # the product library's ABI
PROBE_HEADER = ROOT / "include" / "flash_mhc_probe.h"  # bench.py's probe library
PROBE_LIB = _abi.LIB_PATH.parent / "libflash_mhc_probe.so"


def declared_functions(headers=HEADERS) -> set[str]:
    names = set()
    for h in headers:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(fmhc_\w+)\s*\(", text))
    return names


def test_every_header_is_checked():
    assert sorted((ROOT / "include").glob("*.h")) == sorted(HEADERS + [PROBE_HEADER])


def test_header_declares_the_abi():
    names = declared_functions()
    assert {"fmhc_k1_fwd", "fmhc_k1_bwd_dx", "fmhc_k3_fwd", "fmhc_k3_bwd", "fmhc_k4_fwd",
            "fmhc_k4_bwd", "fmhc_error_string", "fmhc_abi_version"} <= names
    assert names == set(_abi.SIGNATURES), "ctypes bindings and header disagree"


def test_library_exports_every_declared_symbol():
    path = _abi.lib_path()
    assert path.exists(), f"build the extension first: {path}"
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\b(fmhc_\w+)\b", out))
    missing = declared_functions() - exported
    assert not missing, missing


def test_probe_library_is_separate():
    """The bandwidth probe lives in its own library (bench.py only): the
    product library exports none of its symbols, and the probe library
    exports every function its header declares."""
    assert PROBE_LIB.exists(), f"build the extension first: {PROBE_LIB}"
    probe = declared_functions([PROBE_HEADER])
    assert probe == {"fmhc_stream_probe", "fmhc_probe_abi_version"}
    out = subprocess.run(["nm", "-D", "--defined-only", str(PROBE_LIB)], capture_output=True, text=True,
                         check=True).stdout
    assert probe <= set(re.findall(r"\b(fmhc_\w+)\b", out))
    main = subprocess.run(["nm", "-D", "--defined-only", str(_abi.lib_path())], capture_output=True, text=True,
                          check=True).stdout
    assert not probe & set(re.findall(r"\b(fmhc_\w+)\b", main))
    lib = ctypes.CDLL(str(PROBE_LIB))
    assert lib.fmhc_probe_abi_version() == 2
    # Host-side argument checks (no launch): odd size, unknown kind, null source.
    lib.fmhc_stream_probe.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                      ctypes.c_void_p]
    assert lib.fmhc_stream_probe(0, _FAKE, _FAKE, 15, None) == 1
    assert lib.fmhc_stream_probe(9, _FAKE, _FAKE, 16, None) == 1
    assert lib.fmhc_stream_probe(3, None, _FAKE, 16, None) == 1


def test_library_is_gfx950_code():
    path = _abi.lib_path()
    blob = path.read_bytes()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob  # device code object for gfx950


def test_loads_and_reports_version():
    lib = _abi.load()
    assert lib.fmhc_abi_version() == _abi.ABI_VERSION
    assert lib.fmhc_error_string(0) == b"ok"
    assert b"invalid argument" in lib.fmhc_error_string(1)
    assert lib.fmhc_error_string(123) == b"unknown flash_mhc status"
    assert b"no-allocation" in lib.fmhc_error_string(2)


_FAKE = 4096  # a non-null address that the host-side checks never dereference


@pytest.mark.parametrize(
    "call",
    [
        lambda L: L.fmhc_k3_fwd(None, None, None, 8, 16, 3, None),        # n != 4
        lambda L: L.fmhc_k3_fwd(None, None, None, -1, 16, 4, None),       # T < 0
        lambda L: L.fmhc_k3_fwd(None, None, None, 8, 0, 4, None),         # C == 0
        lambda L: L.fmhc_k3_fwd(None, None, None, 8, 16, 4, None),        # null pointers
        lambda L: L.fmhc_k3_bwd(None, None, None, None, None, 8, 16, 5, None),
        lambda L: L.fmhc_k4_fwd(None, None, None, None, None, 8, 16, 2, None),
        lambda L: L.fmhc_k4_bwd(None, None, None, None, None, None, None, None, None, 8, 16, 4, None),
        lambda L: L.fmhc_k1_fwd(None, None, None, None, 8, 64, 31, None),  # D_out != 32
        lambda L: L.fmhc_k1_fwd(None, None, None, None, 8, 64, 32, None),  # null pointers
        lambda L: L.fmhc_k1_bwd_dx(None, None, None, None, None, None, 8, 0, 32, None),
        lambda L: L.fmhc_k1_fwd_ws(None, None, None, None, None, 0, 8, 64, 32, None),  # null pointers
        # K2 parameter dtype other than FMHC_PARAM_F32 (0) / FMHC_PARAM_BF16 (1)
        lambda L: L.fmhc_k2_fwd(*[_FAKE] * 6, 2, *[_FAKE] * 3, 8, 4, None),
        lambda L: L.fmhc_k2_fwd(*[None] * 6, 0, *[None] * 3, 8, 4, None),  # null parameters
        lambda L: L.fmhc_premap_fwd(*[_FAKE] * 7, -1, *[_FAKE] * 6, None, None, None, 0, 8, 16, 4, None),
        lambda L: L.fmhc_premap_fwd_noalloc(*[_FAKE] * 7, 0, *[_FAKE] * 6, None, None, 8, 16, 5, None),  # n != 4
        lambda L: L.fmhc_premap_fwd_noalloc(*[_FAKE] * 7, 0, *[_FAKE] * 6, None, None, -3, 16, 4, None),
        # C beyond the pre-map's 2^24 (its int offsets), forward and backward
        lambda L: L.fmhc_premap_fwd(*[_FAKE] * 7, 0, *[_FAKE] * 6, None, None, _FAKE, 1 << 40, 8, (1 << 24) + 8,
                                    4, None),
        lambda L: L.fmhc_premap_bwd(*[_FAKE] * 7, 0, *[_FAKE] * 14, 1 << 40, 8, (1 << 24) + 8, 4, None),
    ],
)
def test_invalid_arguments_rejected_before_launch(call):
    assert call(_abi.load()) == 1


def test_empty_batch_is_a_noop():
    lib = _abi.load()
    assert lib.fmhc_k3_fwd(None, None, None, 0, 16, 4, None) == 0
    assert lib.fmhc_k4_bwd(None, None, None, None, None, None, None, None, None, 0, 16, 4, None) == 0
    assert lib.fmhc_k1_fwd(None, None, None, None, 0, 64, 32, None) == 0


def test_check_raises_runtime_error():
    with pytest.raises(RuntimeError, match="status 1"):
        _abi.check(1, "k3_fwd")
    _abi.check(0, "k3_fwd")


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setenv("FLASH_MHC_HIP_LIB", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_abi, "_lib", None)
    with pytest.raises(_abi.ExtensionMissingError):
        _abi.load()
    assert not _abi.is_available()


def test_shares_torchs_hip_runtime():
    """Loading the extension maps no second libamdhip64 (soname resolution
    binds it to the runtime torch loaded)."""
    _abi.load()
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            if "libamdhip64" in line:
                paths.add(line.split()[-1])
    assert len(paths) <= 1, paths


def test_ctypes_signatures_cover_argument_counts():
    text = re.sub(r"/\*.*?\*/", "", "\n".join(h.read_text() for h in HEADERS), flags=re.S)
    for name, argtypes in _abi.SIGNATURES.items():
        m = re.search(rf"\b{name}\s*\((.*?)\)\s*;", text, flags=re.S)
        assert m, name
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(argtypes), (name, params)
        assert all(isinstance(a, type) and issubclass(a, ctypes._SimpleCData) for a in argtypes)


def test_noalloc_scratch_covers_every_shape():
    """fmhc_premap_fwd_noalloc's static scratch (4 MiB) holds the column-split
    partial sums of every shape: the workspace sizing (a host computation) over
    every T the split takes (T <= 1024 up to C = 1024, T <= 2720 above) and C
    up to 4096 peaks at 2,145,792 bytes, reached at T = 2032, C = 1040."""
    lib = _abi.load()
    f = lib.fmhc_premap_fwd_workspace_bytes
    assert f(2032, 1040) == 2145792
    assert f(2032, 1024) == 0 and f(1024, 1024) > 0  # rows up to 64 chunks: T <= 1024
    assert f(2721, 4096) == 0 and f(2720, 4096) > 0
    assert f(4096, 1024) == 0 and f(0, 1024) == 0
    peak = 0
    for C in range(8, 4097, 8):
        for T in list(range(1, 129)) + list(range(1904, 2721)):
            peak = max(peak, f(T, C))
    assert peak == 2145792 <= 4 << 20
