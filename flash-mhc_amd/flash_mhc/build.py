"""Build the gfx950 HIP extension ``_lib/libflash_mhc_hip.so`` in-tree, and
beside it ``_lib/libflash_mhc_probe.so``, the bandwidth probe and cache flush
that only bench.py loads (include/flash_mhc_probe.h; not part of the path),
and the evidence variants of VARIANTS (``_lib/libflash_mhc_hip_<name>.so``,
same ABI; nothing loads them unless FLASH_MHC_HIP_LIB names one).

Usage: ``python -m flash_mhc.build`` (run from ``flash-mhc_amd/``) or
``flash_mhc.build.build()``.  hipcc cross-compiles for gfx950 without a GPU.

Every HIP source is compiled with ``-Xclang -target-feature -Xclang
-packed-fp32-ops`` so the compiler never emits packed fp32 VALU instructions
(v_pk_add/mul/fma_f32); the host pass prints a harmless "not a recognized
feature" warning for it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent  # flash-mhc_amd/
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
BUILD_DIR = ROOT / "_build"
LIB_DIR = PKG_DIR / "_lib"
LIB_NAME = "libflash_mhc_hip.so"
LIB_PATH = LIB_DIR / LIB_NAME
PROBE_LIB_PATH = LIB_DIR / "libflash_mhc_probe.so"

SOURCES = ("k1.hip", "k2.hip", "k3.hip", "k4.hip", "premap.hip", "premap_resident.hip", "premap_split.hip",
           "abi.hip")
PROBE_SOURCES = ("stream_probe.hip",)

ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]

# Per-source flags.  k1.hip: let the MFMA accumulators live in ordinary VGPRs
# (gfx950 allows VGPR srcC/dst).  Without it the compiler keeps the backward's
# loop-carried weight-gradient accumulators in VGPRs and copies them to and
# from AGPRs around every MFMA, which doubles the kernel's register footprint.
SOURCE_FLAGS = {"k1.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
                "premap_resident.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}

# Evidence builds of the same library, selected at compile time.  k1_valu: the
# K1 forward and backward-dx contractions as fp32 FMAs on the VALU instead of
# the matrix cores (same tiles, loads and pipeline), to time the two.
# premap_three_kernels: the pre-map forward of many tokens as K1, K2, K3 in
# three kernels, against the product's one kernel (K1 on a tile of 16 to 64
# tokens, then K2 and K3 on it by the same workgroup).  premap_tile_nt: the one kernel
# with nontemporal loads of x in its K1 part, so that its K3 part re-reads the
# tile from HBM instead of the memory-side cache.  premap_reread: the forward's
# tile kernel instead of the single read.  premap_bwd_split: the pre-map
# backward with one read of x (premap_split.hip) instead of K3's reduce pass,
# K2 and K1.  no_lds_cap: K1's backward dx, K3 and K4 launched without the
# residency caps of fmhc_common.h.
VARIANTS = {"k1_valu": ["-DFMHC_K1_VALU=1"], "premap_three_kernels": ["-DFMHC_PREMAP_TILE=0"],
            "premap_tile_nt": ["-DFMHC_PREMAP_TILE_NT=1"], "premap_reread": ["-DFMHC_PREMAP_RESIDENT=0"],
            "premap_bwd_split": ["-DFMHC_PREMAP_SPLIT=1"], "no_lds_cap": ["-DFMHC_LDS_CAP=0"]}


def variant_path(name: str) -> Path:
    return LIB_DIR / f"libflash_mhc_hip_{name}.so"


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the HIP toolchain (ROCm) is required to build flash_mhc")
    return exe


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            f"command failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}"
        )
    if verbose:
        # Drop the host pass's warning about the device-only target feature.
        noise = "packed-fp32-ops' is not a recognized feature"
        for line in (proc.stdout + proc.stderr).splitlines():
            if noise not in line and line.strip():
                print(line)


def _link(cc: str, objs: list[Path], out: Path, verbose: bool) -> None:
    tmp = out.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, out)


def build(verbose: bool = False, extra_flags: list[str] | None = None, out: Path | None = None,
          probe: bool = True) -> Path:
    """Compile every HIP source and link the shared library (and, with probe,
    the probe library beside the default one). Returns the library's path.

    extra_flags / out build a variant of the library under another name (its
    objects go to a build directory of their own)."""
    cc = hipcc()
    out = Path(out) if out is not None else LIB_PATH
    build_dir = BUILD_DIR if out == LIB_PATH else BUILD_DIR / out.stem
    build_dir.mkdir(parents=True, exist_ok=True)
    out.parent.mkdir(parents=True, exist_ok=True)
    flags = COMMON_FLAGS + [f"-I{INCLUDE}"] + list(extra_flags or [])
    sources = SOURCES + (PROBE_SOURCES if probe and out == LIB_PATH else ())

    def compile_one(src: str) -> Path:
        obj = build_dir / (Path(src).stem + ".o")
        _run([cc, *flags, *SOURCE_FLAGS.get(src, []), "-c", str(CSRC / src), "-o", str(obj)], verbose)
        return obj

    jobs = min(len(sources), max(1, (os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = dict(zip(sources, ex.map(compile_one, sources)))
    _link(cc, [objs[s] for s in SOURCES], out, verbose)
    if probe and out == LIB_PATH:
        _link(cc, [objs[s] for s in PROBE_SOURCES], PROBE_LIB_PATH, verbose)
    return out


def build_variants(verbose: bool = False) -> list[Path]:
    """Every evidence variant (nothing on the product path loads them; their
    GPU tests skip when they are absent)."""
    return [build(verbose=verbose, extra_flags=flags, out=variant_path(name), probe=False)
            for name, flags in VARIANTS.items()]


def build_all(verbose: bool = False) -> Path:
    """The product library, the probe library and every evidence variant."""
    path = build(verbose=verbose)
    build_variants(verbose=verbose)
    return path


if __name__ == "__main__":
    # python -m flash_mhc.build [-v] [--variants]: the product and probe
    # libraries, and with --variants the evidence builds too.
    verbose = "-v" in sys.argv
    path = build_all(verbose=verbose) if "--variants" in sys.argv else build(verbose=verbose)
    print(path)
