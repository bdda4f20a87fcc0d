"""CPU tests of bench.py's command line: it measures one GPU only, and says so
for --gpus N > 1 (exit status 2, before touching a GPU); it takes the reference
benchmark's flags (--n 4 only, --peak-gbps, --iters, --seed)."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""  # no JSON line


def _bench(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=300, cwd=ROOT, env={**os.environ, "CUDA_VISIBLE_DEVICES": "", "HIP_VISIBLE_DEVICES": ""})


def test_bench_refuses_other_stream_counts():
    r = _bench("--n", "3")
    assert r.returncode == 2
    assert "n = 4 only" in r.stderr
    assert r.stdout == ""


def test_bench_accepts_the_reference_benchmark_command_line():
    # scripts/benchmark_kernels.py's documented invocation; without a GPU the
    # parse succeeds and bench.py stops at the device check.
    r = _bench("--T", "65536", "--C", "1024", "--n", "4", "--peak-gbps", "1792", "--iters", "5", "--seed", "1")
    assert r.returncode == 1, r.stderr
    assert "needs a GPU" in r.stderr
    r = _bench("--peak-gbps", "0")
    assert r.returncode == 2 and "positive" in r.stderr


def test_bench_accepts_the_extras_command_lines():
    # The profiler runs' flags (--only train and its options among them) parse;
    # without a GPU bench.py stops at the device check.
    for extra in (["--only", "train", "--layers", "2", "--eager"], ["--only", "premap_bwd"], ["--only", "block"],
                  ["--only", "placement", "--pads", "0,4096"]):
        r = _bench("--T", "4096", "--C", "1024", "--steps", "1", *extra)
        assert r.returncode == 1, (extra, r.stderr)
        assert "needs a GPU" in r.stderr
