"""The native C-ABI harness (tests/native/mhc_pre_runner.cpp) on the GPU.

It mirrors the reference's own runner: its case matrix and glibc-rand inputs
(cloud_runner/runner.cpp:320-327,368-382), its host wall-clock latency mode
(1 warm-up, 20 x launch + stream synchronize, min / median / avg,
:458-490), and the probe's relaunch of one executor
(cloud_runner/probe_e1e2.cpp:312-326), each output checked against the C
oracle.  The harness is a C++ program over include/mhc_pre.h, so this covers
the ABI as a native caller links it (no Python binding in between).
"""
from __future__ import annotations

import re
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

RUNNER = Path(__file__).resolve().parent / "native" / "mhc_pre_runner"


def _run(args, timeout=240):
    if not RUNNER.exists():
        pytest.fail(f"{RUNNER} not built (make -C tests/native, or __graft_entry__.build())")
    print(f"[native] {RUNNER.name} {' '.join(args)}", flush=True)
    p = subprocess.run([str(RUNNER)] + args, capture_output=True, text=True, timeout=timeout)
    sys.stdout.write(p.stdout)
    sys.stdout.flush()
    return p


def test_reference_matrix_through_native_abi():
    p = _run([])
    assert p.returncode == 0, p.stdout[-3000:] + p.stderr[-2000:]
    assert "All cases passed: 6 cases" in p.stdout
    lat = re.findall(r"latency: min=([\d.]+) us  median=([\d.]+) us  avg=([\d.]+) us", p.stdout)
    assert len(lat) == 6
    for mn, med, avg in lat:
        assert 0 < float(mn) <= float(med)


def test_headline_shape_latency_through_native_abi():
    """The headline shape (n=4, D=7168, 8192 tokens as B=1, S=8192, bf16,
    gamma on) in the harness's latency mode."""
    p = _run(["--shape", "1", "8192", "4", "7168", "1", "1"])
    assert p.returncode == 0, p.stdout[-3000:] + p.stderr[-2000:]
    assert "path=strip" in p.stdout
