"""Writes tests/golden/config1_oracle.npz: the CPU oracle's outputs for the
plumbing configuration (n=4, D=256, T=128, fp16, gamma off), plus a SHA-256 of
the generated x, as a regression fixture.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "tests")]

from inputs import WORKLOADS, make_case  # noqa: E402
from oracle import oracle  # noqa: E402


def main() -> None:
    case = WORKLOADS[1]
    x, phi, alpha, bias, gamma = make_case(case)
    out = oracle.mhc_pre(x, case.is_bf16, phi, alpha, bias, gamma)
    np.savez_compressed(
        Path(__file__).resolve().parent / "config1_oracle.npz",
        x_sha256=np.array(hashlib.sha256(x.tobytes()).hexdigest()),
        h_in=out["h_in"], h_post=out["h_post"], h_res=out["h_res"], h_pre=out["h_pre"])


if __name__ == "__main__":
    main()
