"""Deterministic synthetic inputs for the MhcPre configurations.

A counter-based generator (splitmix64 of (seed, tensor id, index) -> two
uniforms -> Box-Muller in float64 -> float32), so any subset of rows can be
regenerated and CPU and GPU see identical inputs.  Seeds are
20261201 + configuration number; tensor ids: x=1, phi=2, bias=3, gamma=4,
outlier mask=5.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = np.asarray(z, dtype=np.uint64) + _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def _keys(seed: int, tid: int, count: int, start: int = 0) -> np.ndarray:
    base = splitmix64(np.uint64(seed) ^ splitmix64(np.uint64(tid)))
    with np.errstate(over="ignore"):
        idx = np.arange(start, start + count, dtype=np.uint64)
        return base + idx * np.uint64(2)


def uniform01(seed: int, tid: int, count: int, start: int = 0) -> np.ndarray:
    """float64 uniforms in (0, 1)."""
    u = splitmix64(_keys(seed, tid, count, start))
    return ((u >> np.uint64(11)).astype(np.float64) + 0.5) * (2.0 ** -53)


def normal(seed: int, tid: int, count: int, start: int = 0) -> np.ndarray:
    """float32 N(0, 1) via Box-Muller on two independent uniform streams."""
    k = _keys(seed, tid, count, start)
    with np.errstate(over="ignore"):
        u1 = ((splitmix64(k) >> np.uint64(11)).astype(np.float64) + 0.5) * (2.0 ** -53)
        u2 = ((splitmix64(k + np.uint64(1)) >> np.uint64(11)).astype(np.float64)) * (2.0 ** -53)
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return z.astype(np.float32)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-half-even fp32 -> bf16 bit patterns (finite inputs)."""
    b = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    with np.errstate(over="ignore"):
        r = (b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def f32_to_f16_bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)


def bits_to_f32(bits: np.ndarray, is_bf16: bool) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    if is_bf16:
        return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)
    return bits.view(np.float16).astype(np.float32)


def to_bits(a: np.ndarray, is_bf16: bool) -> np.ndarray:
    return f32_to_bf16_bits(a) if is_bf16 else f32_to_f16_bits(a)


@dataclass(frozen=True)
class Case:
    n: int
    D: int
    T: int
    is_bf16: bool
    gamma: bool
    seed: int
    outliers: bool = False
    alpha: tuple = (0.01, 0.01, 0.01)
    norm_eps: float = 1e-6
    hc_eps: float = 1e-6

    @property
    def K(self) -> int:
        return self.n * self.D

    @property
    def M(self) -> int:
        return self.n * self.n + 2 * self.n


# The five workloads: plumbing, mid-size, headline prefill, decode, ragged tail.
WORKLOADS = {
    1: Case(n=4, D=256, T=128, is_bf16=False, gamma=False, seed=20261201 + 1),
    2: Case(n=4, D=4096, T=1024, is_bf16=True, gamma=True, seed=20261201 + 2),
    3: Case(n=4, D=7168, T=8192, is_bf16=True, gamma=True, seed=20261201 + 3),
    4: Case(n=8, D=7168, T=64, is_bf16=False, gamma=False, seed=20261201 + 4),
    5: Case(n=8, D=8192, T=5472, is_bf16=True, gamma=True, seed=20261201 + 5, outliers=True),
}


# The reference's legal extremes (audit_group_vec.py:37,41-45,123-146: any
# D % 16 == 0 up to 16384 for every n, up to B * S = 4 * 32768 rows) at the
# shapes that stress the library's paths: n = 4 widths whose strip teams span
# the XCDs (32 and 64 slices), the widest n = 4 and n = 6 rows, and the
# headline width over 131072 rows (x passed as [4, 32768, n, D]).
EXTREMES = {
    "n4_D8192_T8192": Case(n=4, D=8192, T=8192, is_bf16=True, gamma=True, seed=20261301),
    "n4_D16384_T4096": Case(n=4, D=16384, T=4096, is_bf16=True, gamma=True, seed=20261302),
    "n6_D16384_T4096": Case(n=6, D=16384, T=4096, is_bf16=False, gamma=True, seed=20261303),
    "n4_D7168_B4_S32768": Case(n=4, D=7168, T=131072, is_bf16=True, gamma=True, seed=20261304),
    # a width with a partial last strip slice (27 slices of 256 columns and one of 192)
    "n4_D7104_T8192": Case(n=4, D=7104, T=8192, is_bf16=True, gamma=True, seed=20261305),
}
EXTREME_LEAD = {"n4_D7168_B4_S32768": (4, 32768)}


def outlier_rows(case: Case) -> np.ndarray:
    """Rows scaled x50: splitmix64(seed, 5, r) % 100 == 0, plus the last row."""
    if not case.outliers:
        return np.zeros(0, dtype=np.int64)
    h = splitmix64(_keys(case.seed, 5, case.T))
    rows = np.nonzero((h % np.uint64(100)) == 0)[0]
    return np.union1d(rows, [case.T - 1]).astype(np.int64)


def make_weights(case: Case):
    """phi (memory [M][K]), alpha [3], bias [M], gamma [K] or None."""
    K, M = case.K, case.M
    phi = (normal(case.seed, 2, M * K) * np.float32(1.0 / np.sqrt(K))).reshape(M, K)
    bias = (uniform01(case.seed, 3, M) * 0.2 - 0.1).astype(np.float32)
    alpha = np.asarray(case.alpha, dtype=np.float32)
    gamma = None
    if case.gamma:
        gamma = (1.0 + 0.1 * normal(case.seed, 4, K).astype(np.float64)).astype(np.float32)
    return phi.astype(np.float32), alpha, bias, gamma


def make_x_rows(case: Case, row_start: int, row_count: int) -> np.ndarray:
    """16-bit x patterns for rows [row_start, row_start + row_count), shape [R, n, D]."""
    K = case.K
    x = normal(case.seed, 1, row_count * K, start=row_start * K).reshape(row_count, K)
    if case.outliers:
        rows = outlier_rows(case)
        sel = rows[(rows >= row_start) & (rows < row_start + row_count)] - row_start
        x[sel] *= np.float32(50.0)
    return to_bits(x, case.is_bf16).reshape(row_count, case.n, case.D)


def make_case(case: Case):
    phi, alpha, bias, gamma = make_weights(case)
    x = make_x_rows(case, 0, case.T)
    return x, phi, alpha, bias, gamma


def audit_formula_case(n: int, d: int, has_gamma: bool, is_bf16: bool, rows: int, seed: int):
    """Inputs of the reference's offline formula audit (audit_group_vec.py:259-276):
    a Park-Miller LCG (x48271 mod 2^31-1) drawn in the order x, phi, gamma,
    alpha, bias.  Returns x bits [rows, n, d], phi [M, K], alpha, bias, gamma|None."""
    state = seed
    flat, mix = n * d, n * n + 2 * n

    def draws(count: int) -> np.ndarray:
        nonlocal state
        out = np.empty(count, dtype=np.float64)
        s = state
        for i in range(count):
            s = (s * 48271) % 2147483647
            out[i] = (s % 2000000) / 1000000.0 - 1.0
        state = s
        return out

    x = (draws(rows * flat) * 0.5).astype(np.float32).reshape(rows, n, d)
    phi = (draws(mix * flat) * 0.1).astype(np.float32).reshape(mix, flat)
    gamma = (1.0 + draws(flat) * 0.1).astype(np.float32) if has_gamma else None
    alpha = (draws(3) * 0.2).astype(np.float32)
    bias = (draws(mix) * 0.2).astype(np.float32)
    return to_bits(x, is_bf16), phi, alpha, bias, gamma


def audit_formula_cases():
    """The 13 (n, d, gamma, dtype, rows, seed) cases of audit_group_vec.py:336-344."""
    cases = []
    seed = 20260905
    for n in (4, 6, 8):
        for is_bf16 in (False, True):
            cases.append((n, 16, True, is_bf16, 36, seed))
            seed += 1
            cases.append((n, 32, False, is_bf16, 36, seed))
            seed += 1
    cases.append((8, 1024, True, False, 8, seed))
    return cases


# The reference device harness's E3 matrix (cloud_runner/runner.cpp:320-327):
# (B, S, n, D, gamma, bf16); inputs from glibc rand() after srand(42).
E3_CASES = [
    (1, 2048, 4, 2560, True, False),
    (1, 2048, 6, 1024, True, False),
    (1, 1024, 8, 1024, True, False),
    (1, 2048, 4, 2560, False, False),
    (1, 2048, 6, 1024, True, True),
    (1, 1024, 8, 1024, False, True),
]
E3_ALPHA = (0.5, 0.3, 0.2)  # cloud_runner/runner.cpp:369
