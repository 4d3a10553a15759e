"""ctypes binding of the CPU oracle (liboracle_mhcpre.so).

TEST INFRASTRUCTURE ONLY: imported by the test suite, the smoke check and the
benchmark's cpu_baseline leg, always as the checker or as the timed CPU
baseline, never by the product path.  The arithmetic lives in
mhc_pre_oracle.c, which cites the reference lines it restates.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle_mhcpre.so"

_lib: Optional[ctypes.CDLL] = None


def build() -> None:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "-B"], check=True)


def _load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    u16p = ctypes.POINTER(ctypes.c_uint16)
    f32p = ctypes.POINTER(ctypes.c_float)
    i64p = ctypes.POINTER(ctypes.c_int64)
    lib.oracle_f32_to_f16_n.argtypes = [f32p, u16p, ctypes.c_int64]
    lib.oracle_f32_to_bf16_n.argtypes = [f32p, u16p, ctypes.c_int64]
    lib.oracle_f16_to_f32_n.argtypes = [u16p, f32p, ctypes.c_int64]
    lib.oracle_bf16_to_f32_n.argtypes = [u16p, f32p, ctypes.c_int64]
    lib.oracle_mhc_pre.argtypes = [u16p, ctypes.c_int, ctypes.c_int64, ctypes.c_int,
                                   ctypes.c_int64, f32p, f32p, f32p, f32p, ctypes.c_float,
                                   ctypes.c_float, i64p, ctypes.c_int64, u16p, f32p, f32p,
                                   f32p, f32p, f32p, ctypes.c_int]
    lib.oracle_mhc_pre.restype = ctypes.c_int
    lib.oracle_max_threads.restype = ctypes.c_int
    lib.oracle_weighted_stream_sum.argtypes = [u16p, ctypes.c_int, ctypes.c_int64, ctypes.c_int,
                                               ctypes.c_int64, f32p, u16p]
    lib.oracle_weighted_stream_sum.restype = ctypes.c_int
    lib.oracle_reference_harness_inputs.argtypes = [ctypes.c_uint, ctypes.c_int64, ctypes.c_int,
                                                    ctypes.c_int64, f32p, f32p, f32p, f32p]
    _lib = lib
    return lib


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def f32_to_f16_bits(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    _load().oracle_f32_to_f16_n(_ptr(a, ctypes.c_float), _ptr(out, ctypes.c_uint16), a.size)
    return out


def f32_to_bf16_bits(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    _load().oracle_f32_to_bf16_n(_ptr(a, ctypes.c_float), _ptr(out, ctypes.c_uint16), a.size)
    return out


def f16_bits_to_f32(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    _load().oracle_f16_to_f32_n(_ptr(a, ctypes.c_uint16), _ptr(out, ctypes.c_float), a.size)
    return out


def bf16_bits_to_f32(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    _load().oracle_bf16_to_f32_n(_ptr(a, ctypes.c_uint16), _ptr(out, ctypes.c_float), a.size)
    return out


def bits_to_f32(a, is_bf16: bool) -> np.ndarray:
    return bf16_bits_to_f32(a) if is_bf16 else f16_bits_to_f32(a)


def f32_to_bits(a, is_bf16: bool) -> np.ndarray:
    return f32_to_bf16_bits(a) if is_bf16 else f32_to_f16_bits(a)


def max_threads() -> int:
    return int(_load().oracle_max_threads())


def mhc_pre(x_bits: np.ndarray, is_bf16: bool, phi: np.ndarray, alpha, bias, gamma=None,
            norm_eps: float = 1e-6, hc_eps: float = 1e-6,
            rows: Optional[Sequence[int]] = None, nthreads: int = 0) -> dict:
    """Evaluate the operator on `rows` of x ([T, n, D] 16-bit patterns).

    phi is the fp32 memory [M][K] (any shape with K*M elements).  Returns a dict
    of compact per-row outputs: h_in (uint16 [R, D]), h_post [R, n],
    h_res [R, n, n], h_pre [R, n], mix [R, M], inv_rms [R].
    """
    lib = _load()
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    if x_bits.ndim != 3:
        x_bits = x_bits.reshape((-1,) + x_bits.shape[-2:])
    T, n, D = (int(v) for v in x_bits.shape)
    K, M = n * D, n * n + 2 * n
    phi = np.ascontiguousarray(phi, dtype=np.float32).reshape(-1)
    alpha = np.ascontiguousarray(alpha, dtype=np.float32).reshape(-1)
    bias = np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
    if phi.size != K * M or alpha.size != 3 or bias.size != M:
        raise ValueError("bad phi/alpha/bias size")
    g = None
    if gamma is not None:
        g = np.ascontiguousarray(gamma, dtype=np.float32).reshape(-1)
        if g.size != K:
            raise ValueError("bad gamma size")
    if rows is None:
        rows_arr = None
        R = T
    else:
        rows_arr = np.ascontiguousarray(rows, dtype=np.int64).reshape(-1)
        R = rows_arr.size
    out = {
        "h_in": np.empty((R, D), dtype=np.uint16),
        "h_post": np.empty((R, n), dtype=np.float32),
        "h_res": np.empty((R, n, n), dtype=np.float32),
        "h_pre": np.empty((R, n), dtype=np.float32),
        "mix": np.empty((R, M), dtype=np.float32),
        "inv_rms": np.empty((R,), dtype=np.float32),
    }
    st = lib.oracle_mhc_pre(
        _ptr(x_bits, ctypes.c_uint16), int(bool(is_bf16)), T, n, D, _ptr(phi, ctypes.c_float),
        _ptr(alpha, ctypes.c_float), _ptr(bias, ctypes.c_float),
        _ptr(g, ctypes.c_float) if g is not None else None, ctypes.c_float(norm_eps),
        ctypes.c_float(hc_eps),
        _ptr(rows_arr, ctypes.c_int64) if rows_arr is not None else None, R,
        _ptr(out["h_in"], ctypes.c_uint16), _ptr(out["h_post"], ctypes.c_float),
        _ptr(out["h_res"], ctypes.c_float), _ptr(out["h_pre"], ctypes.c_float),
        _ptr(out["mix"], ctypes.c_float), _ptr(out["inv_rms"], ctypes.c_float), int(nthreads))
    if st != 0:
        raise RuntimeError(f"oracle_mhc_pre failed with {st}")
    # The inputs (references, not copies), for checks that evaluate the
    # formula in fp64 beside the oracle.
    out["inputs"] = {"phi": phi, "alpha": alpha, "bias": bias, "gamma": g,
                     "norm_eps": float(norm_eps), "hc_eps": float(hc_eps), "rows": rows_arr}
    return out


def weighted_stream_sum(x_bits: np.ndarray, is_bf16: bool, h_pre: np.ndarray) -> np.ndarray:
    """hIn from given hPre weights in the reference order (oracle_weighted_stream_sum)."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    x_bits = x_bits.reshape((-1,) + x_bits.shape[-2:])
    R, n, D = (int(v) for v in x_bits.shape)
    h_pre = np.ascontiguousarray(h_pre, dtype=np.float32).reshape(R, n)
    out = np.empty((R, D), dtype=np.uint16)
    st = _load().oracle_weighted_stream_sum(_ptr(x_bits, ctypes.c_uint16), int(bool(is_bf16)), R,
                                            n, D, _ptr(h_pre, ctypes.c_float),
                                            _ptr(out, ctypes.c_uint16))
    if st != 0:
        raise RuntimeError(f"oracle_weighted_stream_sum failed with {st}")
    return out


def reference_harness_inputs(seed: int, T: int, n: int, D: int):
    """x (fp32, before the cast), phi [K*M], bias [M], gamma [K] as the reference
    harnesses draw them with glibc rand() (cloud_runner/runner.cpp:370-382,
    cloud_runner/probe_e1e2.cpp:242-254)."""
    K, M = n * D, n * n + 2 * n
    x = np.empty((T, n, D), dtype=np.float32)
    phi = np.empty((K * M,), dtype=np.float32)
    bias = np.empty((M,), dtype=np.float32)
    gamma = np.empty((K,), dtype=np.float32)
    _load().oracle_reference_harness_inputs(seed, T, n, D, _ptr(x, ctypes.c_float),
                                            _ptr(phi, ctypes.c_float),
                                            _ptr(bias, ctypes.c_float),
                                            _ptr(gamma, ctypes.c_float))
    return x, phi, bias, gamma
