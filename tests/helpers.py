"""Comparison helpers: the tolerances every parity test applies.

hPre / hPost / hRes (fp32): |got - want| <= 1e-5 + 1e-4 * |want|.
hIn (fp16 / bf16):          at most 1 unit in the last place of the output dtype.
"""
from __future__ import annotations

import numpy as np

RTOL = 1e-4
ATOL = 1e-5
HIN_MAX_ULP = 1


def ordered16(bits: np.ndarray) -> np.ndarray:
    """Sign-magnitude 16-bit float patterns -> integers in value order (+0 == -0)."""
    b = np.asarray(bits).astype(np.int32)
    mag = b & 0x7FFF
    return np.where(b & 0x8000, -mag, mag)


def ulp_distance(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    return np.abs(ordered16(a_bits) - ordered16(b_bits))


def assert_close_f32(name: str, got: np.ndarray, want: np.ndarray, rtol: float = RTOL,
                     atol: float = ATOL) -> None:
    got = np.asarray(got, dtype=np.float32)
    want = np.asarray(want, dtype=np.float32)
    assert got.shape == want.shape, (name, got.shape, want.shape)
    assert np.isfinite(got).all(), f"{name}: non-finite values"
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    tol = atol + rtol * np.abs(want.astype(np.float64))
    bad = err > tol
    if bad.any():
        i = np.unravel_index(np.argmax(err - tol), err.shape)
        raise AssertionError(
            f"{name}: {int(bad.sum())}/{bad.size} out of tolerance; worst at {i}: "
            f"got {got[i]!r} want {want[i]!r} err {err[i]:.3e} tol {tol[i]:.3e}")


def assert_hin_close(got_bits: np.ndarray, want_bits: np.ndarray,
                     max_ulp: int = HIN_MAX_ULP) -> None:
    got_bits = np.asarray(got_bits).view(np.uint16) if np.asarray(got_bits).dtype != np.uint16 \
        else np.asarray(got_bits)
    assert got_bits.shape == want_bits.shape, (got_bits.shape, want_bits.shape)
    d = ulp_distance(got_bits, want_bits)
    if d.max() > max_ulp:
        i = np.unravel_index(np.argmax(d), d.shape)
        raise AssertionError(f"hIn: {int((d > max_ulp).sum())}/{d.size} beyond {max_ulp} ulp; "
                             f"worst {int(d[i])} ulp at {i}")
