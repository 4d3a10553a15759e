"""Comparison helpers: the tolerances every parity test applies.

hPre / hPost / hRes (fp32): |got - want| <= 1e-5 + 1e-4 * |want|.
hIn (fp16 / bf16):
  * the device's weighted stream reduction is bit-exact: hIn equals
    RNE(sum_s fl(hPre[s] * x[s])) evaluated by the oracle, in the reference's
    stream order, on the device's own hPre;
  * against the oracle's hIn, at most 1 unit in the last place of the output
    dtype -- except where the sum cancels so far that the (tolerated) fp32
    difference between the device's and the oracle's hPre moves it further.
    Those elements must still lie within 1 ulp + sum_s |dhPre[s] * x[s]| +
    the fp32 rounding of both n-term sums (2 n 2^-24 sum_s |hPre[s] x[s]|),
    and they must be rare: at most 1 in 10^3, or 8 elements in outputs of a
    few rows (one row with a far-off hPre column moves a handful of its
    cancelling elements, which the fraction alone would fail at T = 1 or 2).
    The GEMM's summation order is
    hardware-defined in the reference (CANN Cube) and cannot be matched, so
    hPre agrees to fp32 rounding, not bit for bit.
"""
from __future__ import annotations

import numpy as np

RTOL = 1e-4
ATOL = 1e-5
HIN_MAX_ULP = 1

# Use of the hPre-propagation allowance over the session (printed at the end
# of the run by tests/conftest.py).
HIN_STATS = {"checks": 0, "elements": 0, "beyond": 0, "max_ulp": 0}


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


def _decode16(bits: np.ndarray, is_bf16: bool) -> np.ndarray:
    bits = np.asarray(bits, dtype=np.uint16)
    if is_bf16:
        return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32).astype(np.float64)
    return bits.view(np.float16).astype(np.float64)


def _ulp16(bits: np.ndarray, is_bf16: bool) -> np.ndarray:
    mag = np.asarray(bits, dtype=np.uint16) & np.uint16(0x7FFF)
    nxt = np.minimum(mag.astype(np.uint32) + 1, 0x7FFF).astype(np.uint16)
    return np.abs(_decode16(nxt, is_bf16) - _decode16(mag, is_bf16))


def assert_hin(got_bits, want_bits, x_bits, is_bf16: bool, got_pre, want_pre, orc,
               max_rare_fraction: float = 1e-3) -> None:
    """hIn check (see the module docstring).  got_pre=None when the device did
    not return hPre: the bound then uses the hPre tolerance instead."""
    got_bits = np.ascontiguousarray(got_bits).view(np.uint16)
    want_bits = np.ascontiguousarray(want_bits, dtype=np.uint16)
    R, D = want_bits.shape
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16).reshape(R, -1, D)
    assert got_bits.shape == want_bits.shape, (got_bits.shape, want_bits.shape)
    if got_pre is not None:
        got_pre = np.asarray(got_pre, dtype=np.float32).reshape(R, -1)
        exact = orc.weighted_stream_sum(x_bits, is_bf16, got_pre)
        neq = got_bits != exact
        if neq.any():
            i = np.unravel_index(np.argmax(neq), neq.shape)
            raise AssertionError(f"hIn stage: {int(neq.sum())}/{neq.size} differ from the "
                                 f"reference stream sum on the device hPre; first at {i}")
        dpre = np.abs(got_pre.astype(np.float64) - np.asarray(want_pre, np.float64).reshape(R, -1))
    else:
        wp = np.abs(np.asarray(want_pre, np.float64).reshape(R, -1))
        dpre = ATOL + RTOL * wp
    d = ulp_distance(got_bits, want_bits)
    far = d > HIN_MAX_ULP
    # How many elements use the hPre-propagation allowance, and how far.
    max_ulp = int(d.max()) if d.size else 0
    print(f"[hin-allowance] {int(far.sum())}/{far.size} elements beyond {HIN_MAX_ULP} ulp "
          f"(max {max_ulp} ulp)", flush=True)
    HIN_STATS["checks"] += 1
    HIN_STATS["elements"] += int(far.size)
    HIN_STATS["beyond"] += int(far.sum())
    HIN_STATS["max_ulp"] = max(HIN_STATS["max_ulp"], max_ulp)
    if far.any():
        xf = np.abs(_decode16(x_bits, is_bf16))                      # [R, n, D]
        n = xf.shape[1]
        wp = np.abs(np.asarray(want_pre, np.float64).reshape(R, -1))
        arith = 2 * n * 2.0 ** -24 * (wp[:, :, None] * xf).sum(1)
        bound = (dpre[:, :, None] * xf).sum(1) * (1 + 1e-6) + arith + _ulp16(want_bits, is_bf16)
        diff = np.abs(_decode16(got_bits, is_bf16) - _decode16(want_bits, is_bf16))
        bad = far & (diff > bound)
        if bad.any():
            i = np.unravel_index(np.argmax(bad), bad.shape)
            raise AssertionError(f"hIn: {int(bad.sum())} elements beyond 1 ulp + hPre "
                                 f"propagation; first at {i}: diff {diff[i]:.3e} "
                                 f"bound {bound[i]:.3e} ({int(d[i])} ulp)")
        frac = far.sum() / far.size
        assert far.sum() <= max(max_rare_fraction * far.size, 8), \
            f"hIn: {int(far.sum())} elements ({frac:.2e}) beyond 1 ulp"
