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
# of the run by tests/conftest.py), and its attribution: for each element
# beyond 1 ulp whose check had the oracle's inputs, hIn evaluated in fp64
# from an fp64 hPre (the formula with no rounding but the inputs'), and which
# of the device's and the oracle's hIn lies closer to it; and the largest
# hPre error of each against that fp64 hPre on those rows.
HIN_STATS = {"checks": 0, "elements": 0, "beyond": 0, "max_ulp": 0,
             "attributed": 0, "device_closer": 0, "oracle_closer": 0, "tied": 0,
             "device_pre_err": 0.0, "oracle_pre_err": 0.0,
             "device_hin_l1": 0.0, "oracle_hin_l1": 0.0,
             "pre_count": 0, "device_pre_l1": 0.0, "oracle_pre_l1": 0.0}


def _pre64(x_bits, is_bf16: bool, inputs: dict, n: int) -> np.ndarray:
    """hPre of the rows of x in fp64: mix = (x * gamma) . phi_j, invRms =
    1 / sqrt(sum x^2 / K + normEps), sigmoid(mix * invRms * alphaPre + b) +
    hcEps, with no intermediate rounding."""
    R, _, D = x_bits.shape
    K = n * D
    xf = _decode16(x_bits, is_bf16).reshape(R, K)
    phi = np.asarray(inputs["phi"], np.float64).reshape(-1, K)[:n]
    g = inputs["gamma"]
    xg = xf * np.asarray(g, np.float64)[None, :] if g is not None else xf
    mix = xg @ phi.T
    inv = 1.0 / np.sqrt((xf * xf).sum(1) / K + inputs["norm_eps"])
    a = np.asarray(inputs["alpha"], np.float64)
    b = np.asarray(inputs["bias"], np.float64)[:n]
    return 1.0 / (1.0 + np.exp(-(mix * (inv * a[0])[:, None] + b))) + inputs["hc_eps"]


def _attribute(got_bits, want_bits, x_bits, is_bf16, got_pre, want_pre, far, inputs):
    rows = np.nonzero(far.any(1))[0]
    n = x_bits.shape[1]
    pre64 = _pre64(x_bits[rows], is_bf16, inputs, n)                   # [r, n]
    xf = _decode16(x_bits[rows], is_bf16)                               # [r, n, D]
    h64 = (pre64[:, :, None] * xf).sum(1)                               # [r, D]
    f = far[rows]
    dev = np.abs(_decode16(got_bits[rows], is_bf16) - h64)[f]
    orc = np.abs(_decode16(want_bits[rows], is_bf16) - h64)[f]
    HIN_STATS["attributed"] += int(f.sum())
    HIN_STATS["device_closer"] += int((dev < orc).sum())
    HIN_STATS["oracle_closer"] += int((orc < dev).sum())
    HIN_STATS["tied"] += int((dev == orc).sum())
    # Relative to the fp64 value, so that rows of every scale weigh alike.
    scale = np.maximum(np.abs(h64[f]), 1e-30)
    HIN_STATS["device_hin_l1"] += float((dev / scale).sum())
    HIN_STATS["oracle_hin_l1"] += float((orc / scale).sum())
    op = np.abs(np.asarray(want_pre, np.float64).reshape(-1, n)[rows] - pre64)
    HIN_STATS["oracle_pre_err"] = max(HIN_STATS["oracle_pre_err"], float(op.max()))
    if got_pre is not None:
        dp = np.abs(np.asarray(got_pre, np.float64)[rows] - pre64)
        HIN_STATS["device_pre_err"] = max(HIN_STATS["device_pre_err"], float(dp.max()))
        HIN_STATS["pre_count"] += int(dp.size)
        HIN_STATS["device_pre_l1"] += float(dp.sum())
        HIN_STATS["oracle_pre_l1"] += float(op.sum())


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
               max_rare_fraction: float = 1e-3, ref: dict = None) -> None:
    """hIn check (see the module docstring).  got_pre=None when the device did
    not return hPre: the bound then uses the hPre tolerance instead.  ref, the
    oracle's result dict for these rows, enables the fp64 attribution of the
    elements beyond 1 ulp (HIN_STATS)."""
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
    if far.any() and ref is not None and "inputs" in ref:
        _attribute(got_bits, want_bits, x_bits, is_bf16, got_pre, want_pre, far, ref["inputs"])
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
