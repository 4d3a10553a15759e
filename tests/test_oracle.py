"""Pins the CPU oracle (CPU only).

Each check is chosen so that a plausible mistake fails it: a wrong rounding
mode or subnormal rule (exhaustive conversions against numpy / torch), a
transposed phi or a dropped gamma (one-hot rows), squares taken after gamma
(gamma on vs off), a wrong invRms chain (closed forms), a sigmoid/affine mixup
(mix = 0 rows), hIn on x*gamma instead of raw x (equal streams with gamma),
and drift from the reference harness's own CPU formula
(cloud_runner/runner.cpp:122-192).
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

from inputs import (WORKLOADS, E3_ALPHA, audit_formula_case, audit_formula_cases, make_case,
                    to_bits)

GOLDEN = Path(__file__).resolve().parent / "golden"


def f32(v) -> np.float32:
    return np.float32(v)


# ---------------------------------------------------------------- conversions

def test_reference_kats(orc):
    """The reference's known answers (audit_group_vec.py:225-235)."""
    kats = json.loads((GOLDEN / "audit_kats.json").read_text())
    vals = np.array([v for v, _ in kats["f16_bits"]], dtype=np.float32)
    want = np.array([b for _, b in kats["f16_bits"]], dtype=np.uint16)
    assert np.array_equal(orc.f32_to_f16_bits(vals), want)
    for v, w in kats["bf16_value"]:
        got = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(np.array([v], dtype=np.float32)))[0]
        assert got == np.float32(w)


def test_reference_rint_kats_pin_the_tie_rule(orc):
    """The reference's round-half-even KATs (audit_group_vec.py:233-234:
    rint(2.5) = 2, rint(3.5) = 4, rint(-2.5) = -2), applied to the oracle's
    fp16 / bf16 conversions where one unit is the last place of the format
    (fp16 in [1024, 2048), bf16 in [128, 256)): a tie must go to the even
    neighbour, on both signs."""
    kats = json.loads((GOLDEN / "audit_kats.json").read_text())["rint_half_even"]
    assert len(kats) == 3
    for base, enc, dec in ((1024.0, orc.f32_to_f16_bits, orc.f16_bits_to_f32),
                           (128.0, orc.f32_to_bf16_bits, orc.bf16_bits_to_f32)):
        for v, want in kats:
            off = np.float32(base if v >= 0 else -base)
            got = dec(enc(np.array([off + np.float32(v)], dtype=np.float32)))[0] - off
            assert got == np.float32(want), (base, v, got, want)


def test_f16_exhaustive_against_numpy(orc):
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = orc.f16_bits_to_f32(bits)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # Narrowing: random fp32 over the whole fp16 range (normals, subnormals,
    # overflow, exact halfway points) against numpy's IEEE round-half-even.
    rng = np.random.default_rng(1)
    mags = np.exp2(rng.uniform(-30, 17, 400000)).astype(np.float32)
    sign = np.where(rng.random(400000) < 0.5, -1, 1).astype(np.float32)
    halfway = ((want[~nan][:-1].astype(np.float64) + want[~nan][1:].astype(np.float64)) / 2)
    halfway = halfway[np.isfinite(halfway)].astype(np.float32)
    x = np.concatenate([mags * sign, halfway, np.float32([0.0, -0.0, 65504, 65520, 65519.996])])
    with np.errstate(over="ignore"):
        exp_bits = x.astype(np.float16).view(np.uint16)
    got_bits = orc.f32_to_f16_bits(x)
    assert np.array_equal(got_bits, exp_bits)


def test_bf16_exhaustive_against_torch(orc):
    import torch

    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    want = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    got = orc.bf16_bits_to_f32(bits)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    rng = np.random.default_rng(2)
    raw = rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    x = raw.view(np.float32)
    x = x[np.isfinite(x)]
    # Exact ties: low 16 bits = 0x8000, both parities of the kept bit.
    ties = ((raw[:4096] & np.uint32(0xFFFF0000)) | np.uint32(0x8000)).view(np.float32)
    x = np.concatenate([x, ties[np.isfinite(ties)]])
    exp_bits = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.f32_to_bf16_bits(x), exp_bits)


# ---------------------------------------------------------------- the formula

def _weights(n, D, seed, gamma=True):
    rng = np.random.default_rng(seed)
    K, M = n * D, n * n + 2 * n
    phi = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    bias = rng.uniform(-0.1, 0.1, M).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if gamma else None
    return phi, bias, g


def test_inv_rms_closed_forms(orc):
    n, D = 4, 256  # K = 1024: invFlatDim = 2^-10 exactly
    K = n * D
    phi, bias, g = _weights(n, D, 3)
    alpha = np.full(3, 0.01, dtype=np.float32)
    xf = np.zeros((2, n, D), dtype=np.float32)
    xf[1] = 0.75
    x = to_bits(xf, True)
    eps = 1e-6
    out = orc.mhc_pre(x, True, phi, alpha, bias, g, eps, 1e-6)
    assert out["inv_rms"][0] == f32(1.0) / np.sqrt(f32(eps))
    # Constant row c: every partial sum of c^2 = 0.5625 is exact, sumsq = K c^2.
    c2 = f32(0.5625)
    want = f32(1.0) / np.sqrt(f32(f32(f32(K) * c2) * f32(1.0 / K)) + f32(eps))
    assert out["inv_rms"][1] == want
    # Squares are taken on raw x, before gamma: gamma must not change invRms.
    out_g = orc.mhc_pre(x, True, phi, alpha, bias, None, eps, 1e-6)
    assert np.array_equal(out_g["inv_rms"], out["inv_rms"])


def test_inv_rms_against_float64(orc):
    n, D, T = 6, 512, 24
    rng = np.random.default_rng(4)
    x = to_bits(rng.standard_normal((T, n, D)).astype(np.float32) * 3, False)
    phi, bias, g = _weights(n, D, 5)
    out = orc.mhc_pre(x, False, phi, np.full(3, 0.01, np.float32), bias, g)
    xf = orc.f16_bits_to_f32(x).reshape(T, -1).astype(np.float64)
    want = 1.0 / np.sqrt((xf * xf).sum(1) / (n * D) + 1e-6)
    np.testing.assert_allclose(out["inv_rms"], want, rtol=2e-6)


def test_gemm_one_hot_rows_pin_phi_layout_and_gamma(orc):
    """A one-hot x row e_k returns column k of gamma (.) phi_mem[M][K] exactly."""
    n, D = 4, 64
    K, M = n * D, n * n + 2 * n
    phi, bias, g = _weights(n, D, 6)
    ks = [0, 1, 63, 64, 200, K - 1]
    xf = np.zeros((len(ks), n, D), dtype=np.float32)
    for r, k in enumerate(ks):
        xf.reshape(len(ks), K)[r, k] = 1.0
    x = to_bits(xf, True)
    out = orc.mhc_pre(x, True, phi, np.full(3, 0.01, np.float32), bias, g)
    for r, k in enumerate(ks):
        want = (phi[:, k] * g[k]).astype(np.float32)
        assert np.array_equal(out["mix"][r], want), k


def test_gemm_against_float64(orc):
    n, D, T = 8, 256, 12
    K = n * D
    rng = np.random.default_rng(7)
    x = to_bits(rng.standard_normal((T, n, D)).astype(np.float32), True)
    phi, bias, g = _weights(n, D, 8)
    out = orc.mhc_pre(x, True, phi, np.full(3, 0.01, np.float32), bias, g)
    xf = orc.bf16_bits_to_f32(x).reshape(T, K).astype(np.float64)
    xg = (orc.bf16_bits_to_f32(x).reshape(T, K) * g).astype(np.float64)  # fp32 x*gamma
    want = xg @ phi.astype(np.float64).T
    scale = np.abs(xf) @ np.abs(phi.astype(np.float64).T * g[None, :].T) + 1e-30
    assert (np.abs(out["mix"] - want) / scale).max() < 2e-6


def test_gamma_folds_into_phi(orc):
    """gamma on equals gamma off with phi*gamma (to fp32 rounding level)."""
    n, D, T = 4, 512, 8
    rng = np.random.default_rng(9)
    x = to_bits(rng.standard_normal((T, n, D)).astype(np.float32), True)
    phi, bias, g = _weights(n, D, 10)
    alpha = np.full(3, 0.01, np.float32)
    a = orc.mhc_pre(x, True, phi, alpha, bias, g)
    b = orc.mhc_pre(x, True, (phi * g[None, :]).astype(np.float32), alpha, bias, None)
    np.testing.assert_allclose(a["mix"], b["mix"], rtol=0, atol=2e-6)
    assert np.array_equal(a["inv_rms"], b["inv_rms"])


def test_zero_mix_epilogue(orc):
    """x = 0: hPre = sigmoid(b) + hcEps, hPost = 2 sigmoid(b), hRes = b."""
    n, D = 8, 64
    phi, bias, g = _weights(n, D, 11)
    bias = np.linspace(-3, 3, bias.size).astype(np.float32)
    hc = 1e-3
    x = np.zeros((1, n, D), dtype=np.uint16)
    out = orc.mhc_pre(x, False, phi, np.float32([0.7, 0.8, 0.9]), bias, g, 1e-6, hc)
    sig = lambda v: 1.0 / (1.0 + math.exp(-float(v)))
    for i in range(n):
        assert abs(out["h_pre"][0, i] - (sig(bias[i]) + hc)) < 2e-7
        assert abs(out["h_post"][0, i] - 2 * sig(bias[n + i])) < 4e-7
    assert np.array_equal(out["h_res"][0].reshape(-1), bias[2 * n:])
    assert not out["h_in"].any()


def test_alpha_zero_isolates_bias(orc):
    n, D, T = 6, 64, 5
    rng = np.random.default_rng(12)
    x = to_bits(rng.standard_normal((T, n, D)).astype(np.float32), True)
    phi, bias, g = _weights(n, D, 13)
    out = orc.mhc_pre(x, True, phi, np.zeros(3, np.float32), bias, g)
    assert np.array_equal(out["h_res"].reshape(T, -1), np.broadcast_to(bias[2 * n:], (T, n * n)))
    assert np.array_equal(out["h_post"][0], out["h_post"][T - 1])


def test_hin_uses_raw_x_and_stream_order(orc):
    """Equal streams: hIn = RNE(x * sum_s hPre[s]); gamma (far from 1) must not
    enter hIn (mhc_pre.cpp:761-826 reads raw x)."""
    n, D, T = 4, 128, 6
    rng = np.random.default_rng(14)
    base = rng.standard_normal((T, 1, D)).astype(np.float32)
    xf = np.repeat(base, n, axis=1)
    x = to_bits(xf, True)
    phi, bias, g = _weights(n, D, 15)
    g = (g * 3).astype(np.float32)
    out = orc.mhc_pre(x, True, phi, np.full(3, 0.5, np.float32), bias, g)
    xb = orc.bf16_bits_to_f32(x)[:, 0, :].astype(np.float64)
    want = xb * out["h_pre"].astype(np.float64).sum(1, keepdims=True)
    got = orc.bf16_bits_to_f32(out["h_in"]).astype(np.float64)
    ulp = np.abs(got - want) / np.maximum(np.abs(want), 1e-30)
    assert (ulp <= 2 ** -8).all()


def _runner_cpu_reference(x_bits, is_bf16, phi, alpha, bias, gamma, orc):
    """The reference harness's CPU reference (cloud_runner/runner.cpp:122-192):
    double-precision sumsq, fp32 k-sequential GEMM, then (mix*invRms)*alpha+bias."""
    T, n, D = x_bits.shape
    K, M = n * D, n * n + 2 * n
    xf = orc.bits_to_f32(x_bits, is_bf16).reshape(T, K)
    inv = (1.0 / np.sqrt((xf.astype(np.float64) ** 2).sum(1) / K + 1e-6)).astype(np.float32)
    xg = xf * gamma if gamma is not None else xf
    acc = np.zeros((T, M), dtype=np.float32)
    phi = phi.reshape(M, K)
    for k in range(K):
        acc += xg[:, k:k + 1] * phi[None, :, k]
    mix = acc * inv[:, None]
    a = alpha
    wpre = mix[:, :n] * a[0] + bias[:n]
    pre = (f32(1) / (f32(1) + np.exp(-wpre))) + f32(1e-6)
    wpost = mix[:, n:2 * n] * a[1] + bias[n:2 * n]
    post = f32(2) / (f32(1) + np.exp(-wpost))
    res = mix[:, 2 * n:] * a[2] + bias[2 * n:]
    x3 = xf.reshape(T, n, D)
    h = pre[:, 0:1] * x3[:, 0]
    for s in range(1, n):
        h = h + pre[:, s:s + 1] * x3[:, s]
    return pre, post, res.reshape(T, n, n), orc.f32_to_bits(h, is_bf16)


@pytest.mark.parametrize("n,D,has_gamma,is_bf16", [(4, 2560, True, False), (6, 1024, True, True),
                                                   (8, 1024, False, True)])
def test_matches_reference_harness_cpu_formula(orc, n, D, has_gamma, is_bf16):
    """The oracle agrees with the reference's own CPU reference on the
    reference's own inputs (glibc rand after srand(42), runner.cpp:368-382)."""
    from helpers import assert_close_f32, assert_hin_close

    T = 12
    xf, phi, bias, gamma = orc.reference_harness_inputs(42, T, n, D)
    x = orc.f32_to_bits(xf, is_bf16)
    alpha = np.asarray(E3_ALPHA, np.float32)
    g = gamma if has_gamma else None
    out = orc.mhc_pre(x, is_bf16, phi, alpha, bias, g)
    pre, post, res, hin = _runner_cpu_reference(x, is_bf16, phi, alpha, bias, g, orc)
    assert_close_f32("hPre", out["h_pre"], pre, rtol=1e-5, atol=1e-6)
    assert_close_f32("hPost", out["h_post"], post, rtol=1e-5, atol=1e-6)
    assert_close_f32("hRes", out["h_res"], res, rtol=1e-5, atol=1e-6)
    assert_hin_close(out["h_in"], hin)


def test_reference_harness_generator_is_glibc_rand(orc):
    """First draws after srand(42) follow glibc's rand() (TYPE_3 additive feedback)."""
    import ctypes

    libc = ctypes.CDLL("libc.so.6")
    libc.srand(42)
    raw = [libc.rand() for _ in range(8)]
    xf, _, _, _ = orc.reference_harness_inputs(42, 1, 4, 16)
    want = np.array([(r % 2000) / 10000.0 for r in raw], dtype=np.float64)
    want = (want.astype(np.float32) - np.float32(0.1)).astype(np.float32)
    assert np.array_equal(xf.reshape(-1)[:8], want)


@pytest.mark.parametrize("case", audit_formula_cases())
def test_audit_formula_ranges(orc, case):
    """The audit's formula cases and range checks (audit_group_vec.py:259-344)."""
    n, d, has_gamma, is_bf16, rows, seed = case
    x, phi, alpha, bias, gamma = audit_formula_case(n, d, has_gamma, is_bf16, rows, seed)
    out = orc.mhc_pre(x, is_bf16, phi, alpha, bias, gamma)
    hin = orc.bits_to_f32(out["h_in"], is_bf16)
    assert (np.abs(hin) < 5.0).all()
    assert ((out["h_pre"] > 0.0) & (out["h_pre"] < 1.1)).all()
    assert (out["h_post"] > 0.0).all()


def test_rows_subset_and_threads_are_exact(orc):
    case = WORKLOADS[1]
    x, phi, alpha, bias, gamma = make_case(case)
    full = orc.mhc_pre(x, case.is_bf16, phi, alpha, bias, gamma, nthreads=1)
    rows = [127, 0, 64, 3]
    sub = orc.mhc_pre(x, case.is_bf16, phi, alpha, bias, gamma, rows=rows, nthreads=4)
    for k in ("h_in", "h_post", "h_res", "h_pre", "mix", "inv_rms"):
        assert np.array_equal(full[k][rows], sub[k]), k


def test_golden_fixture_config1(orc):
    """Regression pin: the committed config-1 outputs (tests/golden/make_golden.py)."""
    data = np.load(GOLDEN / "config1_oracle.npz")
    case = WORKLOADS[1]
    x, phi, alpha, bias, gamma = make_case(case)
    import hashlib

    assert hashlib.sha256(x.tobytes()).hexdigest() == str(data["x_sha256"])
    out = orc.mhc_pre(x, case.is_bf16, phi, alpha, bias, gamma)
    for k in ("h_in", "h_post", "h_res", "h_pre"):
        assert np.array_equal(out[k], data[k]), k


def test_weighted_stream_sum_is_the_oracle_hin_stage(orc):
    """oracle.weighted_stream_sum on the oracle's own hPre reproduces its hIn bit
    for bit (the GPU tests use it to check the device's hIn stage exactly)."""
    for cfg in (1, 2):
        case = WORKLOADS[cfg]
        x, phi, alpha, bias, gamma = make_case(case)
        x = x[:64]
        out = orc.mhc_pre(x, case.is_bf16, phi, alpha, bias, gamma)
        again = orc.weighted_stream_sum(x, case.is_bf16, out["h_pre"])
        assert np.array_equal(again, out["h_in"])


@pytest.mark.parametrize("n,D,gamma_on,is_bf16", [(4, 256, True, True), (8, 128, False, False),
                                                  (6, 64, True, False)])
def test_fp64_hpre_restatement_matches_the_oracle(orc, n, D, gamma_on, is_bf16):
    """The fp64 hPre the hIn-allowance attribution uses (tests/helpers.py
    _pre64) agrees with the oracle's fp32 hPre to fp32 rounding, and moves
    with alphaPre, the bias, gamma and hcEps as the formula says (a wrong
    sign, index or eps placement would fail one of these)."""
    from helpers import _pre64

    rng = np.random.default_rng(1000 + n + D)
    T, K, M = 40, n * D, n * n + 2 * n
    x = orc.f32_to_bits(rng.standard_normal((T, n, D)).astype(np.float32), is_bf16)
    phi = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    alpha = np.asarray([0.7, -0.3, 0.2], np.float32)
    bias = rng.uniform(-0.5, 0.5, M).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if gamma_on else None
    ref = orc.mhc_pre(x, is_bf16, phi, alpha, bias, gamma, 1e-6, 3e-3)
    pre64 = _pre64(x, is_bf16, ref["inputs"], n)
    assert np.allclose(pre64, ref["h_pre"], rtol=2e-6, atol=2e-7)
    # alpha = 0 leaves sigmoid(bias) + hcEps exactly.
    inputs = dict(ref["inputs"], alpha=np.asarray([0.0, 1.0, 1.0], np.float32))
    want = 1.0 / (1.0 + np.exp(-bias[:n].astype(np.float64))) + 3e-3
    assert np.allclose(_pre64(x, is_bf16, inputs, n), want[None, :], rtol=0, atol=1e-15)
