"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

Tolerances (tests/helpers.py): hPre/hPost/hRes rtol 1e-4, atol 1e-5; hIn
within 1 ulp of the output dtype.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from helpers import assert_close_f32, assert_hin, ulp_distance
from inputs import (WORKLOADS, E3_ALPHA, E3_CASES, audit_formula_case, audit_formula_cases,
                    make_case, to_bits)

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def to_device(pkg, device, x_bits, is_bf16, phi, alpha, bias, gamma, lead=None):
    import torch

    dt = torch.bfloat16 if is_bf16 else torch.float16
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    if lead is not None:
        x_bits = x_bits.reshape(tuple(lead) + x_bits.shape[-2:])
    xt = torch.from_numpy(x_bits.view(np.int16)).to(device).view(dt)
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)
    return xt, f(phi), f(alpha), f(bias), (f(gamma) if gamma is not None else None)


def run_gpu(pkg, device, x_bits, is_bf16, phi, alpha, bias, gamma, norm_eps=1e-6, hc_eps=1e-6,
            lead=None, h_pre=True, force_path=None, launch=None):
    import os

    import torch

    xt, pt, at, bt, gt = to_device(pkg, device, x_bits, is_bf16, phi, alpha, bias, gamma, lead)
    if force_path is not None:
        os.environ["MHCPRE_FORCE_PATH"] = force_path
    if launch is not None:
        os.environ["MHCPRE_LAUNCH"] = launch
    try:
        op = pkg.MhcPreOp(xt, pt, at, bt, gt, norm_eps, hc_eps, h_pre=True if h_pre else None)
    finally:
        os.environ.pop("MHCPRE_FORCE_PATH", None)
        os.environ.pop("MHCPRE_LAUNCH", None)
    _say(f"  path={op.path}")
    op.launch()
    torch.cuda.synchronize()
    assert op.device_status() == 0
    out = fetch(op)
    out["path"] = op.path
    op.close()
    return out


def fetch(op):
    import torch

    T = op.h_in.shape[:-1].numel()
    n = op.h_post.shape[-1]
    out = {
        "h_in": op.h_in.view(torch.int16).cpu().numpy().view(np.uint16).reshape(T, -1),
        "h_post": op.h_post.cpu().numpy().reshape(T, n),
        "h_res": op.h_res.cpu().numpy().reshape(T, n, n),
    }
    if op.h_pre is not None:
        out["h_pre"] = op.h_pre.cpu().numpy().reshape(T, n)
    return out


def check(out, ref, x_bits, is_bf16, orc):
    assert_close_f32("hPost", out["h_post"], ref["h_post"])
    assert_close_f32("hRes", out["h_res"], ref["h_res"])
    if "h_pre" in out:
        assert_close_f32("hPre", out["h_pre"], ref["h_pre"])
    assert_hin(out["h_in"], ref["h_in"], x_bits, is_bf16, out.get("h_pre"), ref["h_pre"], orc,
               ref=ref)


@pytest.mark.parametrize("cfg,force", [(1, None), (2, None), (4, None), (1, "split"),
                                       (2, "split"), (1, "fused"), (2, "fused"), (1, "rows"),
                                       (2, "rows"), (1, "strip")])
def test_config_full_parity(pkg, orc, device, cfg, force):
    case = WORKLOADS[cfg]
    _say(f"[parity] config {cfg} force={force}: {case}")
    x, phi, alpha, bias, gamma = make_case(case)
    out = run_gpu(pkg, device, x, case.is_bf16, phi, alpha, bias, gamma, force_path=force)
    ref = orc.mhc_pre(x, case.is_bf16, phi, alpha, bias, gamma)
    check(out, ref, x, case.is_bf16, orc)


@pytest.mark.parametrize("force", ["fused", "strip"])
def test_cooperative_launch_matches(pkg, orc, device, force):
    """The cooperative launch mode (MHCPRE_LAUNCH=cooperative) runs the same
    kernel: bit-identical outputs to the default launch, and parity."""
    case = WORKLOADS[2]
    _say(f"[parity] config 2 cooperative launch ({force}): {case}")
    x, phi, alpha, bias, gamma = make_case(case)
    coop = run_gpu(pkg, device, x, case.is_bf16, phi, alpha, bias, gamma, launch="cooperative",
                   force_path=force)
    plain = run_gpu(pkg, device, x, case.is_bf16, phi, alpha, bias, gamma, force_path=force)
    assert coop["path"] == plain["path"] == force
    for k in ("h_in", "h_post", "h_res", "h_pre"):
        assert np.array_equal(coop[k], plain[k]), k
    ref = orc.mhc_pre(x, case.is_bf16, phi, alpha, bias, gamma)
    check(coop, ref, x, case.is_bf16, orc)


@pytest.mark.parametrize("B,S,n,D,has_gamma,is_bf16", E3_CASES)
def test_reference_e3_matrix(pkg, orc, device, B, S, n, D, has_gamma, is_bf16):
    """The reference harness's shape matrix and inputs (cloud_runner/runner.cpp:320-382)."""
    _say(f"[e3] B={B} S={S} n={n} D={D} gamma={has_gamma} bf16={is_bf16}")
    T = B * S
    xf, phi, bias, gamma = orc.reference_harness_inputs(42, T, n, D)
    x = orc.f32_to_bits(xf, is_bf16)
    alpha = np.asarray(E3_ALPHA, dtype=np.float32)
    g = gamma if has_gamma else None
    out = run_gpu(pkg, device, x, is_bf16, phi, alpha, bias, g, lead=(B, S))
    ref = orc.mhc_pre(x, is_bf16, phi, alpha, bias, g)
    check(out, ref, x, is_bf16, orc)
    # The harness's own acceptance rule (cloud_runner/runner.cpp:279-301):
    # |a-b| / max(1,|a|,|b|) <= 5e-2 for all but 0.1 % of elements.
    got = orc.bits_to_f32(out["h_in"], is_bf16)
    want = orc.bits_to_f32(ref["h_in"], is_bf16)
    rel = np.abs(got - want) / np.maximum(1.0, np.maximum(np.abs(got), np.abs(want)))
    assert np.count_nonzero(rel > 5e-2) <= got.size // 1000


def test_probe_e1_e2_relaunch(pkg, orc, device):
    """E1: first launch completes and matches; E2: a second launch of the same
    executor matches again, bit for bit (cloud_runner/probe_e1e2.cpp:223-326)."""
    import torch

    B, S, n, D = 1, 64, 4, 256
    xf, phi, bias, gamma = orc.reference_harness_inputs(7, B * S, n, D)
    x = orc.f32_to_f16_bits(xf)
    alpha = np.asarray((0.5, 0.3, 0.2), dtype=np.float32)
    xt, pt, at, bt, gt = to_device(pkg, device, x, False, phi, alpha, bias, gamma, lead=(B, S))
    op = pkg.MhcPreOp(xt, pt, at, bt, gt)
    ref = orc.mhc_pre(x, False, phi, alpha, bias, gamma)
    op.launch()
    torch.cuda.synchronize()
    first = fetch(op)
    check(first, ref, x, False, orc)
    for t in (op.h_in, op.h_post, op.h_res):
        t.zero_()
    op.launch()
    torch.cuda.synchronize()
    second = fetch(op)
    check(second, ref, x, False, orc)
    for k in first:
        assert np.array_equal(first[k], second[k]), k
    op.close()


@pytest.mark.parametrize("case", audit_formula_cases())
def test_audit_formula_cases(pkg, orc, device, case):
    """The offline audit's 13 formula cases (audit_group_vec.py:259-344) on the GPU."""
    n, d, has_gamma, is_bf16, rows, seed = case
    x, phi, alpha, bias, gamma = audit_formula_case(n, d, has_gamma, is_bf16, rows, seed)
    out = run_gpu(pkg, device, x, is_bf16, phi, alpha, bias, gamma)
    ref = orc.mhc_pre(x, is_bf16, phi, alpha, bias, gamma)
    check(out, ref, x, is_bf16, orc)
    # The audit's own range checks (audit_group_vec.py:326-333).
    hin = orc.bits_to_f32(out["h_in"], is_bf16)
    assert (np.abs(hin) < 5.0).all()
    assert ((out["h_pre"] > 0.0) & (out["h_pre"] < 1.1)).all()
    assert (out["h_post"] > 0.0).all()


@pytest.mark.parametrize("T,n,D,is_bf16,has_gamma", [
    (1, 4, 16, True, True),
    (17, 6, 48, False, True),
    (33, 8, 64, True, False),
    (100, 6, 1024, True, True),
    (257, 4, 512, False, True),
    (333, 4, 7168, True, True),
    (49, 4, 1792, False, False),
    (1000, 4, 64, True, True),
    (64, 4, 7168, True, True),     # decode batch at the headline width: the rows path
    (16, 4, 7936, False, True),
    (160, 4, 5120, True, False),   # n = 4, T = 160: the rows path's block GEMM
    (300, 8, 1024, True, True),    # below the split window: the rows path
])
def test_ragged_rows_and_small_widths(pkg, orc, device, T, n, D, is_bf16, has_gamma):
    rng = np.random.default_rng(T * 131 + n * 7 + D)
    K, M = n * D, n * n + 2 * n
    x = to_bits(rng.standard_normal((T, n, D)).astype(np.float32), is_bf16)
    phi = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    alpha = np.asarray([0.3, -0.2, 0.05], dtype=np.float32)
    bias = rng.uniform(-0.5, 0.5, M).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if has_gamma else None
    out = run_gpu(pkg, device, x, is_bf16, phi, alpha, bias, gamma)
    ref = orc.mhc_pre(x, is_bf16, phi, alpha, bias, gamma)
    check(out, ref, x, is_bf16, orc)


@pytest.mark.parametrize("T,D,is_bf16,has_gamma", [
    (6144 + 5, 1536, True, True),    # P = 6: 4 teams per XCD, 2 reducers each; 12+ steps per team
    (4096, 3584, False, True),       # P = 14: 2 teams per XCD, 2 reducers each
    (3072 - 3, 7936, True, False),   # P = 31: teams across XCDs (7 teams, 4 reducers)
    (40, 7168, True, True),          # 3 row tiles for 8 teams: most teams have no tile
    (2048 + 7, 8192, False, True),   # P = 32: teams across XCDs, ragged last tile
    (1024, 12288, True, True),       # P = 48: 4 teams
    (64 * 16 * 3 + 16, 16384, False, False),  # P = 64: 3 teams; one team gets an extra tile
    (2000 + 3, 2304, True, True),    # P = 9: 19 teams across XCDs, 4 reducers each
    (1500, 5120, False, True),       # P = 20: 10 teams across XCDs
    (2500, 2560, True, False),       # P = 10: 2 teams per XCD, 4 reducers each
    (3000 + 1, 5632, True, True),    # P = 22: one team per XCD
    (4096 + 3, 256, True, True),     # P = 1: 80 single-slice teams of 2 reducers (the default from T = 1025)
    (5000 + 1, 256, False, False),
    (777, 3840, True, True),         # P = 15: 13 teams across XCDs
    (1234, 4352, False, False),      # P = 17: 12 teams across XCDs, reducers sized for 32 slices
    (2222, 4864, True, False),       # P = 19: 11 teams across XCDs
    # D % 256 != 0: the last slice has 1-3 strips of columns, the others
    # load zeros and store nothing
    (300, 448, True, True),          # P = 2, the last slice three strips
    (1000 + 3, 192, False, True),    # one slice, three live strips
    (2048, 320, True, False),        # P = 2, the last slice one strip
    (777, 1216, False, False),       # P = 5, the last slice three strips
    (1500, 4160, True, True),        # P = 17 across XCDs, the last slice one strip
    (3000 + 1, 7104, True, True),    # P = 28 in an XCD, the last slice three strips
    (600, 8000, False, True),        # P = 32 across XCDs, the last slice one strip
    # D % 64 == 32: the last live strip has 32 columns, its other lanes load
    # and store nothing
    (500, 224, True, True),          # one slice of 3.5 strips
    (1111, 480, False, True),        # P = 2
    (2000, 2272, True, False),       # P = 9 across XCDs
    (3000 + 1, 7072, True, True),    # P = 28, the last slice 2.5 strips
])
def test_strip_team_shapes(pkg, orc, device, T, D, is_bf16, has_gamma):
    """Team geometries of the strip kernel on a device of 8 XCDs x 32 CUs:
    teams inside an XCD and across XCDs, two and four reducers (the exchange
    ring's size argument covers R = 1, 2, 4), reducer instances sized for 8,
    16, 32 and 64 slices, the largest slice count, enough tiles per team to
    wrap the ring of 10 slots several times, and teams without tiles."""
    n = 4
    rng = np.random.default_rng(T * 7 + D)
    K, M = n * D, n * n + 2 * n
    x = to_bits(rng.standard_normal((T, n, D)).astype(np.float32), is_bf16)
    phi = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    alpha = np.asarray([0.3, -0.2, 0.05], dtype=np.float32)
    bias = rng.uniform(-0.5, 0.5, M).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if has_gamma else None
    _say(f"[strip-teams] T={T} D={D} bf16={is_bf16} gamma={has_gamma}")
    out = run_gpu(pkg, device, x, is_bf16, phi, alpha, bias, gamma, force_path="strip")
    assert out["path"] == "strip"
    ref = orc.mhc_pre(x, is_bf16, phi, alpha, bias, gamma)
    check(out, ref, x, is_bf16, orc)


@pytest.mark.parametrize("T,D,is_bf16,has_gamma", [
    (2048, 7936, True, True),        # 31 slices: 7 teams of 4 reducers across the device
    (4096 - 5, 8192, False, False),  # 32 slices, ragged last tile
    (3072, 9216, True, False),       # 36 slices
    (1500, 10240, False, True),      # 40 slices: 5 teams
    (700, 16384, True, True),        # 64 slices, the widest team: 3 teams
])
def test_wide_widths_take_strip_teams_across_xcds(pkg, orc, device, T, D, is_bf16, has_gamma):
    """n = 4 widths of 31 or more 256-column slices: the strip kernel with
    teams that span XCDs (their exchange words written through to memory at
    device scope) instead of the rows path."""
    n = 4
    rng = np.random.default_rng(T * 11 + D)
    K, M = n * D, n * n + 2 * n
    x = to_bits(rng.standard_normal((T, n, D)).astype(np.float32), is_bf16)
    phi = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    alpha = np.asarray([0.3, -0.2, 0.05], dtype=np.float32)
    bias = rng.uniform(-0.5, 0.5, M).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if has_gamma else None
    _say(f"[wide-strip] T={T} D={D} bf16={is_bf16} gamma={has_gamma}")
    out = run_gpu(pkg, device, x, is_bf16, phi, alpha, bias, gamma)
    assert out["path"] == "strip"
    ref = orc.mhc_pre(x, is_bf16, phi, alpha, bias, gamma)
    check(out, ref, x, is_bf16, orc)


@pytest.mark.parametrize("T,D,is_bf16,has_gamma", [
    (1024, 4096, True, True),           # 12 teams across XCDs: 5 or 6 tiles per team
    (1024 - 7, 7168, False, False),     # 8 teams: 8 tiles per team, ragged last tile
    (16 * 24 * 7 + 5, 2048, True, True),  # 24 teams of 7 or 8 tiles (own tiles 4 and 3)
    (16 * 8 * 5, 7168, False, True),    # 5 tiles per team: own tiles 3 and 2
    (16 * 8 * 9, 7168, True, False),    # 9 tiles per team: own tiles 5 and 4, one whole ring round
    (16 * 8 + 16, 1024, True, True),    # 40 teams: 9 row tiles, most teams without a tile
])
def test_strip_few_tiles_per_team(pkg, orc, device, T, D, is_bf16, has_gamma):
    """Batches that never wrap the x ring (at most 5 own tiles per wave
    group): the prologue's two tiles, the steps' loads past the last tile
    (size-0 resources), the drain steps, and one whole ring round."""
    n = 4
    rng = np.random.default_rng(T * 13 + D)
    K, M = n * D, n * n + 2 * n
    x = to_bits(rng.standard_normal((T, n, D)).astype(np.float32), is_bf16)
    phi = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    alpha = np.asarray([0.3, -0.2, 0.05], dtype=np.float32)
    bias = rng.uniform(-0.5, 0.5, M).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if has_gamma else None
    _say(f"[strip-few] T={T} D={D} bf16={is_bf16} gamma={has_gamma}")
    out = run_gpu(pkg, device, x, is_bf16, phi, alpha, bias, gamma, force_path="strip")
    assert out["path"] == "strip"
    ref = orc.mhc_pre(x, is_bf16, phi, alpha, bias, gamma)
    check(out, ref, x, is_bf16, orc)


def test_attributes_and_hpre_off(pkg, orc, device):
    """Non-default normEps/hcEps (hcEps = 0 skips the add, mhc_pre.cpp:552) and the
    3-output entry point (no hPre)."""
    case = WORKLOADS[1]
    x, phi, alpha, bias, _ = make_case(case)
    for norm_eps, hc_eps in ((1e-3, 0.0), (0.5, 0.25)):
        out = run_gpu(pkg, device, x, case.is_bf16, phi, alpha, bias, None, norm_eps, hc_eps,
                      h_pre=False)
        ref = orc.mhc_pre(x, case.is_bf16, phi, alpha, bias, None, norm_eps, hc_eps)
        check(out, ref, x, case.is_bf16, orc)


def test_zero_and_constant_rows(pkg, orc, device):
    """x = 0 rows: invRms = 1/sqrt(eps), mix = 0, hIn = 0; constant rows."""
    T, n, D = 32, 4, 256
    K, M = n * D, n * n + 2 * n
    rng = np.random.default_rng(5)
    xf = np.zeros((T, n, D), dtype=np.float32)
    xf[16:] = 0.75
    x = to_bits(xf, True)
    phi = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    alpha = np.full(3, 0.01, dtype=np.float32)
    bias = rng.uniform(-0.1, 0.1, M).astype(np.float32)
    out = run_gpu(pkg, device, x, True, phi, alpha, bias, None)
    ref = orc.mhc_pre(x, True, phi, alpha, bias, None)
    check(out, ref, x, True, orc)
    assert (ulp_distance(out["h_in"][:16], np.zeros_like(out["h_in"][:16])) == 0).all()


@pytest.mark.parametrize("cfg", [2, 4])
def test_determinism(pkg, device, cfg):
    """Two launches give bitwise-identical outputs (fixed-order reductions, no atomics)."""
    import torch

    case = WORKLOADS[cfg]
    x, phi, alpha, bias, gamma = make_case(case)
    xt, pt, at, bt, gt = to_device(pkg, device, x, case.is_bf16, phi, alpha, bias, gamma)
    op = pkg.MhcPreOp(xt, pt, at, bt, gt, h_pre=True)
    op.launch()
    torch.cuda.synchronize()
    a = fetch(op)
    op.launch()
    torch.cuda.synchronize()
    b = fetch(op)
    for k in a:
        assert np.array_equal(a[k], b[k]), k
    op.close()


@pytest.mark.parametrize("force,expect,n,T,D", [(None, "strip", 4, 400, 7168),
                                               ("fused", "fused", 4, 400, 7168),
                                               (None, "rows", 8, 300, 2048),
                                               (None, "rows", 8, 48, 2048)])
def test_shared_workspace_back_to_back(pkg, orc, device, force, expect, n, T, D):
    """Two executors with different inputs launched back to back on ONE
    workspace: nothing from the first launch (exchange records, published
    hPre) may leak into the second."""
    import os

    import torch

    K, M = n * D, n * n + 2 * n
    ops, refs, xs = [], [], []
    ws = None
    for seed in (11, 12):
        rng = np.random.default_rng(seed)
        x = to_bits(rng.standard_normal((T, n, D)).astype(np.float32), True)
        phi = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
        alpha = np.full(3, 0.01, dtype=np.float32)
        bias = rng.uniform(-0.1, 0.1, M).astype(np.float32)
        gamma = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
        xt, pt, at, bt, gt = to_device(pkg, device, x, True, phi, alpha, bias, gamma)
        if force is not None:
            os.environ["MHCPRE_FORCE_PATH"] = force
        try:
            op = pkg.MhcPreOp(xt, pt, at, bt, gt, h_pre=True, workspace=ws)
        finally:
            os.environ.pop("MHCPRE_FORCE_PATH", None)
        ws = op.workspace
        ops.append(op)
        refs.append(orc.mhc_pre(x, True, phi, alpha, bias, gamma))
        xs.append(x)
    assert ops[0].path == expect
    for _ in range(2):
        for op in ops:
            op.launch()
        torch.cuda.synchronize()
        for op, ref, x in zip(ops, refs, xs):
            assert op.device_status() == 0
            check(fetch(op), ref, x, True, orc)
    for op in ops:
        op.close()


@pytest.mark.parametrize("T,n,D,is_bf16,has_gamma", [
    (300, 8, 1024, True, True),     # two 256-row blocks, the second with 44 rows
    (513, 6, 2048, False, True),    # three blocks, the last with one row; fp16 x split
    (1, 8, 128, True, False),       # one row
    (2000, 8, 512, True, True),     # eight blocks, short K-ranges
    (257, 6, 7168, True, False),    # long K (43008): many stages per K-range
    (96, 8, 2048, False, False),    # fp16, one partial block
    (64, 6, 1024, True, True),      # small-batch GEMM (T <= 64): B built from phi in registers
    (40, 8, 4096, True, True),      # small-batch GEMM, rows past T in the last 16-row block
    (2, 6, 2048, False, False),     # small-batch GEMM, fp16, two rows
    (20000, 8, 64, True, True),     # 79 row blocks, K = 512: one stage per K-range
    (64, 8, 16384, True, True),     # small-batch GEMM, K = 131072: 512 K-ranges
    (600, 8, 16384, False, True),   # K = 131072 on the block GEMM, fp16
    (40, 8, 2064, True, False),     # epilogue rows split in 2 parts of 129 / 129 octets
    (80, 6, 4160, False, True),     # n = 6, 3 parts of 174 / 174 / 172 octets
    (24, 8, 3088, True, True),      # 3 parts of 129 / 129 / 128 octets
    (100, 4, 256, False, False),    # n = 4 small-batch GEMM (128 rows per wave), 100 rows
    (128, 4, 7168, True, True),     # n = 4 small-batch GEMM, full 128 rows, K = 28672
    (200, 4, 4096, True, True),     # wide small-batch GEMM (n = 4: 256 rows), 200 rows
    (256, 4, 7168, False, True),    # wide small-batch GEMM, full 256 rows, fp16
    (128, 6, 4096, True, False),    # wide small-batch GEMM (n = 6, 8: 128 rows), full
    (65, 8, 2048, True, True),      # wide small-batch GEMM, one row past the narrow one
])
def test_rows_path_shapes(pkg, orc, device, T, n, D, is_bf16, has_gamma):
    """Row-block path (n = 6, 8): ragged row blocks, several K-ranges, fp16 and
    bf16 x, gamma on and off, against the oracle.  The path is forced: the
    plan takes the split path for some of these shapes."""
    rng = np.random.default_rng(T * 17 + n * 5 + D)
    K, M = n * D, n * n + 2 * n
    xf = rng.standard_normal((T, n, D)).astype(np.float32)
    xf[::7] *= 50.0  # large rows exercise the RMS scale
    x = to_bits(xf, is_bf16)
    phi = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    alpha = np.asarray([0.3, -0.2, 0.05], dtype=np.float32)
    bias = rng.uniform(-0.5, 0.5, M).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if has_gamma else None
    _say(f"[rows] T={T} n={n} D={D} bf16={is_bf16} gamma={has_gamma}")
    out = run_gpu(pkg, device, x, is_bf16, phi, alpha, bias, gamma, force_path="rows")
    assert out["path"] == "rows"
    ref = orc.mhc_pre(x, is_bf16, phi, alpha, bias, gamma)
    check(out, ref, x, is_bf16, orc)


@pytest.mark.parametrize("n,force,want", [(4, None, "split"), (8, None, "split"), (8, "rows", "rows")])
def test_epilogue_launches_in_row_chunks(pkg, orc, device, n, force, want):
    """More than 2^20 rows: the one-workgroup-per-row epilogues run as several
    launches (a grid's work-items must stay below 2^32).  The rows on both
    sides of the launch boundary and the last rows are checked against the
    oracle; rows are independent, so a subset is exact for the rows it
    covers."""
    T, D = (1 << 20) + 100, 16
    rng = np.random.default_rng(4242 + n)
    K, M = n * D, n * n + 2 * n
    x = to_bits(rng.standard_normal((T, n, D)).astype(np.float32), True)
    phi = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    alpha = np.asarray([0.3, -0.2, 0.05], dtype=np.float32)
    bias = rng.uniform(-0.5, 0.5, M).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    _say(f"[chunks] T={T} n={n} D={D} force={force}")
    out = run_gpu(pkg, device, x, True, phi, alpha, bias, gamma, force_path=force)
    assert out["path"] == want
    sel = np.r_[0:4, (1 << 20) - 8:(1 << 20) + 8, T - 8:T]
    ref = orc.mhc_pre(x[sel], True, phi, alpha, bias, gamma)
    sub = {k: v[sel] for k, v in out.items() if k != "path"}
    check(sub, ref, x[sel], True, orc)


@pytest.mark.parametrize("force,n,T,D", [("strip", 4, 2048, 7168), ("fused", 4, 2048, 1024)])
def test_expired_wait_is_reported_and_cleared(pkg, orc, device, force, n, T, D):
    """MHCPRE_SPIN_LIMIT=0 at phase 1: a bounded wait between workgroups gives
    up at its first poll that finds the data missing (a reducer's first poll
    finds no record yet).  The launch still ends; every output element it
    could not finish is NaN and every other one is exactly the clean value;
    mhcPreQueryDeviceStatus reports the timeout and launch(check=True)
    raises.  A normal executor on the same workspace then runs clean and
    correct."""
    import os

    import torch

    K, M = n * D, n * n + 2 * n
    rng = np.random.default_rng(77)
    x = to_bits(rng.standard_normal((T, n, D)).astype(np.float32), True)
    phi = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    alpha = np.full(3, 0.01, dtype=np.float32)
    bias = rng.uniform(-0.1, 0.1, M).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    xt, pt, at, bt, gt = to_device(pkg, device, x, True, phi, alpha, bias, gamma)
    os.environ["MHCPRE_FORCE_PATH"] = force
    os.environ["MHCPRE_SPIN_LIMIT"] = "0"
    try:
        bad = pkg.MhcPreOp(xt, pt, at, bt, gt, h_pre=True)
    finally:
        os.environ.pop("MHCPRE_SPIN_LIMIT", None)
    try:
        good = pkg.MhcPreOp(xt, pt, at, bt, gt, h_pre=True, workspace=bad.workspace)
    finally:
        os.environ.pop("MHCPRE_FORCE_PATH", None)
    assert bad.path == force and good.path == force
    _say(f"[timeout] {force} T={T} D={D}")
    timeout_code = pkg.binding.STATUS_CODE["MHC_STATUS_DEVICE_TIMEOUT"]
    with pytest.raises(pkg.MhcPreError) as ei:
        bad.launch(check=True)
    assert ei.value.status == timeout_code
    torch.cuda.synchronize()
    assert bad.device_status() == timeout_code
    good.launch()
    torch.cuda.synchronize()
    assert good.device_status() == 0
    # The status word still holds the first launch's timeout, under its id.
    assert bad.device_status() == timeout_code
    clean = fetch(good)
    check(clean, orc.mhc_pre(x, True, phi, alpha, bias, gamma), x, True, orc)
    # The timed-out launch: NaN where it gave up, the clean value elsewhere.
    poisoned = fetch(bad)
    hin_bad = poisoned["h_in"]
    hin_nan = (hin_bad & 0x7F80) == 0x7F80
    hin_nan &= (hin_bad & 0x007F) != 0
    assert np.array_equal(hin_bad[~hin_nan], clean["h_in"][~hin_nan])
    counts = {"h_in": int(hin_nan.sum())}
    for k in ("h_post", "h_res", "h_pre"):
        nan = np.isnan(poisoned[k])
        assert np.array_equal(poisoned[k][~nan], clean[k][~nan]), k
        counts[k] = int(nan.sum())
    _say(f"[timeout] NaN elements of the timed-out launch: {counts}")
    # Which outputs a given wait covers depends on the path (a fused-path
    # reducer may find every record at its first poll while the slices'
    # broadcast waits expire), but some hIn row always waited on hPre.
    assert counts["h_in"] > 0
    good.close()
    bad.close()


@pytest.mark.parametrize("force,n,T,D", [("strip", 4, 1000, 7168), ("fused", 4, 600, 1024),
                                         ("rows", 8, 300, 1024)])
def test_graph_replays_get_fresh_exchange_epochs(pkg, orc, device, force, n, T, D):
    """One launch captured into a HIP graph and replayed with new x each time
    (eager copies and synchronizations between the replays).  The strip
    kernel's exchange ring reuses its slots within a launch at this size and
    the fused kernel's records sit at fixed places, so a replay that reused
    the captured launch's epoch would accept the previous replay's words;
    every replay must instead match the oracle for its own x and equal an
    eager launch bit for bit."""
    import os

    import torch

    K, M = n * D, n * n + 2 * n
    rng = np.random.default_rng(4100 + T)
    phi = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    alpha = np.asarray([0.3, -0.2, 0.05], dtype=np.float32)
    bias = rng.uniform(-0.5, 0.5, M).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    xs = [to_bits(rng.standard_normal((T, n, D)).astype(np.float32) * (1 + 3 * i), True)
          for i in range(3)]
    xt, pt, at, bt, gt = to_device(pkg, device, xs[0], True, phi, alpha, bias, gamma)
    os.environ["MHCPRE_FORCE_PATH"] = force
    try:
        op = pkg.MhcPreOp(xt, pt, at, bt, gt, h_pre=True)
    finally:
        os.environ.pop("MHCPRE_FORCE_PATH", None)
    assert op.path == force
    _say(f"[graph] {force} T={T} n={n} D={D}")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        op.launch(side)  # eager launch before capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        op.launch()
    torch.cuda.synchronize()
    for i in (1, 2, 0, 1):
        src = torch.from_numpy(xs[i].view(np.int16)).to(device).view(torch.bfloat16)
        xt.copy_(src)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert op.device_status() == 0
        replayed = fetch(op)
        check(replayed, orc.mhc_pre(xs[i], True, phi, alpha, bias, gamma), xs[i], True, orc)
        op.launch()
        torch.cuda.synchronize()
        eager = fetch(op)
        for k in replayed:
            assert np.array_equal(replayed[k], eager[k]), (i, k)
    del graph
    op.close()
