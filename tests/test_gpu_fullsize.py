"""Full-size configurations (headline prefill and the ragged n=8 case).

Inputs of this size are generated on the GPU (seeded torch generator).  Three
independent checks:
  * sampled rows (first, last -- including the ragged tail tile -- random, and
    every x50 outlier row) against the CPU oracle;
  * every row's hPre / hPost / hRes against a float64 restatement of the
    formula evaluated with torch on the GPU (GEMM and epilogue in fp64);
  * every row's hIn bit for bit against the reference's stream order evaluated
    with torch on the GPU from the kernel's own hPre.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from helpers import assert_close_f32, assert_hin
from inputs import WORKLOADS, EXTREME_LEAD, EXTREMES, make_weights, outlier_rows

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _gpu_inputs(case, device):
    import torch

    gen = torch.Generator(device=device)
    gen.manual_seed(case.seed)
    x32 = torch.randn((case.T, case.n, case.D), generator=gen, device=device,
                      dtype=torch.float32)
    out_rows = outlier_rows(case)
    if out_rows.size:
        x32[torch.from_numpy(out_rows).to(device)] *= 50.0
    x = x32.to(torch.bfloat16 if case.is_bf16 else torch.float16)
    del x32
    phi, alpha, bias, gamma = make_weights(case)
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)
    return x, phi, alpha, bias, gamma, f(phi), f(alpha), f(bias), (
        f(gamma) if gamma is not None else None), out_rows


@pytest.mark.parametrize("cfg", [3, 5] + sorted(EXTREMES))
def test_full_size(pkg, orc, device, cfg):
    import torch

    case = WORKLOADS[cfg] if cfg in WORKLOADS else EXTREMES[cfg]
    _say(f"[fullsize] {cfg}: {case}")
    x, phi, alpha, bias, gamma, pt, at, bt, gt, out_rows = _gpu_inputs(case, device)
    lead = EXTREME_LEAD.get(cfg)
    if lead is not None:
        # x as [B, S, n, D] (and outputs of the same leading dims), as the
        # reference's 4-D contract.
        x4 = x.view(*lead, case.n, case.D)
        h_in4 = torch.empty(*lead, case.D, dtype=x.dtype, device=device)
        op = pkg.MhcPreOp(x4, pt, at, bt, gt, case.norm_eps, case.hc_eps, h_pre=True,
                          h_in=h_in4)
        op.h_in = h_in4.view(case.T, case.D)
        op.h_post = op.h_post.view(case.T, case.n)
        op.h_res = op.h_res.view(case.T, case.n, case.n)
        op.h_pre = op.h_pre.view(case.T, case.n)
    else:
        op = pkg.MhcPreOp(x, pt, at, bt, gt, case.norm_eps, case.hc_eps, h_pre=True)
    _say(f"[fullsize] path={op.path} workspace={op.workspace_size}")
    op.launch()
    torch.cuda.synchronize()
    assert op.device_status() == 0
    T, n, D = case.T, case.n, case.D
    h_in = op.h_in.view(torch.int16)
    h_post, h_res, h_pre = op.h_post, op.h_res, op.h_pre

    # 1) Sampled rows against the CPU oracle.
    rng = np.random.default_rng(case.seed)
    rows = np.unique(np.concatenate([
        np.arange(0, 32), np.arange(T - 48, T), rng.choice(T, 192, replace=False), out_rows]))
    rows_t = torch.from_numpy(rows).to(device)
    x_rows = x[rows_t].view(torch.int16).cpu().numpy().view(np.uint16)
    ref = orc.mhc_pre(x_rows, case.is_bf16, phi, alpha, bias, gamma, case.norm_eps,
                      case.hc_eps)
    _say(f"[fullsize] oracle rows: {rows.size}")
    assert_close_f32("hPost", h_post[rows_t].cpu().numpy(), ref["h_post"])
    assert_close_f32("hRes", h_res[rows_t].cpu().numpy(), ref["h_res"])
    assert_close_f32("hPre", h_pre[rows_t].cpu().numpy(), ref["h_pre"])
    assert_hin(h_in[rows_t].cpu().numpy().view(np.uint16), ref["h_in"], x_rows, case.is_bf16,
               h_pre[rows_t].cpu().numpy(), ref["h_pre"], orc, ref=ref)

    # 2) Every row against an fp64 restatement on the GPU (in row chunks of
    # at most 16384 rows, to bound its fp64 copy of x).
    K, M = case.K, case.M
    b64 = pt.double() * (gt.double()[None, :] if gt is not None else 1.0)
    mix = torch.empty((T, M), dtype=torch.float64, device=device)
    inv = torch.empty((T,), dtype=torch.float64, device=device)
    for r0 in range(0, T, 16384):
        x64 = x[r0:r0 + 16384].reshape(-1, K).double()
        mix[r0:r0 + 16384] = x64 @ b64.t()
        inv[r0:r0 + 16384] = 1.0 / torch.sqrt((x64 * x64).sum(1) / K + case.norm_eps)
        del x64
    a = at.double()
    bb = bt.double()
    pre64 = torch.sigmoid(mix[:, :n] * (inv * a[0])[:, None] + bb[:n]) + case.hc_eps
    post64 = 2.0 * torch.sigmoid(mix[:, n:2 * n] * (inv * a[1])[:, None] + bb[n:2 * n])
    res64 = mix[:, 2 * n:] * (inv * a[2])[:, None] + bb[2 * n:]
    for name, got, want in (("hPre", h_pre, pre64), ("hPost", h_post, post64),
                            ("hRes", h_res.reshape(T, n * n), res64)):
        err = (got.double().reshape(want.shape) - want).abs()
        tol = 1e-5 + 1e-4 * want.abs()
        bad = int((err > tol).sum())
        assert bad == 0, f"{name}: {bad} values beyond tolerance vs fp64 (max err {err.max():.3e})"
    # hIn on every row, bit for bit, from the kernel's own hPre: products
    # fl(hPre[s] * x[s]) in fp32, summed over s = 0 .. n-1 in that order in
    # fp32, rounded half-even to the output dtype -- the reference's stream
    # order (code/op_kernel/mhc_pre.cpp:787-813, the oracle's
    # weighted_stream_sum).  Each torch elementwise op is one IEEE rounding.
    xs = x.reshape(T, n, D)
    acc = h_pre[:, 0:1].float() * xs[:, 0, :].float()
    for s_ in range(1, n):
        acc = acc + h_pre[:, s_:s_ + 1].float() * xs[:, s_, :].float()
    want_hin = acc.to(x.dtype).view(torch.int16)
    del acc
    # The restatement agrees with the oracle's stream sum on the sampled rows.
    sampled = want_hin[rows_t].cpu().numpy().view(np.uint16)
    assert np.array_equal(sampled, orc.weighted_stream_sum(
        x_rows, case.is_bf16, h_pre[rows_t].cpu().numpy()))
    neq = int((h_in != want_hin).sum())
    _say(f"[fullsize] hIn rows {T}: {neq} elements differ from the stream sum on the device hPre")
    assert neq == 0, f"hIn: {neq} of {h_in.numel()} elements differ from the reference stream order"
    del mix

    # 3) Relaunch: bitwise identical.
    snap = [t.clone() for t in (h_in, h_post, h_res, h_pre)]
    op.launch()
    torch.cuda.synchronize()
    for a_, b_ in zip(snap, (h_in, h_post, h_res, h_pre)):
        assert torch.equal(a_, b_)
    op.close()
