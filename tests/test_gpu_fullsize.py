"""Full-size configurations (headline prefill and the ragged n=8 case).

Inputs of this size are generated on the GPU (seeded torch generator).  Two
independent checks:
  * sampled rows (first, last -- including the ragged tail tile -- random, and
    every x50 outlier row) against the CPU oracle;
  * every row against a float64 restatement of the formula evaluated with
    torch on the GPU (GEMM in fp64, epilogue in fp64); hIn is checked from the
    kernel's own hPre with an fp64 stream sum.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from helpers import assert_close_f32, assert_hin
from inputs import CONFIGS, make_weights, outlier_rows

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


@pytest.mark.parametrize("cfg", [3, 5])
def test_full_size(pkg, orc, device, cfg):
    import torch

    case = CONFIGS[cfg]
    _say(f"[fullsize] config {cfg}: {case}")
    x, phi, alpha, bias, gamma, pt, at, bt, gt, out_rows = _gpu_inputs(case, device)
    op = pkg.MhcPreOp(x, pt, at, bt, gt, case.norm_eps, case.hc_eps, h_pre=True)
    _say(f"[fullsize] path={op.path} workspace={op.workspace_size}")
    op.launch()
    torch.cuda.synchronize()
    assert op.device_status() == 0
    T, n, D = case.T, case.n, case.D
    h_in = op.h_in.view(torch.int16)
    h_post, h_res, h_pre = op.h_post, op.h_res, op.h_pre

    # 1) Sampled rows against the CPU oracle.
    rng = np.random.default_rng(cfg)
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
               h_pre[rows_t].cpu().numpy(), ref["h_pre"], orc)

    # 2) Every row against an fp64 restatement on the GPU.
    K, M = case.K, case.M
    x64 = x.reshape(T, K).double()
    b64 = pt.double() * (gt.double()[None, :] if gt is not None else 1.0)
    mix = x64 @ b64.t()
    inv = 1.0 / torch.sqrt((x64 * x64).sum(1) / K + case.norm_eps)
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
    # hIn from the kernel's own hPre, summed in fp64: the kernel's fp32 sum of
    # n rounded products differs from it by far less than one output ulp, so
    # after rounding the two agree to 1 ulp except at exact-tie boundaries.
    hin64 = (h_pre.double()[:, :, None] * x64.reshape(T, n, D)).sum(1)
    hin_ref = hin64.float().to(x.dtype).view(torch.int16)

    def ordered(v):  # sign-magnitude 16-bit patterns -> value order
        v = v.int() & 0xFFFF
        mag = v & 0x7FFF
        return torch.where((v & 0x8000) != 0, -mag, mag)

    dist = (ordered(h_in) - ordered(hin_ref)).abs()
    far = int((dist > 1).sum())
    assert far <= h_in.numel() // 100000, f"hIn vs fp64 stream sum: {far} beyond 1 ulp"
    del x64, mix

    # 3) Relaunch: bitwise identical.
    snap = [t.clone() for t in (h_in, h_post, h_res, h_pre)]
    op.launch()
    torch.cuda.synchronize()
    for a_, b_ in zip(snap, (h_in, h_post, h_res, h_pre)):
        assert torch.equal(a_, b_)
    op.close()
