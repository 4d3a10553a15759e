"""mhcPreNoAlloc: the launch whose workspace is the library's built-in
per-device scratch array, against mhcPre with a caller workspace.

Same executor, same kernels: outputs must be bit-identical to the workspace
entry point's, on two calls in a row where the second has a smaller input
(the array keeps the first call's contents), and match the oracle.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from helpers import assert_close_f32, assert_hin
from inputs import to_bits

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _case(T, n, D, seed, device):
    """Inputs; x as bf16 bits on the host, or for large T (where the host
    generator is slow) as a device tensor drawn by torch."""
    import torch

    rng = np.random.default_rng(seed)
    K, M = n * D, n * n + 2 * n
    if T * K <= (1 << 26):
        x = to_bits(rng.standard_normal((T, n, D)).astype(np.float32), True)
    else:
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        x = torch.randn((T, n, D), generator=gen, device=device).to(torch.bfloat16)
    phi = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    alpha = np.asarray([0.3, -0.2, 0.05], dtype=np.float32)
    bias = rng.uniform(-0.5, 0.5, M).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    return x, phi, alpha, bias, gamma


def _outputs(op):
    import torch

    return [t.view(torch.int16).clone() if t.dtype != torch.float32 else t.clone()
            for t in op.outputs()]


@pytest.mark.parametrize("shapes,path", [([(2048, 4, 7168), (512, 4, 7168)], "strip"),
                                         # above ~11k rows the strip workspace used to
                                         # exceed the 64 MiB array; its rings do not grow
                                         ([(16384, 4, 7168), (12288, 4, 7168)], "strip"),
                                         ([(600, 8, 2048), (100, 8, 2048)], "rows"),
                                         ([(600, 8, 1024), (520, 8, 1024)], "split")])
def test_no_alloc_matches_workspace_launch(pkg, orc, device, shapes, path):
    import torch

    f = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)
    for i, (T, n, D) in enumerate(shapes):
        _say(f"[no-alloc] call {i}: T={T} n={n} D={D}")
        x, phi, alpha, bias, gamma = _case(T, n, D, 900 + i, device)
        if isinstance(x, np.ndarray):
            xt = torch.from_numpy(x.view(np.int16)).to(device).view(torch.bfloat16)
        else:
            xt = x
        op = pkg.MhcPreOp(xt, f(phi), f(alpha), f(bias), f(gamma), h_pre=True)
        assert op.path == path
        assert op.workspace_size <= 64 << 20
        op.launch()
        torch.cuda.synchronize()
        assert op.device_status() == 0
        want = _outputs(op)
        for t in op.outputs():
            t.fill_(0)
        op.launch_no_alloc()
        torch.cuda.synchronize()
        got = _outputs(op)
        for g, w, name in zip(got, want, ("hIn", "hPost", "hRes", "hPre")):
            assert torch.equal(g, w), name
        h_in, h_post, h_res, h_pre = (t.cpu().numpy() for t in got)
        # The oracle on every row up to 4096 rows, else on the first and last
        # 256 rows and 512 seeded others (rows are independent).
        rows = np.arange(T) if T <= 4096 else np.unique(np.concatenate([
            np.arange(256), np.arange(T - 256, T),
            np.random.default_rng(910 + i).choice(T, 512, replace=False)]))
        R = len(rows)
        if isinstance(x, np.ndarray):
            xr = np.ascontiguousarray(x[rows])
        else:
            xr = xt[torch.from_numpy(rows).to(device)].view(torch.int16).cpu().numpy().view(np.uint16)
        ref = orc.mhc_pre(xr, True, phi, alpha, bias, gamma)
        assert_close_f32("hPost", h_post.reshape(T, n)[rows], ref["h_post"])
        assert_close_f32("hRes", h_res.reshape(T, n, n)[rows], ref["h_res"])
        assert_close_f32("hPre", h_pre.reshape(T, n)[rows], ref["h_pre"])
        assert_hin(h_in.view(np.uint16).reshape(T, D)[rows], ref["h_in"], xr, True,
                   h_pre.reshape(T, n)[rows], ref["h_pre"], orc, ref=ref)
        assert R == len(ref["h_pre"])
        op.close()


def test_no_alloc_status_query_reports_an_expired_wait(pkg, device):
    """mhcPreQueryDeviceStatus(NULL, 0, ...) reads the built-in workspace of
    mhcPreNoAlloc launches: MHCPRE_SPIN_LIMIT=0 (a phase-1 test knob; a wait
    gives up at its first poll that finds the data missing, and the kernel
    ends normally) makes the strip launch report a timeout there, and a
    normal executor's later no-alloc launch reports none."""
    import os

    import torch

    T, n, D = 2048, 4, 7168
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)
    x, phi, alpha, bias, gamma = _case(T, n, D, 930, device)
    xt = torch.from_numpy(x.view(np.int16)).to(device).view(torch.bfloat16)
    args = (xt, f(phi), f(alpha), f(bias), f(gamma))
    os.environ["MHCPRE_SPIN_LIMIT"] = "0"
    try:
        bad = pkg.MhcPreOp(*args, h_pre=True)
    finally:
        os.environ.pop("MHCPRE_SPIN_LIMIT", None)
    good = pkg.MhcPreOp(*args, h_pre=True)
    assert bad.path == "strip" and good.path == "strip"
    timeout = pkg.binding.STATUS_CODE["MHC_STATUS_DEVICE_TIMEOUT"]
    _say("[no-alloc] status query, spin limit 0")
    bad.launch_no_alloc()
    assert bad.no_alloc_device_status() == timeout
    good.launch_no_alloc()
    assert good.no_alloc_device_status() == 0
    assert not torch.isnan(good.h_in.float()).any()
    # The word under the first executor's launch id still reads as its timeout.
    assert bad.no_alloc_device_status() == timeout
    bad.close()
    good.close()


@pytest.mark.parametrize("T,n,D,path", [(1000, 4, 7168, "strip"), (300, 8, 1024, "rows")])
def test_no_alloc_launch_in_a_graph(pkg, orc, device, T, n, D, path):
    """mhcPreNoAlloc captured into a HIP graph (its scratch address is
    resolved when the executor is created, so the capture makes no symbol
    lookup) and replayed with new x, with eager copies and synchronizations
    between the replays: every replay equals an eager no-alloc launch bit
    for bit and matches the oracle."""
    import torch

    f = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)
    xs = [_case(T, n, D, 940 + i, device) for i in range(3)]
    _, phi, alpha, bias, gamma = xs[0]
    xt = torch.from_numpy(xs[0][0].view(np.int16)).to(device).view(torch.bfloat16)
    op = pkg.MhcPreOp(xt, f(phi), f(alpha), f(bias), f(gamma), h_pre=True)
    assert op.path == path
    _say(f"[no-alloc graph] {path} T={T} n={n} D={D}")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        op.launch_no_alloc()
    torch.cuda.synchronize()
    for i in (1, 2, 0, 1):
        xb = xs[i][0]
        xt.copy_(torch.from_numpy(xb.view(np.int16)).to(device).view(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert op.no_alloc_device_status() == 0
        replayed = _outputs(op)
        h_in, h_post, h_res, h_pre = (t.cpu().numpy() for t in replayed)
        ref = orc.mhc_pre(xb, True, phi, alpha, bias, gamma)
        assert_close_f32("hPost", h_post.reshape(T, n), ref["h_post"])
        assert_close_f32("hRes", h_res.reshape(T, n, n), ref["h_res"])
        assert_close_f32("hPre", h_pre.reshape(T, n), ref["h_pre"])
        assert_hin(h_in.view(np.uint16).reshape(T, D), ref["h_in"], xb, True,
                   h_pre.reshape(T, n), ref["h_pre"], orc, ref=ref)
        op.launch_no_alloc()
        torch.cuda.synchronize()
        eager = _outputs(op)
        for g, w, name in zip(replayed, eager, ("hIn", "hPost", "hRes", "hPre")):
            assert torch.equal(g, w), (i, name)
    del graph
    op.close()
