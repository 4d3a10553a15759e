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


def _case(T, n, D, seed):
    rng = np.random.default_rng(seed)
    K, M = n * D, n * n + 2 * n
    x = to_bits(rng.standard_normal((T, n, D)).astype(np.float32), True)
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
                                         ([(600, 8, 2048), (100, 8, 2048)], "rows"),
                                         ([(600, 8, 1024), (520, 8, 1024)], "split")])
def test_no_alloc_matches_workspace_launch(pkg, orc, device, shapes, path):
    import torch

    f = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)
    for i, (T, n, D) in enumerate(shapes):
        _say(f"[no-alloc] call {i}: T={T} n={n} D={D}")
        x, phi, alpha, bias, gamma = _case(T, n, D, seed=900 + i)
        xt = torch.from_numpy(x.view(np.int16)).to(device).view(torch.bfloat16)
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
        ref = orc.mhc_pre(x, True, phi, alpha, bias, gamma)
        assert_close_f32("hPost", h_post.reshape(T, n), ref["h_post"])
        assert_close_f32("hRes", h_res.reshape(T, n, n), ref["h_res"])
        assert_close_f32("hPre", h_pre.reshape(T, n), ref["h_pre"])
        assert_hin(h_in.view(np.uint16).reshape(T, D), ref["h_in"], x, True,
                   h_pre.reshape(T, n), ref["h_pre"], orc)
        op.close()
