"""Expired waits reported without an extra synchronize.

The strip and fused kernels' workgroups wait on each other with a bound;
MHCPRE_SPIN_LIMIT=0 at phase 1 (a test knob, read under MHCPRE_TESTING=1)
makes a wait give up at its first poll that finds the data missing, from the
host side, so every kernel still ends normally.  A launch whose wait expired
stores MHC_STATUS_DEVICE_TIMEOUT into the executor's sticky status word
(mhcPreExecutorSetStatusWord), which the caller reads after a synchronization
of its own; nothing else writes the word.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

from inputs import to_bits

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _inputs(pkg, device, T, n, D, seed):
    import torch

    K, M = n * D, n * n + 2 * n
    rng = np.random.default_rng(seed)
    x = to_bits(rng.standard_normal((T, n, D)).astype(np.float32), True)
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)
    xt = torch.from_numpy(x.view(np.int16)).to(device).view(torch.bfloat16)
    phi = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    return (xt, f(phi), f(np.full(3, 0.01, dtype=np.float32)),
            f(rng.uniform(-0.1, 0.1, M)), f(1 + 0.1 * rng.standard_normal(K)))


def _op(pkg, args, force, spin_zero):
    os.environ["MHCPRE_FORCE_PATH"] = force
    if spin_zero:
        os.environ["MHCPRE_SPIN_LIMIT"] = "0"
    try:
        return pkg.MhcPreOp(*args, h_pre=True)
    finally:
        os.environ.pop("MHCPRE_FORCE_PATH", None)
        os.environ.pop("MHCPRE_SPIN_LIMIT", None)


@pytest.mark.parametrize("force,n,T,D", [("strip", 4, 2048, 7168), ("fused", 4, 2048, 1024)])
def test_status_word_reports_an_expired_wait(pkg, device, force, n, T, D):
    import torch

    timeout = pkg.binding.STATUS_CODE["MHC_STATUS_DEVICE_TIMEOUT"]
    args = _inputs(pkg, device, T, n, D, 81)
    bad = _op(pkg, args, force, True)
    good = _op(pkg, args, force, False)
    assert bad.path == force and good.path == force
    _say(f"[status word] {force} T={T} D={D}")
    word_bad = torch.zeros(1, dtype=torch.int32, device=device)
    word_good = torch.zeros(1, dtype=torch.int32, device=device)
    bad.set_status_word(word_bad)
    good.set_status_word(word_good)
    bad.launch()
    good.launch()
    good.launch()
    torch.cuda.synchronize()  # the caller's own synchronization; the library adds none
    assert int(word_bad.item()) == timeout
    assert int(word_good.item()) == 0
    assert torch.isnan(bad.h_pre).any() or torch.isnan(bad.h_in.float()).any()
    assert not torch.isnan(good.h_in.float()).any()
    # Sticky: a clean launch does not clear it; the caller does.
    good.set_status_word(word_bad)
    good.launch()
    torch.cuda.synchronize()
    assert int(word_bad.item()) == timeout
    word_bad.zero_()
    good.launch()
    torch.cuda.synchronize()
    assert int(word_bad.item()) == 0
    # Turned off: the word is not written any more.
    bad.set_status_word(None)
    bad.launch()
    torch.cuda.synchronize()
    assert int(word_bad.item()) == 0
    assert bad.device_status() == timeout
    bad.close()
    good.close()


def test_torch_op_reports_expired_waits_in_its_status_word(pkg, device):
    import torch

    torch_op = pkg.torch_ops()
    ops = torch.ops.mhcpre
    timeout = pkg.binding.STATUS_CODE["MHC_STATUS_DEVICE_TIMEOUT"]
    xt, phi, alpha, bias, gamma = _inputs(pkg, device, 2048, 4, 7168, 82)
    torch_op.clear_device_status()
    ops.mhc_pre(xt, phi, alpha, bias, gamma)
    assert torch_op.device_status() == 0
    _say("[status word] torch op, spin limit 0")
    os.environ["MHCPRE_SPIN_LIMIT"] = "0"
    try:
        h_in, _, _ = ops.mhc_pre(xt, phi, alpha, bias, gamma)
    finally:
        os.environ.pop("MHCPRE_SPIN_LIMIT", None)
    torch.cuda.synchronize()
    assert torch_op.device_status() == timeout
    assert torch.isnan(h_in.float()).any()
    torch_op.clear_device_status()
    h_in, _, _ = ops.mhc_pre(xt, phi, alpha, bias, gamma)
    assert torch_op.device_status() == 0
    assert not torch.isnan(h_in.float()).any()
