"""torch.library registration of the operator (``torch.ops.mhcpre``).

CPU part: the schema, shape/dtype inference of the fake implementation (meta
and fake tensors), and that host tensors have no kernel.  GPU part: the
operator against the ctypes executor and the CPU oracle, and under
torch.compile (which traces with the fake implementation).
"""
from __future__ import annotations

import numpy as np
import pytest


@pytest.fixture(scope="module")
def ops(pkg):
    import torch

    pkg.torch_ops()
    return torch.ops.mhcpre


@pytest.mark.parametrize("lead", [(5,), (2, 3)])
@pytest.mark.parametrize("n", [4, 6, 8])
def test_fake_shapes(ops, lead, n):
    import torch

    D, M = 64, n * n + 2 * n
    x = torch.empty(*lead, n, D, dtype=torch.bfloat16, device="meta")
    phi = torch.empty(n * D, M, device="meta")
    alpha, bias = torch.empty(3, device="meta"), torch.empty(M, device="meta")
    h_in, h_post, h_res = ops.mhc_pre(x, phi, alpha, bias)
    assert (h_in.shape, h_in.dtype) == (torch.Size(lead + (D,)), torch.bfloat16)
    assert (h_post.shape, h_post.dtype) == (torch.Size(lead + (n,)), torch.float32)
    assert (h_res.shape, h_res.dtype) == (torch.Size(lead + (n, n)), torch.float32)
    outs = ops.mhc_pre_with_h_pre(x, phi, alpha, bias, torch.empty(n, D, device="meta"),
                                  1e-5, 0.0)
    assert len(outs) == 4 and outs[3].shape == torch.Size(lead + (n,))


def test_fake_tensor_mode(ops):
    import torch
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        x = torch.empty(7, 4, 128, dtype=torch.float16, device="cuda")
        outs = ops.mhc_pre(x, torch.empty(512, 24, device="cuda"), torch.empty(3, device="cuda"),
                           torch.empty(24, device="cuda"))
        assert [tuple(o.shape) for o in outs] == [(7, 128), (7, 4), (7, 4, 4)]
        assert outs[0].dtype == torch.float16


def test_rejects_bad_rank_in_tracing(ops):
    import torch

    with pytest.raises(ValueError):
        ops.mhc_pre(torch.empty(4, 64, dtype=torch.bfloat16, device="meta"),
                    torch.empty(256, 24, device="meta"), torch.empty(3, device="meta"),
                    torch.empty(24, device="meta"))


def test_host_tensors_have_no_kernel(ops):
    import torch

    with pytest.raises(NotImplementedError):
        ops.mhc_pre(torch.zeros(1, 4, 64, dtype=torch.bfloat16), torch.zeros(256, 24),
                    torch.zeros(3), torch.zeros(24))


def _inputs(device, T=160, n=4, D=512, seed=3):
    import torch

    rng = np.random.default_rng(seed)
    K, M = n * D, n * n + 2 * n
    x = torch.from_numpy(rng.standard_normal((T, n, D)).astype(np.float32)).to(
        device).to(torch.bfloat16)
    f = lambda a: torch.from_numpy(np.asarray(a, dtype=np.float32)).to(device)
    phi = f(rng.standard_normal((M, K)) / np.sqrt(K))  # memory [M][K], as the kernel reads it
    alpha = f([0.3, -0.2, 0.05])
    bias = f(rng.uniform(-0.5, 0.5, M))
    gamma = f(1 + 0.1 * rng.standard_normal((n, D)))
    return x, phi, alpha, bias, gamma


@pytest.mark.gpu
def test_op_matches_executor_and_oracle(pkg, orc, device, ops):
    import torch

    from helpers import assert_close_f32

    x, phi, alpha, bias, gamma = _inputs(device)
    h_in, h_post, h_res, h_pre = ops.mhc_pre_with_h_pre(x, phi, alpha, bias, gamma)
    op = pkg.MhcPreOp(x, phi, alpha, bias, gamma, h_pre=True)
    op.launch()
    torch.cuda.synchronize()
    assert op.device_status() == 0
    for a, b in zip((h_in, h_post, h_res, h_pre), op.outputs()):
        assert torch.equal(a, b)
    op.close()
    three = ops.mhc_pre(x, phi, alpha, bias, gamma)
    for a, b in zip(three, (h_in, h_post, h_res)):
        assert torch.equal(a, b)
    x_bits = x.view(torch.int16).cpu().numpy().view(np.uint16)
    ref = orc.mhc_pre(x_bits, True, phi.cpu().numpy(), alpha.cpu().numpy(), bias.cpu().numpy(),
                      gamma.cpu().numpy().reshape(-1))
    assert_close_f32("hPre", h_pre.cpu().numpy(), ref["h_pre"])
    assert_close_f32("hPost", h_post.cpu().numpy(), ref["h_post"])
    assert_close_f32("hRes", h_res.cpu().numpy(), ref["h_res"])


@pytest.mark.gpu
def test_op_under_torch_compile(pkg, device, ops):
    import torch

    x, phi, alpha, bias, gamma = _inputs(device, T=48, D=256, seed=5)

    def f(x, phi, alpha, bias, gamma):
        h_in, h_post, h_res = ops.mhc_pre(x, phi, alpha, bias, gamma)
        return h_in.float().sum(-1), h_post * 2, h_res

    eager = f(x, phi, alpha, bias, gamma)
    compiled = torch.compile(f, backend="aot_eager", fullgraph=True)(x, phi, alpha, bias, gamma)
    for a, b in zip(eager, compiled):
        assert torch.equal(a, b)
