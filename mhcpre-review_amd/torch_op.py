"""PyTorch operator registration: ``torch.ops.mhcpre.mhc_pre`` and
``torch.ops.mhcpre.mhc_pre_with_h_pre``.

The two operators mirror the two phase-1 entry points of the C ABI
(``mhcPreGetWorkspaceSize`` and ``mhcPreGetWorkspaceSizeWithHPre``, the
latter also writing hPre): each call runs phase 1 on the given tensors,
allocates the workspace from PyTorch's caching allocator and launches on the
current stream.  Arguments, defaults and validation are those of the
reference operator (``code/op_host/mhc_pre.cpp:57-79,126-130,217-257,
297-298``): x ``[..., n, D]`` fp16/bf16, phi ``[n*D, M]`` fp32 read as memory
``[M][K]``, alpha ``[3]``, bias ``[M]``, gamma ``[n, D]`` or None.  Outputs are
new tensors: hIn ``[..., D]`` (x's dtype), hPost ``[..., n]``, hRes
``[..., n, n]`` and hPre ``[..., n]`` (fp32).

Only device (ROCm "cuda") tensors have a kernel; the fake implementation
gives shapes and dtypes for tracing (meta / fake tensors, torch.compile).
There is no CPU implementation and no autograd formula (the reference
operator is forward-only).
"""
from __future__ import annotations

import os
from typing import Optional

import torch

from .binding import MhcPreOp

_LIB_NAME = "mhcpre"


def _check_status() -> bool:
    # MHCPRE_CHECK_STATUS=1: every launch waits for its stream and raises
    # MhcPreError(MHC_STATUS_DEVICE_TIMEOUT) if a bounded wait between
    # workgroups expired.  Off by default (it synchronizes); without it such a
    # launch leaves NaN in the outputs of the rows it could not finish.
    return os.environ.get("MHCPRE_CHECK_STATUS", "") not in ("", "0")


def _launch(x, phi, alpha, bias, gamma, norm_eps, hc_eps, with_h_pre):
    args = [t.contiguous() for t in (x, phi, alpha, bias)]
    g = gamma.contiguous() if gamma is not None else None
    op = MhcPreOp(*args, g, norm_eps, hc_eps, h_pre=True if with_h_pre else None)
    try:
        op.launch(check=_check_status())
    finally:
        # The executor is host data; the workspace tensor returns to the caching
        # allocator when `op` goes, in the order of the current stream, after
        # the launch that uses it.
        op.close()
    return op.h_in, op.h_post, op.h_res, op.h_pre


@torch.library.custom_op(f"{_LIB_NAME}::mhc_pre", mutates_args=(), device_types="cuda")
def mhc_pre(x: torch.Tensor, phi: torch.Tensor, alpha: torch.Tensor, bias: torch.Tensor,
            gamma: Optional[torch.Tensor] = None, norm_eps: float = 1e-6,
            hc_eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    h_in, h_post, h_res, _ = _launch(x, phi, alpha, bias, gamma, norm_eps, hc_eps, False)
    return h_in, h_post, h_res


@torch.library.custom_op(f"{_LIB_NAME}::mhc_pre_with_h_pre", mutates_args=(),
                         device_types="cuda")
def mhc_pre_with_h_pre(x: torch.Tensor, phi: torch.Tensor, alpha: torch.Tensor,
                       bias: torch.Tensor, gamma: Optional[torch.Tensor] = None,
                       norm_eps: float = 1e-6, hc_eps: float = 1e-6
                       ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    return _launch(x, phi, alpha, bias, gamma, norm_eps, hc_eps, True)


def _fake_outputs(x):
    # The C ABI accepts x as [B, S, n, D] (the reference's layout) or [T, n, D].
    if x.dim() not in (3, 4):
        raise ValueError(f"x must be [B, S, n, D] or [T, n, D], got {tuple(x.shape)}")
    lead = tuple(x.shape[:-2])
    n, D = x.shape[-2], x.shape[-1]
    return (x.new_empty(lead + (D,)),
            x.new_empty(lead + (n,), dtype=torch.float32),
            x.new_empty(lead + (n, n), dtype=torch.float32),
            x.new_empty(lead + (n,), dtype=torch.float32))


@mhc_pre.register_fake
def _(x, phi, alpha, bias, gamma=None, norm_eps=1e-6, hc_eps=1e-6):
    return _fake_outputs(x)[:3]


@mhc_pre_with_h_pre.register_fake
def _(x, phi, alpha, bias, gamma=None, norm_eps=1e-6, hc_eps=1e-6):
    return _fake_outputs(x)
