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

Phase 1 is cheap on a repeated shape: the library caches the plan per shape,
dtypes, gamma presence, eps and device, and each call only validates and
binds the new tensors.

Expired waits.  The persistent kernels' workgroups wait on each other with a
bound; if another kernel holds CUs they need (an RCCL kernel on a
communication stream, say), a wait can expire and the rows it was for come
out NaN.  Every executor this module creates reports such a launch in a
per-device sticky status word (mhcPreExecutorSetStatusWord): read it with
:func:`device_status` after any synchronization of your own, clear it with
:func:`clear_device_status`.  MHCPRE_CHECK_STATUS=1 instead synchronizes after
every call and raises.
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


_STATUS_WORDS: dict = {}


def _status_word(device: torch.device) -> torch.Tensor:
    """The per-device sticky status word of this module's executors (one
    int32, zero until a launch's bounded wait expires)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    word = _STATUS_WORDS.get(index)
    if word is None:
        word = torch.zeros(1, dtype=torch.int32, device=torch.device("cuda", index))
        _STATUS_WORDS[index] = word
    return word


def device_status(device=None) -> int:
    """0, or MHC_STATUS_DEVICE_TIMEOUT (8) if a launch of this module on
    ``device`` (default: the current one) left NaN rows since the last
    :func:`clear_device_status`.  Reading the word waits for the launches
    enqueued before it on the current stream, as any read of a device tensor
    does; it adds no synchronization of the op's own."""
    dev = torch.device("cuda", torch.cuda.current_device() if device is None else
                       torch.device(device).index)
    return int(_status_word(dev).item())


def clear_device_status(device=None) -> None:
    dev = torch.device("cuda", torch.cuda.current_device() if device is None else
                       torch.device(device).index)
    _status_word(dev).zero_()


def _launch(x, phi, alpha, bias, gamma, norm_eps, hc_eps, with_h_pre):
    args = [t.contiguous() for t in (x, phi, alpha, bias)]
    g = gamma.contiguous() if gamma is not None else None
    op = MhcPreOp(*args, g, norm_eps, hc_eps, h_pre=True if with_h_pre else None)
    op.set_status_word(_status_word(x.device))
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
