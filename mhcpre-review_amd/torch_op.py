"""PyTorch operators ``torch.ops.mhcpre.mhc_pre`` and
``torch.ops.mhcpre.mhc_pre_with_h_pre``.

The operators are native: ``libmhcpre_torch.so`` (built from
``csrc/mhc_pre_torch.cpp``) registers them with PyTorch's dispatcher and calls
the C ABI of ``libmhcpre.so`` from C++.  They mirror the two phase-1 entry
points of the C ABI (``mhcPreGetWorkspaceSize`` and
``mhcPreGetWorkspaceSizeWithHPre``, the latter also writing hPre): each call
runs phase 1 on the given tensors, allocates the outputs and the workspace
from PyTorch's caching allocator and launches on the current stream.
Arguments, defaults and validation are those of the reference operator
(``code/op_host/mhc_pre.cpp:57-79,126-130,217-257,297-298``): x
``[..., n, D]`` fp16/bf16, phi ``[n*D, M]`` fp32 read as memory ``[M][K]``,
alpha ``[3]``, bias ``[M]``, gamma ``[n, D]`` or None.  Outputs are new
tensors: hIn ``[..., D]`` (x's dtype), hPost ``[..., n]``, hRes
``[..., n, n]`` and hPre ``[..., n]`` (fp32).  A status the library returns
is raised as RuntimeError naming it.

Only device (ROCm "cuda") tensors have a kernel; the fake implementation
registered here gives shapes and dtypes for tracing (meta / fake tensors,
torch.compile).  There is no CPU implementation and no autograd formula (the
reference operator is forward-only).

Phase 1 is cheap on a repeated shape: the library caches the plan per shape,
dtypes, gamma presence, eps and device, and each call only validates and
binds the new tensors.

Expired waits.  The persistent kernels' workgroups wait on each other with a
bound; if another kernel holds CUs they need (an RCCL kernel on a
communication stream, say), a wait can expire and the rows it was for come
out NaN.  Every executor the operators create reports such a launch in a
per-device sticky status word (mhcPreExecutorSetStatusWord): read it with
:func:`device_status` after any synchronization of your own, clear it with
:func:`clear_device_status`.  MHCPRE_CHECK_STATUS=1 instead synchronizes after
every call and raises.
"""
from __future__ import annotations

from pathlib import Path

import torch

from .binding import load_library

_LIB_NAME = "mhcpre"
_PKG_DIR = Path(__file__).resolve().parent


def library_path() -> Path:
    return _PKG_DIR / "libmhcpre_torch.so"


def _load() -> None:
    """Load the native operators.  Raises if they are not built: there is no
    Python fallback."""
    load_library()  # libmhcpre.so first (the operators' library links it in place)
    path = library_path()
    if not path.exists():
        raise FileNotFoundError(
            f"{path} not built; build it with `make -C mhcpre-review_amd/csrc torch` "
            "or __graft_entry__.build()")
    torch.ops.load_library(str(path))


_load()


def _device_index(device) -> int:
    if device is None:
        return torch.cuda.current_device()
    d = torch.device(device)
    return d.index if d.index is not None else torch.cuda.current_device()


def device_status(device=None) -> int:
    """0, or MHC_STATUS_DEVICE_TIMEOUT (8) if a launch of the operators on
    ``device`` (default: the current one) left NaN rows since the last
    :func:`clear_device_status`.  Reading the word waits for the launches
    enqueued before it on the current stream, as any read of a device tensor
    does; it adds no synchronization of the operators' own."""
    return int(torch.ops.mhcpre.status_word(_device_index(device)).item())


def clear_device_status(device=None) -> None:
    torch.ops.mhcpre.status_word(_device_index(device)).zero_()


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


@torch.library.register_fake(f"{_LIB_NAME}::mhc_pre")
def _(x, phi, alpha, bias, gamma=None, norm_eps=1e-6, hc_eps=1e-6):
    return _fake_outputs(x)[:3]


@torch.library.register_fake(f"{_LIB_NAME}::mhc_pre_with_h_pre")
def _(x, phi, alpha, bias, gamma=None, norm_eps=1e-6, hc_eps=1e-6):
    return _fake_outputs(x)
