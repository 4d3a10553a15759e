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

import ctypes
import os
import threading
from typing import Optional

import torch

from .binding import MhcPreError, _torch_dtype_code, load_library, make_tensor

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


class _Descs:
    """The ctypes descriptors of one call shape (dims and dtypes fixed), built
    once per thread; a call only stores its tensors' addresses into them."""

    def __init__(self, x, phi, alpha, bias, gamma, with_h_pre):
        lead = list(x.shape[:-2])
        n, D = int(x.shape[-2]), int(x.shape[-1])
        f32 = _torch_dtype_code(torch.float32)
        xdt = _torch_dtype_code(x.dtype)
        self.lead, self.n, self.D = lead, n, D
        self.x = make_tensor(0, xdt, list(x.shape))
        self.phi = make_tensor(0, f32, list(phi.shape))
        self.alpha = make_tensor(0, f32, list(alpha.shape))
        self.bias = make_tensor(0, f32, list(bias.shape))
        self.gamma = make_tensor(0, f32, list(gamma.shape)) if gamma is not None else None
        self.h_in = make_tensor(0, xdt, lead + [D])
        self.h_post = make_tensor(0, f32, lead + [n])
        self.h_res = make_tensor(0, f32, lead + [n, n])
        self.h_pre = make_tensor(0, f32, lead + [n]) if with_h_pre else None
        self.ws = ctypes.c_uint64(0)
        self.exe = ctypes.c_void_p(None)


_DESCS: dict = {}
_DESCS_LOCK = threading.Lock()


def _descs(x, phi, alpha, bias, gamma, with_h_pre) -> _Descs:
    key = (tuple(x.shape), x.dtype, tuple(phi.shape), tuple(alpha.shape), tuple(bias.shape),
           None if gamma is None else tuple(gamma.shape), with_h_pre, threading.get_ident())
    d = _DESCS.get(key)
    if d is None:
        d = _Descs(x, phi, alpha, bias, gamma, with_h_pre)
        with _DESCS_LOCK:
            if len(_DESCS) >= 256:
                _DESCS.clear()
            _DESCS[key] = d
    return d


def _launch(x, phi, alpha, bias, gamma, norm_eps, hc_eps, with_h_pre):
    """Phase 1 (the library's plan cache makes it a validation and a pointer
    bind on a repeated shape), the workspace from the caching allocator, the
    status word, phase 2 on the current stream, and the executor freed.  The
    descriptors are this thread's, reused per call shape."""
    if x.device.index is not None and x.device.index != torch.cuda.current_device():
        # The library launches on the current device, which must hold x.
        with torch.cuda.device(x.device):
            return _launch(x, phi, alpha, bias, gamma, norm_eps, hc_eps, with_h_pre)
    x, phi, alpha, bias = (t.contiguous() for t in (x, phi, alpha, bias))
    gamma = gamma.contiguous() if gamma is not None else None
    lib = load_library()
    d = _descs(x, phi, alpha, bias, gamma, with_h_pre)
    dev = x.device
    h_in = torch.empty(d.lead + [d.D], dtype=x.dtype, device=dev)
    h_post = torch.empty(d.lead + [d.n], dtype=torch.float32, device=dev)
    h_res = torch.empty(d.lead + [d.n, d.n], dtype=torch.float32, device=dev)
    h_pre = torch.empty(d.lead + [d.n], dtype=torch.float32, device=dev) if with_h_pre else None
    d.x.data, d.phi.data, d.alpha.data, d.bias.data = (
        x.data_ptr(), phi.data_ptr(), alpha.data_ptr(), bias.data_ptr())
    if gamma is not None:
        d.gamma.data = gamma.data_ptr()
    d.h_in.data, d.h_post.data, d.h_res.data = h_in.data_ptr(), h_post.data_ptr(), h_res.data_ptr()
    g = ctypes.byref(d.gamma) if gamma is not None else None
    if with_h_pre:
        d.h_pre.data = h_pre.data_ptr()
        st = lib.mhcPreGetWorkspaceSizeWithHPre(
            ctypes.byref(d.x), ctypes.byref(d.phi), ctypes.byref(d.alpha), ctypes.byref(d.bias), g,
            ctypes.c_float(norm_eps), ctypes.c_float(hc_eps), ctypes.byref(d.h_in),
            ctypes.byref(d.h_post), ctypes.byref(d.h_res), ctypes.byref(d.h_pre),
            ctypes.byref(d.ws), ctypes.byref(d.exe))
    else:
        st = lib.mhcPreGetWorkspaceSize(
            ctypes.byref(d.x), ctypes.byref(d.phi), ctypes.byref(d.alpha), ctypes.byref(d.bias), g,
            ctypes.c_float(norm_eps), ctypes.c_float(hc_eps), ctypes.byref(d.h_in),
            ctypes.byref(d.h_post), ctypes.byref(d.h_res), ctypes.byref(d.ws), ctypes.byref(d.exe))
    if st != 0:
        raise MhcPreError("mhcPreGetWorkspaceSize", st)
    exe = d.exe.value
    try:
        # The workspace returns to the caching allocator when it goes, in the
        # order of the current stream, after the launch that uses it.
        ws = torch.empty(max(int(d.ws.value), 256), dtype=torch.uint8, device=dev)
        stream = torch.cuda.current_stream(dev).cuda_stream
        st = lib.mhcPreExecutorSetStatusWord(exe, _status_word(dev).data_ptr())
        if st == 0:
            st = lib.mhcPre(ws.data_ptr(), d.ws, exe, stream)
        if st != 0:
            raise MhcPreError("mhcPre", st)
        if _check_status():
            st = lib.mhcPreQueryDeviceStatus(ws.data_ptr(), d.ws, exe, stream)
            if st != 0:
                raise MhcPreError("mhcPreQueryDeviceStatus", st)
    finally:
        lib.mhcPreExecutorDestroy(exe)
    return h_in, h_post, h_res, h_pre


# The operators are defined with torch.library.Library and a CUDA kernel
# (device tensors only; there is no CPU kernel and no autograd formula): its
# dispatch costs a few microseconds per call, against ~13 us for the
# torch.library.custom_op wrapper on the same host.
_LIB = torch.library.Library(_LIB_NAME, "DEF")
_LIB.define("mhc_pre(Tensor x, Tensor phi, Tensor alpha, Tensor bias, Tensor? gamma=None, "
            "float norm_eps=1e-06, float hc_eps=1e-06) -> (Tensor, Tensor, Tensor)")
_LIB.define("mhc_pre_with_h_pre(Tensor x, Tensor phi, Tensor alpha, Tensor bias, "
            "Tensor? gamma=None, float norm_eps=1e-06, float hc_eps=1e-06) "
            "-> (Tensor, Tensor, Tensor, Tensor)")


def mhc_pre(x: torch.Tensor, phi: torch.Tensor, alpha: torch.Tensor, bias: torch.Tensor,
            gamma: Optional[torch.Tensor] = None, norm_eps: float = 1e-6,
            hc_eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    h_in, h_post, h_res, _ = _launch(x, phi, alpha, bias, gamma, norm_eps, hc_eps, False)
    return h_in, h_post, h_res


def mhc_pre_with_h_pre(x: torch.Tensor, phi: torch.Tensor, alpha: torch.Tensor,
                       bias: torch.Tensor, gamma: Optional[torch.Tensor] = None,
                       norm_eps: float = 1e-6, hc_eps: float = 1e-6
                       ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    return _launch(x, phi, alpha, bias, gamma, norm_eps, hc_eps, True)


_LIB.impl("mhc_pre", mhc_pre, "CUDA")
_LIB.impl("mhc_pre_with_h_pre", mhc_pre_with_h_pre, "CUDA")


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


@torch.library.register_fake(f"{_LIB_NAME}::mhc_pre", lib=_LIB)
def _(x, phi, alpha, bias, gamma=None, norm_eps=1e-6, hc_eps=1e-6):
    return _fake_outputs(x)[:3]


@torch.library.register_fake(f"{_LIB_NAME}::mhc_pre_with_h_pre", lib=_LIB)
def _(x, phi, alpha, bias, gamma=None, norm_eps=1e-6, hc_eps=1e-6):
    return _fake_outputs(x)
