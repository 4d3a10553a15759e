"""ctypes binding of ``include/mhc_pre.h`` (libmhcpre.so).

Mirrors the reference's two-phase aclnn usage (cloud_runner/runner.cpp:440-476):
phase 1 ``mhcPreGetWorkspaceSize`` validates and returns (workspace bytes,
executor); phase 2 ``mhcPre`` launches on a stream.  PyTorch supplies device
memory and the stream handle only.
"""
from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path
from typing import Optional, Sequence

MHC_DTYPE_FLOAT = 0
MHC_DTYPE_FLOAT16 = 1
MHC_DTYPE_BF16 = 27
MHC_MAX_DIMS = 8

STATUS = {
    0: "MHC_STATUS_SUCCESS",
    1: "MHC_STATUS_NULL_ARGUMENT",
    2: "MHC_STATUS_INVALID_SHAPE",
    3: "MHC_STATUS_UNSUPPORTED_SHAPE",
    4: "MHC_STATUS_INVALID_DTYPE",
    5: "MHC_STATUS_WORKSPACE_TOO_SMALL",
    6: "MHC_STATUS_HIP_ERROR",
    7: "MHC_STATUS_DEVICE_MISMATCH",
    8: "MHC_STATUS_DEVICE_TIMEOUT",
    9: "MHC_STATUS_MISALIGNED",
    10: "MHC_STATUS_SCRATCH_TOO_SMALL",
}
STATUS_CODE = {v: k for k, v in STATUS.items()}

_PKG_DIR = Path(__file__).resolve().parent
_REPO_DIR = _PKG_DIR.parent
HEADER = _REPO_DIR / "include" / "mhc_pre.h"


class MhcTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("dims", ctypes.c_int64 * MHC_MAX_DIMS),
    ]


class MhcPreError(RuntimeError):
    def __init__(self, where: str, status: int):
        super().__init__(f"{where} failed: {STATUS.get(status, status)} ({status})")
        self.status = status


def library_path() -> Path:
    return Path(os.environ.get("MHCPRE_LIB", _PKG_DIR / "libmhcpre.so"))


_LIB: Optional[ctypes.CDLL] = None


def load_library() -> ctypes.CDLL:
    """Load libmhcpre.so.  Raises if it is absent: there is no fallback path."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = library_path()
    if not path.exists():
        raise FileNotFoundError(
            f"{path} not built; build it with `make -C mhcpre-review_amd/csrc` "
            "or __graft_entry__.build()")
    lib = ctypes.CDLL(str(path))
    P = ctypes.POINTER
    T = P(MhcTensor)
    exe = ctypes.c_void_p
    lib.mhcPreGetWorkspaceSize.argtypes = [T, T, T, T, T, ctypes.c_float, ctypes.c_float,
                                           T, T, T, P(ctypes.c_uint64), P(exe)]
    lib.mhcPreGetWorkspaceSize.restype = ctypes.c_int
    lib.mhcPreGetWorkspaceSizeWithHPre.argtypes = [T, T, T, T, T, ctypes.c_float,
                                                   ctypes.c_float, T, T, T, T,
                                                   P(ctypes.c_uint64), P(exe)]
    lib.mhcPreGetWorkspaceSizeWithHPre.restype = ctypes.c_int
    lib.mhcPre.argtypes = [ctypes.c_void_p, ctypes.c_uint64, exe, ctypes.c_void_p]
    lib.mhcPre.restype = ctypes.c_int
    lib.mhcPreExecutorDestroy.argtypes = [exe]
    lib.mhcPreExecutorDestroy.restype = ctypes.c_int
    lib.mhcPreQueryDeviceStatus.argtypes = [ctypes.c_void_p, ctypes.c_uint64, exe,
                                            ctypes.c_void_p]
    lib.mhcPreQueryDeviceStatus.restype = ctypes.c_int
    lib.mhcPreStatusString.argtypes = [ctypes.c_int]
    lib.mhcPreStatusString.restype = ctypes.c_char_p
    lib.mhcPreExecutorPath.argtypes = [exe, P(ctypes.c_char_p)]
    lib.mhcPreExecutorPath.restype = ctypes.c_int
    lib.mhcPreNoAlloc.argtypes = [exe, ctypes.c_void_p]
    lib.mhcPreNoAlloc.restype = ctypes.c_int
    lib.mhcPreExecutorSetStatusWord.argtypes = [exe, ctypes.c_void_p]
    lib.mhcPreExecutorSetStatusWord.restype = ctypes.c_int
    w = ctypes.c_void_p
    lib.mhcPrePrepareWeightsSize.argtypes = [T, T, ctypes.c_int32, P(ctypes.c_uint64)]
    lib.mhcPrePrepareWeightsSize.restype = ctypes.c_int
    lib.mhcPrePrepareWeights.argtypes = [T, T, ctypes.c_int32, ctypes.c_void_p, ctypes.c_uint64,
                                         ctypes.c_uint64, ctypes.c_void_p, P(w)]
    lib.mhcPrePrepareWeights.restype = ctypes.c_int
    lib.mhcPreWeightsVersion.argtypes = [w, P(ctypes.c_uint64)]
    lib.mhcPreWeightsVersion.restype = ctypes.c_int
    lib.mhcPreWeightsDestroy.argtypes = [w]
    lib.mhcPreWeightsDestroy.restype = ctypes.c_int
    lib.mhcPreGetWorkspaceSizePrepared.argtypes = [T, w, T, T, ctypes.c_float, ctypes.c_float,
                                                   T, T, T, T, P(ctypes.c_uint64), P(exe)]
    lib.mhcPreGetWorkspaceSizePrepared.restype = ctypes.c_int
    lib.mhcPreStreamProbe.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p,
                                      ctypes.c_uint64, ctypes.c_int32, ctypes.c_void_p]
    lib.mhcPreStreamProbe.restype = ctypes.c_int
    _LIB = lib
    return lib


def exported_symbols(header: Path = HEADER) -> list[str]:
    """Names of the functions the public header declares (MHC_API ...)."""
    text = header.read_text()
    return re.findall(r"^MHC_API\s+[\w\s\*]*?\b(\w+)\s*\(", text, flags=re.MULTILINE)


def make_tensor(data_ptr: int, dtype: int, dims: Sequence[int]) -> MhcTensor:
    t = MhcTensor()
    t.data = ctypes.c_void_p(int(data_ptr)) if data_ptr else None
    t.dtype = int(dtype)
    t.ndim = len(dims)
    if t.ndim > MHC_MAX_DIMS:
        raise ValueError("too many dims")
    for i, d in enumerate(dims):
        t.dims[i] = int(d)
    return t


def _torch_dtype_code(dt) -> int:
    import torch

    return {torch.float32: MHC_DTYPE_FLOAT, torch.float16: MHC_DTYPE_FLOAT16,
            torch.bfloat16: MHC_DTYPE_BF16}[dt]


def tensor_desc(t, dims: Optional[Sequence[int]] = None) -> MhcTensor:
    """Descriptor over a torch tensor's device memory (must be contiguous)."""
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return make_tensor(t.data_ptr(), _torch_dtype_code(t.dtype),
                       list(t.shape) if dims is None else list(dims))


def _stream_handle(stream) -> int:
    import torch

    if stream is None:
        stream = torch.cuda.current_stream()
    return int(stream.cuda_stream)


class MhcPreWeights:
    """Prepared B operand (mhcPrePrepareWeights): gamma (.) phi as bf16 hi + lo
    MFMA fragments in a device buffer this object owns (a torch tensor).
    ``prepare`` recomputes it in place from new weights of the same shapes and
    records the new version; executors created from this object read the new
    contents from their next launch on."""

    def __init__(self, phi, gamma, n: int, version: int = 0, stream=None):
        import torch

        self.lib = load_library()
        self.n = int(n)
        self.handle = ctypes.c_void_p(None)
        size = ctypes.c_uint64(0)
        pd = tensor_desc(phi)
        gd = tensor_desc(gamma) if gamma is not None else None
        st = self.lib.mhcPrePrepareWeightsSize(ctypes.byref(pd),
                                               ctypes.byref(gd) if gd is not None else None,
                                               ctypes.c_int32(self.n), ctypes.byref(size))
        if st != 0:
            raise MhcPreError("mhcPrePrepareWeightsSize", st)
        self.bytes = int(size.value)
        self.buffer = torch.empty(max(self.bytes, 256), dtype=torch.uint8, device=phi.device)
        self.prepare(phi, gamma, version, stream)

    def prepare(self, phi, gamma, version: int, stream=None) -> None:
        import torch

        pd = tensor_desc(phi)
        gd = tensor_desc(gamma) if gamma is not None else None
        handle = ctypes.c_void_p(None)
        with torch.cuda.device(self.buffer.device):
            st = self.lib.mhcPrePrepareWeights(
                ctypes.byref(pd), ctypes.byref(gd) if gd is not None else None,
                ctypes.c_int32(self.n), ctypes.c_void_p(self.buffer.data_ptr()),
                ctypes.c_uint64(self.bytes), ctypes.c_uint64(int(version)),
                ctypes.c_void_p(_stream_handle(stream)), ctypes.byref(handle))
        if st != 0:
            raise MhcPreError("mhcPrePrepareWeights", st)
        self.close()
        self.handle = handle
        # phi and gamma are read by the enqueued preparation: keep them alive
        # until it has run (the caller's stream order covers later launches).
        self._inputs = (phi, gamma)

    @property
    def version(self) -> int:
        v = ctypes.c_uint64(0)
        st = self.lib.mhcPreWeightsVersion(self.handle, ctypes.byref(v))
        if st != 0:
            raise MhcPreError("mhcPreWeightsVersion", st)
        return int(v.value)

    def close(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            self.lib.mhcPreWeightsDestroy(self.handle)
            self.handle = ctypes.c_void_p(None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MhcPreOp:
    """One executor plus its workspace: phase 1 at construction, phase 2 per launch.

    Outputs not given are allocated on x's device.  ``h_pre=True`` allocates the
    optional hPre output (extension entry point).  phi is passed with its
    declared shape [n*D, M] unless ``phi_dims`` overrides it; its memory is
    read as [M][K] either way.  With ``weights`` (a :class:`MhcPreWeights`)
    the executor comes from mhcPreGetWorkspaceSizePrepared, and phi and gamma
    must be None.
    """

    def __init__(self, x, phi, alpha, bias, gamma=None, norm_eps: float = 1e-6,
                 hc_eps: float = 1e-6, h_in=None, h_post=None, h_res=None, h_pre=None,
                 phi_dims=None, workspace=None, weights=None):
        import torch

        self.lib = load_library()
        lead = list(x.shape[:-2])
        n, D = int(x.shape[-2]), int(x.shape[-1])
        dev = x.device
        self.h_in = h_in if h_in is not None else torch.empty(lead + [D], dtype=x.dtype,
                                                               device=dev)
        self.h_post = h_post if h_post is not None else torch.empty(lead + [n],
                                                                    dtype=torch.float32,
                                                                    device=dev)
        self.h_res = h_res if h_res is not None else torch.empty(lead + [n, n],
                                                                 dtype=torch.float32,
                                                                 device=dev)
        if h_pre is True:
            h_pre = torch.empty(lead + [n], dtype=torch.float32, device=dev)
        self.h_pre = h_pre if h_pre is not False else None
        # Keep the inputs alive as long as the executor that binds them.
        self._keep = (x, phi, alpha, bias, gamma, weights)
        outs = [tensor_desc(self.h_in), tensor_desc(self.h_post), tensor_desc(self.h_res)]
        ws = ctypes.c_uint64(0)
        exe = ctypes.c_void_p(None)
        hp = tensor_desc(self.h_pre) if self.h_pre is not None else None
        hpp = ctypes.byref(hp) if hp is not None else None
        if weights is not None:
            if phi is not None or gamma is not None:
                raise ValueError("with prepared weights, phi and gamma must be None")
            xd, ad, bd = tensor_desc(x), tensor_desc(alpha), tensor_desc(bias)
            st = self.lib.mhcPreGetWorkspaceSizePrepared(
                ctypes.byref(xd), weights.handle, ctypes.byref(ad), ctypes.byref(bd),
                ctypes.c_float(norm_eps), ctypes.c_float(hc_eps), *[ctypes.byref(d) for d in outs],
                hpp, ctypes.byref(ws), ctypes.byref(exe))
        else:
            descs = [tensor_desc(x), tensor_desc(phi, phi_dims), tensor_desc(alpha),
                     tensor_desc(bias)]
            g = tensor_desc(gamma) if gamma is not None else None
            gp = ctypes.byref(g) if g is not None else None
            if hp is not None:
                st = self.lib.mhcPreGetWorkspaceSizeWithHPre(
                    *[ctypes.byref(d) for d in descs], gp, ctypes.c_float(norm_eps),
                    ctypes.c_float(hc_eps), *[ctypes.byref(d) for d in outs], hpp,
                    ctypes.byref(ws), ctypes.byref(exe))
            else:
                st = self.lib.mhcPreGetWorkspaceSize(
                    *[ctypes.byref(d) for d in descs], gp, ctypes.c_float(norm_eps),
                    ctypes.c_float(hc_eps), *[ctypes.byref(d) for d in outs], ctypes.byref(ws),
                    ctypes.byref(exe))
        if st != 0:
            raise MhcPreError("mhcPreGetWorkspaceSize", st)
        self.executor = exe
        self.workspace_size = int(ws.value)
        if workspace is not None:
            if workspace.numel() * workspace.element_size() < self.workspace_size:
                self.close()
                raise MhcPreError("workspace", STATUS_CODE["MHC_STATUS_WORKSPACE_TOO_SMALL"])
            self.workspace = workspace
        else:
            self.workspace = torch.empty(max(self.workspace_size, 256), dtype=torch.uint8,
                                         device=dev)
        # Launch arguments that stay fixed for the executor's lifetime.
        self._dev_index = self.workspace.device.index
        self._ws_ptr = ctypes.c_void_p(self.workspace.data_ptr())
        self._ws_size = ctypes.c_uint64(self.workspace_size)

    @property
    def path(self) -> str:
        name = ctypes.c_char_p()
        st = self.lib.mhcPreExecutorPath(self.executor, ctypes.byref(name))
        if st != 0:
            raise MhcPreError("mhcPreExecutorPath", st)
        return name.value.decode()

    def launch(self, stream=None, check: bool = False) -> None:
        """Enqueue one launch (phase 2) on ``stream`` (default: the current
        stream of the tensors' device).  With ``check=True`` the call then
        synchronizes the stream and raises MhcPreError(MHC_STATUS_DEVICE_TIMEOUT)
        if a bounded wait between workgroups expired; the rows that wait was
        for hold NaN in every output in that case, never a plausible value."""
        import torch

        # The library launches on the current device, which must hold the
        # tensors; the default stream is that device's current stream.
        if torch.cuda.current_device() != self._dev_index:
            with torch.cuda.device(self._dev_index):
                st = self.lib.mhcPre(self._ws_ptr, self._ws_size, self.executor,
                                     ctypes.c_void_p(_stream_handle(stream)))
        else:
            st = self.lib.mhcPre(self._ws_ptr, self._ws_size, self.executor,
                                 ctypes.c_void_p(_stream_handle(stream)))
        if st != 0:
            raise MhcPreError("mhcPre", st)
        if check:
            self.check(stream)

    def launch_no_alloc(self, stream=None) -> None:
        """Enqueue one launch through mhcPreNoAlloc: the library's built-in
        per-device scratch array is the workspace (this object's workspace
        tensor is not used) and the call allocates nothing."""
        import torch

        if torch.cuda.current_device() != self._dev_index:
            with torch.cuda.device(self._dev_index):
                st = self.lib.mhcPreNoAlloc(self.executor, ctypes.c_void_p(_stream_handle(stream)))
        else:
            st = self.lib.mhcPreNoAlloc(self.executor, ctypes.c_void_p(_stream_handle(stream)))
        if st != 0:
            raise MhcPreError("mhcPreNoAlloc", st)

    def set_status_word(self, word) -> None:
        """mhcPreExecutorSetStatusWord: ``word`` (a device int32 tensor, or
        None) becomes this executor's sticky status word; a later launch whose
        bounded wait expires stores MHC_STATUS_DEVICE_TIMEOUT into it.  The
        tensor must outlive the launches that may write it."""
        ptr = ctypes.c_void_p(word.data_ptr()) if word is not None else None
        st = self.lib.mhcPreExecutorSetStatusWord(self.executor, ptr)
        if st != 0:
            raise MhcPreError("mhcPreExecutorSetStatusWord", st)
        self._status_word = word

    def no_alloc_device_status(self, stream=None) -> int:
        """mhcPreQueryDeviceStatus on the built-in workspace of mhcPreNoAlloc
        launches (NULL workspace, size 0): synchronizes ``stream``."""
        return self.lib.mhcPreQueryDeviceStatus(None, ctypes.c_uint64(0), self.executor,
                                                ctypes.c_void_p(_stream_handle(stream)))

    def check(self, stream=None) -> None:
        """Synchronize ``stream`` and raise if this executor's latest launch
        reported an expired wait (mhcPreQueryDeviceStatus)."""
        st = self.device_status(stream)
        if st != 0:
            raise MhcPreError("mhcPreQueryDeviceStatus", st)

    def device_status(self, stream=None) -> int:
        return self.lib.mhcPreQueryDeviceStatus(ctypes.c_void_p(self.workspace.data_ptr()),
                                                ctypes.c_uint64(self.workspace_size),
                                                self.executor,
                                                ctypes.c_void_p(_stream_handle(stream)))

    def close(self) -> None:
        if getattr(self, "executor", None) is not None and self.executor.value:
            self.lib.mhcPreExecutorDestroy(self.executor)
            self.executor = ctypes.c_void_p(None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def outputs(self):
        return self.h_in, self.h_post, self.h_res, self.h_pre


def stream_probe(src, read_bytes: int, dst, write_bytes: int, workgroups: int = 0,
                 stream=None) -> None:
    """Enqueue one launch of the library's stream probe (mhcPreStreamProbe):
    reads `read_bytes` of the device tensor `src` and writes `write_bytes` of
    `dst` in the best-served access pattern, with no arithmetic.  A
    measurement aid: timing it gives a bandwidth ceiling for a byte mix."""
    import torch

    lib = load_library()
    if read_bytes > src.numel() * src.element_size() or write_bytes > dst.numel() * dst.element_size():
        raise ValueError("stream_probe: byte counts exceed the tensors")
    with torch.cuda.device(src.device):
        st = lib.mhcPreStreamProbe(ctypes.c_void_p(src.data_ptr()), ctypes.c_uint64(read_bytes),
                                   ctypes.c_void_p(dst.data_ptr()), ctypes.c_uint64(write_bytes),
                                   ctypes.c_int32(workgroups),
                                   ctypes.c_void_p(_stream_handle(stream)))
    if st != 0:
        raise MhcPreError("mhcPreStreamProbe", st)


def mhc_pre(x, phi, alpha, bias, gamma=None, norm_eps: float = 1e-6, hc_eps: float = 1e-6,
            h_pre: bool = False, stream=None):
    """One call: returns (hIn, hPost, hRes, hPre-or-None) once the launch has
    finished.  The workspace must outlive the launch, so this call waits for
    the stream anyway, and checks the device status on the way: an expired
    wait between workgroups raises MhcPreError."""
    op = MhcPreOp(x, phi, alpha, bias, gamma, norm_eps, hc_eps, h_pre=True if h_pre else None)
    try:
        op.launch(stream, check=True)
    finally:
        outs = op.outputs()
        op.close()
    return outs
