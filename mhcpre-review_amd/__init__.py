"""MhcPre for AMD Instinct MI355X: Python plumbing over the C ABI.

The operator itself lives in ``libmhcpre.so`` (C++ host library + HIP kernels
for gfx950, built from ``csrc/``).  This package only binds that library with
ctypes and uses PyTorch-ROCm for device memory and streams, so tests and the
benchmark drive exactly the entry points a native caller would
(``include/mhc_pre.h``).  Nothing here computes the operator: if the library
is missing the import of :func:`load_library` fails loudly.
"""
from __future__ import annotations

from .binding import (  # noqa: F401
    MHC_DTYPE_BF16,
    MHC_DTYPE_FLOAT,
    MHC_DTYPE_FLOAT16,
    MHC_MAX_DIMS,
    STATUS,
    MhcPreError,
    MhcPreOp,
    MhcPreWeights,
    MhcTensor,
    exported_symbols,
    library_path,
    load_library,
    make_tensor,
    mhc_pre,
    stream_probe,
)


def torch_ops():
    """Register and return the ``torch.ops.mhcpre`` operators (module torch_op)."""
    from . import torch_op

    return torch_op
