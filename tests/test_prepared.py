"""Prepared weights: mhcPrePrepareWeights(Size), mhcPreWeightsVersion /
Destroy and mhcPreGetWorkspaceSizePrepared.

CPU part: the size query and the checks that fail before any device work
(fake, never dereferenced device addresses).  GPU part: on every kernel path,
an executor built from prepared weights gives outputs bit-identical to one
built from phi and gamma (the prepared fragments are the ones each kernel
builds itself) and matches the oracle; preparing again in place with new
weights (a new version) updates an existing executor; x whose n or n*D differs
from the prepared weights is rejected.
"""
from __future__ import annotations

import ctypes
import os
import sys

import numpy as np
import pytest

from helpers import assert_close_f32, assert_hin
from inputs import to_bits

FAKE = 0x100000  # aligned placeholder device address; never dereferenced


@pytest.fixture(scope="module")
def lib(pkg):
    return pkg.load_library()


def code(pkg, name):
    return pkg.binding.STATUS_CODE[name]


def _size(pkg, lib, phi_dims, gamma_dims, n, phi_dtype=0, gamma_dtype=0):
    mk = lambda d, dt: ctypes.byref(pkg.make_tensor(FAKE, dt, d)) if d is not None else None
    out = ctypes.c_uint64(0)
    st = lib.mhcPrePrepareWeightsSize(mk(phi_dims, phi_dtype), mk(gamma_dims, gamma_dtype), n,
                                      ctypes.byref(out))
    return st, int(out.value)


def test_size_query_and_validation(pkg, lib):
    # K * 2M * 2 bytes; phi's element count sets K (its dims are free, as in phase 1).
    assert _size(pkg, lib, [256, 24], [4, 64], 4) == (0, 256 * 48 * 2)
    assert _size(pkg, lib, [24, 256], None, 4) == (0, 256 * 48 * 2)
    assert _size(pkg, lib, [6 * 32, 48], [192], 6) == (0, 192 * 96 * 2)
    assert _size(pkg, lib, [8 * 8192, 80], [8 * 8192], 8) == (0, 65536 * 160 * 2)
    bad = lambda *a, **k: _size(pkg, lib, *a, **k)[0]
    assert bad([256, 24], None, 5) == code(pkg, "MHC_STATUS_UNSUPPORTED_SHAPE")       # n
    assert bad([256, 23], None, 4) == code(pkg, "MHC_STATUS_INVALID_SHAPE")           # K*M
    assert bad([4 * 24, 24], None, 4) == code(pkg, "MHC_STATUS_UNSUPPORTED_SHAPE")    # D % 16
    assert bad([256, 24], [4, 63], 4) == code(pkg, "MHC_STATUS_INVALID_SHAPE")        # gamma
    assert bad([256, 24], None, 4, phi_dtype=27) == code(pkg, "MHC_STATUS_INVALID_DTYPE")
    assert bad([256, 24], [4, 64], 4, gamma_dtype=1) == code(pkg, "MHC_STATUS_INVALID_DTYPE")
    assert lib.mhcPrePrepareWeightsSize(ctypes.byref(pkg.make_tensor(FAKE, 0, [256, 24])), None,
                                        4, None) == code(pkg, "MHC_STATUS_NULL_ARGUMENT")
    assert lib.mhcPrePrepareWeightsSize(None, None, 4, ctypes.byref(ctypes.c_uint64())) == code(
        pkg, "MHC_STATUS_NULL_ARGUMENT")


def test_checks_that_fail_before_device_work(pkg, lib):
    phi = pkg.make_tensor(FAKE, 0, [256, 24])
    w = ctypes.c_void_p(None)

    def prep(buf, nbytes, weights=ctypes.byref(w)):
        return lib.mhcPrePrepareWeights(ctypes.byref(phi), None, 4, ctypes.c_void_p(buf),
                                        ctypes.c_uint64(nbytes), ctypes.c_uint64(1), None, weights)

    assert prep(0, 1 << 20) == code(pkg, "MHC_STATUS_NULL_ARGUMENT")
    assert prep(FAKE, 1000) == code(pkg, "MHC_STATUS_WORKSPACE_TOO_SMALL")
    assert prep(FAKE + 16, 1 << 20) == code(pkg, "MHC_STATUS_MISALIGNED")
    assert prep(FAKE, 1 << 20, weights=None) == code(pkg, "MHC_STATUS_NULL_ARGUMENT")
    assert not w.value
    v = ctypes.c_uint64(0)
    assert lib.mhcPreWeightsVersion(None, ctypes.byref(v)) == code(pkg, "MHC_STATUS_NULL_ARGUMENT")
    assert lib.mhcPreWeightsDestroy(None) == code(pkg, "MHC_STATUS_NULL_ARGUMENT")
    ws, exe = ctypes.c_uint64(0), ctypes.c_void_p(None)
    t = ctypes.byref(pkg.make_tensor(FAKE, 27, [1, 4, 4, 64]))
    assert lib.mhcPreGetWorkspaceSizePrepared(t, None, t, t, ctypes.c_float(1e-6),
                                              ctypes.c_float(1e-6), t, t, t, None,
                                              ctypes.byref(ws), ctypes.byref(exe)) == code(
        pkg, "MHC_STATUS_NULL_ARGUMENT")
    assert not exe.value


# ------------------------------------------------------------------ GPU


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _case(device, T, n, D, bf16, gamma_on, seed):
    import torch

    rng = np.random.default_rng(seed)
    K, M = n * D, n * n + 2 * n
    xf = rng.standard_normal((T, n, D)).astype(np.float32)
    xf[::11] *= 50.0
    x_bits = to_bits(xf, bf16)
    dt = torch.bfloat16 if bf16 else torch.float16
    x = torch.from_numpy(x_bits.view(np.int16)).to(device).view(dt)
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)
    phi = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    alpha = np.asarray([0.3, -0.2, 0.05], dtype=np.float32)
    bias = rng.uniform(-0.5, 0.5, M).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if gamma_on else None
    host = (x_bits, phi, alpha, bias, gamma)
    dev = (x, f(phi), f(alpha), f(bias), f(gamma) if gamma_on else None)
    return host, dev


def _bits(t):
    import torch

    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


def _run(pkg, x, phi, alpha, bias, gamma, weights=None, force=None, rows_b=None, layout=None):
    import torch

    if force:
        os.environ["MHCPRE_FORCE_PATH"] = force
    if rows_b:
        os.environ["MHCPRE_ROWS_B"] = rows_b
    if layout:
        os.environ["MHCPRE_ROWS_PARTIALS"] = layout
    try:
        op = pkg.MhcPreOp(x, None if weights else phi, alpha, bias, None if weights else gamma,
                          h_pre=True, weights=weights)
    finally:
        os.environ.pop("MHCPRE_FORCE_PATH", None)
        os.environ.pop("MHCPRE_ROWS_B", None)
        os.environ.pop("MHCPRE_ROWS_PARTIALS", None)
    op.launch()
    torch.cuda.synchronize()
    assert op.device_status() == 0
    path = op.path
    outs = [t.clone() for t in op.outputs()]
    op.close()
    return path, outs


def _check_oracle(orc, host, outs, bf16):
    x_bits, phi, alpha, bias, gamma = host
    T, n, D = x_bits.shape
    ref = orc.mhc_pre(x_bits, bf16, phi, alpha, bias, gamma)
    h_in, h_post, h_res, h_pre = (t.cpu() for t in outs)
    import torch

    assert_close_f32("hPost", h_post.numpy().reshape(T, n), ref["h_post"])
    assert_close_f32("hRes", h_res.numpy().reshape(T, n, n), ref["h_res"])
    assert_close_f32("hPre", h_pre.numpy().reshape(T, n), ref["h_pre"])
    assert_hin(h_in.view(torch.int16).numpy().view(np.uint16).reshape(T, D), ref["h_in"], x_bits,
               bf16, h_pre.numpy().reshape(T, n), ref["h_pre"], orc, ref=ref)


@pytest.mark.gpu
@pytest.mark.parametrize("T,n,D,bf16,gamma_on,force,path", [
    (300, 4, 512, True, True, "strip", "strip"),  # the plan takes rows here
    (300, 4, 512, False, False, "strip", "strip"),
    (300, 4, 512, True, True, None, "rows"),       # n = 4, T * D <= 3 * 2^17
    (300, 4, 512, True, True, "fused", "fused"),
    (200, 4, 192, True, True, "fused", "fused"),  # the plan takes rows here
    (200, 4, 192, False, True, None, "rows"),     # n = 4 width without a strip slice
    (300, 4, 512, True, True, "split", "split"),
    (77, 6, 48, True, True, None, "split"),
    (77, 6, 256, False, True, None, "rows"),      # n = 6 small-batch GEMM
    (600, 8, 1024, True, True, "rows", "rows"),  # the plan takes split here
    (600, 8, 1024, True, True, None, "split"),
    (300, 6, 2048, False, True, None, "rows"),
    (40, 8, 4096, True, True, None, "rows"),      # small-batch GEMM
    (100, 4, 256, False, False, None, "rows"),    # n = 4 small batch
    (200, 4, 4096, True, True, None, "rows"),     # n = 4 wide small batch
    (100, 8, 2048, False, True, None, "rows"),    # n = 8 wide small batch
    # strip teams at the headline width (28 slices) and the widest (30 by
    # default, 31 forced), both x dtypes, several tiles per team and a ragged
    # last tile
    (1000, 4, 7168, True, True, None, "strip"),
    (1000, 4, 7168, False, True, None, "strip"),
    (1000, 4, 7680, True, True, None, "strip"),      # 30 slices, the widest default team
    (1000, 4, 7936, True, True, None, "strip"),      # 31 slices: teams across XCDs
    (1000, 4, 7936, False, False, None, "strip"),
    (1500, 4, 8192, False, True, None, "strip"),     # 32 slices
    (600, 4, 16384, True, True, None, "strip"),      # 64 slices
    (700, 4, 4160, True, True, "strip", "strip"),    # D % 256 != 0: the last slice one strip wide
    (700, 4, 7104, False, True, "strip", "strip"),   # ... three strips wide
    (700, 4, 7072, True, True, "strip", "strip"),    # ... two and a half strips
    (2048, 4, 7936, True, True, "fused", "fused"),   # the fused kernel (a fallback)
])
def test_prepared_matches_plain(pkg, orc, device, T, n, D, bf16, gamma_on, force, path):
    import torch

    host, (x, phi, alpha, bias, gamma) = _case(device, T, n, D, bf16, gamma_on, seed=T + n + D)
    _say(f"[prepared] T={T} n={n} D={D} bf16={bf16} gamma={gamma_on} force={force}")
    w = pkg.MhcPreWeights(phi, gamma, n, version=7)
    assert w.version == 7
    p_path, p_outs = _run(pkg, x, phi, alpha, bias, gamma, weights=w, force=force)
    path_plain, plain = _run(pkg, x, phi, alpha, bias, gamma, force=force)
    assert p_path == path_plain == path
    for a, b, name in zip(p_outs, plain, ("hIn", "hPost", "hRes", "hPre")):
        assert torch.equal(_bits(a), _bits(b)), name
    _check_oracle(orc, host, p_outs, bf16)
    w.close()


@pytest.mark.gpu
@pytest.mark.parametrize("T,n,D,bf16,gamma_on,force", [
    (600, 8, 1024, True, True, "rows"),
    (300, 6, 2048, False, True, None),
    (1000, 4, 1024, True, True, "rows"),     # n = 4: the half tile of M = 24
    (700, 4, 768, False, False, "rows"),
    (4200, 8, 512, False, False, "rows"),    # 17 row blocks: the plan's prep launch
    (520, 8, 2048, True, True, None),
])
def test_rows_gemm_b_sources_match(pkg, orc, device, T, n, D, bf16, gamma_on, force):
    """The block GEMM's two plain B sources -- built from phi in the GEMM
    (MHCPRE_ROWS_B=phi) or read from fragments a prep launch wrote (=prep) --
    and prepared weights give bit-identical outputs, which match the oracle."""
    import torch

    host, (x, phi, alpha, bias, gamma) = _case(device, T, n, D, bf16, gamma_on, seed=3 * T + D)
    _say(f"[rows B] T={T} n={n} D={D} bf16={bf16} gamma={gamma_on} force={force}")
    outs = {}
    for src in ("phi", "prep"):
        path, outs[src] = _run(pkg, x, phi, alpha, bias, gamma, force=force, rows_b=src)
        assert path == "rows"
    w = pkg.MhcPreWeights(phi, gamma, n)
    path, outs["prepared"] = _run(pkg, x, phi, alpha, bias, gamma, weights=w, force=force)
    assert path == "rows"
    for src in ("prep", "prepared"):
        for a, b, name in zip(outs["phi"], outs[src], ("hIn", "hPost", "hRes", "hPre")):
            assert torch.equal(_bits(a), _bits(b)), (src, name)
    _check_oracle(orc, host, outs["phi"], bf16)
    w.close()


@pytest.mark.gpu
@pytest.mark.parametrize("T,n,D,bf16,gamma_on,force", [
    (100, 4, 256, False, False, None),      # small-batch GEMM, 4 K-ranges
    (40, 8, 4096, True, True, None),        # small-batch GEMM, rows past T in the last block
    (64, 8, 7168, False, False, None),      # 224 K-ranges: the 1024-thread epilogue in 4 parts
    (64, 6, 1024, True, True, None),
    (200, 4, 4096, False, True, None),      # wide small-batch GEMM
    (300, 4, 512, True, True, None),        # block GEMM, B built from phi, the half tile
    (600, 8, 1024, True, True, "rows"),
    (4200, 8, 512, False, False, "rows"),   # 17 row blocks: the prep launch
    (2100, 6, 2048, True, True, None),      # ragged last row block
])
def test_rows_partial_layouts_match(pkg, orc, device, T, n, D, bf16, gamma_on, force):
    """The rows path's partial sums stored K-range-major or row-major
    (MHCPRE_ROWS_PARTIALS=ranges / rows) give bit-identical outputs: the
    layout changes addresses only, not the order of any sum."""
    import torch

    host, (x, phi, alpha, bias, gamma) = _case(device, T, n, D, bf16, gamma_on, seed=5 * T + D + n)
    _say(f"[rows layout] T={T} n={n} D={D} bf16={bf16} gamma={gamma_on} force={force}")
    outs = {}
    for layout in ("ranges", "rows"):
        path, outs[layout] = _run(pkg, x, phi, alpha, bias, gamma, force=force, layout=layout)
        assert path == "rows"
    for a, b, name in zip(outs["ranges"], outs["rows"], ("hIn", "hPost", "hRes", "hPre")):
        assert torch.equal(_bits(a), _bits(b)), name
    _check_oracle(orc, host, outs["rows"], bf16)


@pytest.mark.gpu
@pytest.mark.parametrize("T,n,D,force", [(300, 4, 1024, None), (300, 8, 1024, None),
                                         (300, 4, 1024, "split")])
def test_reprepare_updates_existing_executor(pkg, orc, device, T, n, D, force):
    """Preparing new weights into the same buffer (a new version) changes
    what an existing prepared executor computes, from its next launch on."""
    import torch

    host_a, (x, phi_a, alpha, bias, gamma_a) = _case(device, T, n, D, True, True, seed=11)
    host_b, (_, phi_b, _, _, gamma_b) = _case(device, T, n, D, True, True, seed=12)
    w = pkg.MhcPreWeights(phi_a, gamma_a, n, version=1)
    if force:
        os.environ["MHCPRE_FORCE_PATH"] = force
    try:
        op = pkg.MhcPreOp(x, None, alpha, bias, None, h_pre=True, weights=w)
    finally:
        os.environ.pop("MHCPRE_FORCE_PATH", None)
    _say(f"[prepared] reprepare path={op.path} T={T} n={n} D={D}")
    op.launch()
    torch.cuda.synchronize()
    first = [t.clone() for t in op.outputs()]
    _check_oracle(orc, host_a, first, True)
    w.prepare(phi_b, gamma_b, version=2)
    assert w.version == 2
    op.launch()
    torch.cuda.synchronize()
    second = [t.clone() for t in op.outputs()]
    x_bits = host_a[0]
    _check_oracle(orc, (x_bits,) + host_b[1:2] + host_a[2:4] + host_b[4:], second, True)
    assert not torch.equal(first[1], second[1])
    op.close()
    w.close()


@pytest.mark.gpu
def test_prepared_shape_mismatch_is_rejected(pkg, device):
    import torch

    _, (x, phi, alpha, bias, gamma) = _case(device, 64, 4, 512, True, True, seed=3)
    _, (x2, _, _, _, _) = _case(device, 64, 4, 256, True, True, seed=3)
    w = pkg.MhcPreWeights(phi, gamma, 4)
    with pytest.raises(pkg.MhcPreError) as ei:
        pkg.MhcPreOp(x2, None, alpha, bias, None, weights=w)
    assert ei.value.status == code(pkg, "MHC_STATUS_INVALID_SHAPE")
    w.close()
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_reprepare_with_another_layout_is_refused_while_in_use(pkg, device):
    """A prepared buffer holds the fragments of one (n, K): preparing it again
    with another layout while a weights handle or an executor still reads it
    would make those read fragments in the wrong order, so it fails with
    MHC_STATUS_INVALID_SHAPE; the same layout re-prepares, and once every
    handle and executor on the buffer is gone another layout is accepted."""
    import ctypes

    import torch

    lib = pkg.load_library()
    _, (x, phi, alpha, bias, gamma) = _case(device, 64, 4, 512, True, True, seed=21)
    _, (_, phi_s, _, _, gamma_s) = _case(device, 64, 4, 256, True, True, seed=22)
    w = pkg.MhcPreWeights(phi, gamma, 4)
    op = pkg.MhcPreOp(x, None, alpha, bias, None, weights=w)

    def prepare(phi_t, gamma_t, n):
        handle = ctypes.c_void_p(None)
        pd, gd = pkg.binding.tensor_desc(phi_t), pkg.binding.tensor_desc(gamma_t)
        st = lib.mhcPrePrepareWeights(ctypes.byref(pd), ctypes.byref(gd), ctypes.c_int32(n),
                                      ctypes.c_void_p(w.buffer.data_ptr()),
                                      ctypes.c_uint64(w.bytes), ctypes.c_uint64(7), None,
                                      ctypes.byref(handle))
        return st, handle

    _say("[prepared] re-prepare with another layout")
    st, h = prepare(phi_s, gamma_s, 4)  # K = 1024 into a K = 2048 buffer in use
    assert st == code(pkg, "MHC_STATUS_INVALID_SHAPE") and not h.value
    st, h = prepare(phi, gamma, 4)  # the same layout: fine
    assert st == 0 and h.value
    lib.mhcPreWeightsDestroy(h)
    w.close()  # the executor still reads the buffer
    st, h = prepare(phi_s, gamma_s, 4)
    assert st == code(pkg, "MHC_STATUS_INVALID_SHAPE") and not h.value
    op.close()
    torch.cuda.synchronize()
    st, h = prepare(phi_s, gamma_s, 4)  # nothing reads the buffer any more
    assert st == 0 and h.value
    lib.mhcPreWeightsDestroy(h)
    torch.cuda.synchronize()
