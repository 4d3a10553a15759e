"""Host-side C ABI behaviour without a GPU: exports, validation, workspace sizing.

Validation mirrors the reference TilingFunc (code/op_host/mhc_pre.cpp:57-79,
126-130) and InferShape (:217-249); phase 1 never touches device memory, so
fake (aligned) device addresses are enough here.
"""
from __future__ import annotations

import ctypes
import threading

import pytest

FAKE = 0x100000  # aligned placeholder device address; never dereferenced on the host


@pytest.fixture(scope="module")
def lib(pkg):
    return pkg.load_library()


def _descs(pkg, B=1, S=4, n=4, D=64, xdt=None, gamma=True, **over):
    f32, xdt = pkg.MHC_DTYPE_FLOAT, (pkg.MHC_DTYPE_BF16 if xdt is None else xdt)
    K, M = n * D, n * n + 2 * n
    d = {
        "x": (FAKE, xdt, [B, S, n, D]),
        "phi": (FAKE, f32, [K, M]),
        "alpha": (FAKE, f32, [3]),
        "bias": (FAKE, f32, [M]),
        "gamma": (FAKE, f32, [n, D]) if gamma else None,
        "hIn": (FAKE, xdt, [B, S, D]),
        "hPost": (FAKE, f32, [B, S, n]),
        "hRes": (FAKE, f32, [B, S, n, n]),
    }
    d.update(over)
    return d


def _call(pkg, lib, d, norm_eps=1e-6, hc_eps=1e-6, h_pre=None):
    mk = lambda v: None if v is None else ctypes.byref(pkg.make_tensor(*v))
    ws = ctypes.c_uint64(0)
    exe = ctypes.c_void_p(None)
    args = [mk(d["x"]), mk(d["phi"]), mk(d["alpha"]), mk(d["bias"]), mk(d["gamma"]),
            ctypes.c_float(norm_eps), ctypes.c_float(hc_eps), mk(d["hIn"]), mk(d["hPost"]),
            mk(d["hRes"])]
    if h_pre is not None:
        st = lib.mhcPreGetWorkspaceSizeWithHPre(*args, mk(h_pre), ctypes.byref(ws),
                                                ctypes.byref(exe))
    else:
        st = lib.mhcPreGetWorkspaceSize(*args, ctypes.byref(ws), ctypes.byref(exe))
    if exe.value:
        lib.mhcPreExecutorDestroy(exe)
    return st, int(ws.value)


def code(pkg, name):
    return pkg.binding.STATUS_CODE[name]


def test_library_exports_every_declared_symbol(pkg, lib):
    names = pkg.exported_symbols()
    assert set(names) >= {"mhcPreGetWorkspaceSize", "mhcPre", "mhcPreExecutorDestroy"}
    for name in names:
        assert hasattr(lib, name), name


def test_valid_call_sizes_workspace(pkg, lib):
    st, ws = _call(pkg, lib, _descs(pkg))
    assert st == 0 and ws > 0
    # 3-D x [T, n, D] extension with matching 2-D/3-D outputs.
    n, D, T = 4, 64, 4
    d = _descs(pkg, x=(FAKE, pkg.MHC_DTYPE_BF16, [T, n, D]),
               hIn=(FAKE, pkg.MHC_DTYPE_BF16, [T, D]),
               hPost=(FAKE, pkg.MHC_DTYPE_FLOAT, [T, n]),
               hRes=(FAKE, pkg.MHC_DTYPE_FLOAT, [T, n, n]))
    assert _call(pkg, lib, d) == (st, ws)


def test_workspace_grows_with_shape_on_the_two_pass_paths(pkg, lib):
    # n = 8, D = 4096 takes the rows path: its partial sums grow with T.
    _, small = _call(pkg, lib, _descs(pkg, S=512, n=8, D=4096))
    _, big = _call(pkg, lib, _descs(pkg, S=65536, n=8, D=4096))
    assert _path(pkg, lib, _descs(pkg, S=512, n=8, D=4096)) == "rows"
    assert _path(pkg, lib, _descs(pkg, S=65536, n=8, D=4096)) == "rows"
    assert big > small > 0


def _strip_workspace(pkg, teams, P):
    """The strip layout on the planned device (MI355X's shape here, no GPU is
    visible: 8 XCDs of 32 CUs): the workspace header, then per team a ring
    of 10 broadcast blocks of 4 x 16 tagged words, then per team 10 slots of
    P records of 25 x 16 tagged words (8 bytes each), 256-byte aligned."""
    header = 256 + 4 * 2048
    up = lambda v: (v + 255) // 256 * 256
    ring = teams * 10
    recs = up(header + ring * 64 * 8)
    return up(recs + ring * P * 400 * 8)


@pytest.mark.parametrize("B,S,D,teams", [
    (1, 8192, 7168, 8),     # the headline prefill shape: one team of 28 slices per XCD
    (4, 32768, 7168, 8),    # 131072 rows, the reference's largest T: the same rings
    (1, 8192, 7680, 8),     # 30 slices, the widest strip team with two reducers
    (1, 131072, 1024, 40),  # 4 slices and 2 reducers: 5 teams per XCD
])
def test_strip_workspace_does_not_grow_with_rows(pkg, lib, B, S, D, teams):
    """The strip path keeps its exchange in per-team rings: the workspace is
    the rings of the teams the device holds, whatever T (the fused layout,
    per row tile, is 46 MB at the headline and 739 MB at 131072 rows)."""
    d = _descs(pkg, B=B, S=S, D=D)
    assert _path(pkg, lib, d) == "strip"
    st, ws = _call(pkg, lib, d)
    assert st == 0
    assert ws == _strip_workspace(pkg, teams, D // 256)
    assert ws <= 10 << 20
    if (B, S) == (4, 32768):
        _, head = _call(pkg, lib, _descs(pkg, B=1, S=8192, D=D))
        assert ws == head


@pytest.mark.parametrize("D,teams", [
    (2048, 24),   # 8 slices: 3 teams per XCD with 2 reducers (across: 21 teams)
    (2304, 19),   # 9 slices: across XCDs, 19 teams of 4 reducers (in an XCD: 16)
    (2560, 16),   # 10 slices: 2 teams per XCD (across: 18, less than 15% more)
    (4096, 12),   # 16 slices: across XCDs (in an XCD: 8)
    (5120, 10),   # 20 slices: across XCDs (in an XCD: 8)
    (3840, 13),   # 15 slices: across XCDs (in an XCD: 8)
    (5376, 10),   # 21 slices: across XCDs (in an XCD: 8)
    (5632, 8),    # 22 slices: in an XCD (across: 9)
    (7168, 8),    # 28 slices: in an XCD, 4 reducers (across: 8)
    (7680, 8),    # 30 slices: in an XCD, 2 reducers
    (7936, 7),    # 31 slices: across XCDs only
    (16384, 3),   # 64 slices
])
def test_strip_team_geometry(pkg, lib, D, teams):
    """Where the strip kernel's teams live: inside an XCD unless teams across
    XCDs (four reducers each) put at least 15% more CUs on slices, or two
    reducers do not fit an XCD.  The team count shows in the ring workspace."""
    d = _descs(pkg, S=8192, D=D)
    assert _path(pkg, lib, d) == "strip"
    st, ws = _call(pkg, lib, d)
    assert st == 0
    assert ws == _strip_workspace(pkg, teams, D // 256)


@pytest.mark.parametrize("over,want", [
    ({"x": (FAKE, 27, [4, 4, 64])}, "MHC_STATUS_SUCCESS"),  # 3-D is accepted
    ({"x": (FAKE, 27, [1, 1, 4, 4, 64])}, "MHC_STATUS_INVALID_SHAPE"),
    ({"x": (FAKE, 27, [4, 64])}, "MHC_STATUS_INVALID_SHAPE"),
    ({"x": (FAKE, 27, [0, 4, 4, 64])}, "MHC_STATUS_INVALID_SHAPE"),
    ({"x": (FAKE, 27, [1, 4, 4, 0])}, "MHC_STATUS_INVALID_SHAPE"),
    ({"x": (FAKE, 27, [1, 4, 5, 64])}, "MHC_STATUS_UNSUPPORTED_SHAPE"),
    ({"x": (FAKE, 27, [1, 4, 2, 64])}, "MHC_STATUS_UNSUPPORTED_SHAPE"),
    ({"x": (FAKE, 27, [1, 4, 4, 24])}, "MHC_STATUS_UNSUPPORTED_SHAPE"),
    ({"x": (FAKE, 0, [1, 4, 4, 64])}, "MHC_STATUS_INVALID_DTYPE"),
    ({"hIn": (FAKE, 1, [1, 4, 64])}, "MHC_STATUS_INVALID_DTYPE"),
    ({"phi": (FAKE, 27, [256, 24])}, "MHC_STATUS_INVALID_DTYPE"),
    ({"phi": (FAKE, 0, [256, 23])}, "MHC_STATUS_INVALID_SHAPE"),
    ({"phi": (FAKE, 0, [24, 256])}, "MHC_STATUS_SUCCESS"),  # only the element count matters
    ({"alpha": (FAKE, 0, [2])}, "MHC_STATUS_INVALID_SHAPE"),
    ({"bias": (FAKE, 0, [25])}, "MHC_STATUS_INVALID_SHAPE"),
    ({"gamma": (FAKE, 0, [4, 63])}, "MHC_STATUS_INVALID_SHAPE"),
    ({"gamma": (0, 0, [0])}, "MHC_STATUS_SUCCESS"),  # size 0 => gamma off (mhc_pre.cpp:90)
    ({"gamma": None}, "MHC_STATUS_SUCCESS"),
    ({"hIn": (FAKE, 27, [1, 4, 65])}, "MHC_STATUS_INVALID_SHAPE"),
    ({"hPost": (FAKE, 0, [1, 4, 5])}, "MHC_STATUS_INVALID_SHAPE"),
    ({"hRes": (FAKE, 0, [1, 4, 16])}, "MHC_STATUS_INVALID_SHAPE"),
    ({"hRes": (FAKE, 0, [1, 4, 4, 4])}, "MHC_STATUS_SUCCESS"),
    ({"x": (0, 27, [1, 4, 4, 64])}, "MHC_STATUS_NULL_ARGUMENT"),
    ({"hPost": (0, 0, [1, 4, 4])}, "MHC_STATUS_NULL_ARGUMENT"),
    ({"x": (FAKE + 2, 27, [1, 4, 4, 64])}, "MHC_STATUS_MISALIGNED"),
    ({"phi": (FAKE + 4, 0, [256, 24])}, "MHC_STATUS_MISALIGNED"),
    ({"bias": (FAKE + 2, 0, [24])}, "MHC_STATUS_MISALIGNED"),
])
def test_validation_status_codes(pkg, lib, over, want):
    d = _descs(pkg)
    d.update(over)
    st, _ = _call(pkg, lib, d)
    assert st == code(pkg, want), (over, st)


def test_size_limits_and_overflowing_dims(pkg, lib):
    """Row counts from 2^28 and widths above 2^24 are unsupported (the split
    GEMM's grid and 64-bit byte offsets); dims whose products overflow are
    rejected, not wrapped."""
    ok = _descs(pkg, B=(1 << 28) - 1, S=1, n=4, D=16)
    assert _call(pkg, lib, ok)[0] == code(pkg, "MHC_STATUS_SUCCESS")
    ok8 = _descs(pkg, B=(1 << 28) - 1, S=1, n=8, D=16)
    assert _call(pkg, lib, ok8)[0] == code(pkg, "MHC_STATUS_SUCCESS")
    big = _descs(pkg, B=1 << 27, S=2, n=4, D=16)
    assert _call(pkg, lib, big)[0] == code(pkg, "MHC_STATUS_UNSUPPORTED_SHAPE")
    wrap = _descs(pkg, B=1 << 62, S=4, n=4, D=16)
    assert _call(pkg, lib, wrap)[0] == code(pkg, "MHC_STATUS_UNSUPPORTED_SHAPE")
    wide = _descs(pkg, B=1, S=1, n=4, D=(1 << 24) + 16)
    assert _call(pkg, lib, wide)[0] == code(pkg, "MHC_STATUS_UNSUPPORTED_SHAPE")
    # A phi whose element count wraps modulo 2^64 onto K*M = 6144 exactly.
    d = _descs(pkg)
    d["phi"] = (FAKE, pkg.MHC_DTYPE_FLOAT, [4, (1 << 62) + 1536])
    assert _call(pkg, lib, d)[0] == code(pkg, "MHC_STATUS_INVALID_SHAPE")


def test_null_descriptors_and_outputs(pkg, lib):
    mk = lambda v: ctypes.byref(pkg.make_tensor(*v))
    d = _descs(pkg)
    ws = ctypes.c_uint64(0)
    exe = ctypes.c_void_p(None)
    st = lib.mhcPreGetWorkspaceSize(None, mk(d["phi"]), mk(d["alpha"]), mk(d["bias"]), None,
                                    ctypes.c_float(1e-6), ctypes.c_float(1e-6), mk(d["hIn"]),
                                    mk(d["hPost"]), mk(d["hRes"]), ctypes.byref(ws),
                                    ctypes.byref(exe))
    assert st == 1
    st = lib.mhcPreGetWorkspaceSize(mk(d["x"]), mk(d["phi"]), mk(d["alpha"]), mk(d["bias"]),
                                    None, ctypes.c_float(1e-6), ctypes.c_float(1e-6),
                                    mk(d["hIn"]), mk(d["hPost"]), mk(d["hRes"]), None,
                                    ctypes.byref(exe))
    assert st == 1


def test_hpre_extension_validation(pkg, lib):
    d = _descs(pkg)
    assert _call(pkg, lib, d, h_pre=(FAKE, 0, [1, 4, 4]))[0] == 0
    assert _call(pkg, lib, d, h_pre=(FAKE, 0, [1, 4, 5]))[0] == 2
    assert _call(pkg, lib, d, h_pre=(FAKE, 27, [1, 4, 4]))[0] == 4


def test_launch_rejects_bad_workspace_before_any_device_work(pkg, lib):
    mk = lambda v: ctypes.byref(pkg.make_tensor(*v))
    d = _descs(pkg)
    ws = ctypes.c_uint64(0)
    exe = ctypes.c_void_p(None)
    st = lib.mhcPreGetWorkspaceSize(mk(d["x"]), mk(d["phi"]), mk(d["alpha"]), mk(d["bias"]),
                                    mk(d["gamma"]), ctypes.c_float(1e-6), ctypes.c_float(1e-6),
                                    mk(d["hIn"]), mk(d["hPost"]), mk(d["hRes"]),
                                    ctypes.byref(ws), ctypes.byref(exe))
    assert st == 0
    assert lib.mhcPre(None, ws, exe, None) == 5
    assert lib.mhcPre(ctypes.c_void_p(FAKE), ctypes.c_uint64(ws.value - 1), exe, None) == 5
    assert lib.mhcPre(ctypes.c_void_p(FAKE + 16), ws, exe, None) == 5  # not 256-aligned
    assert lib.mhcPre(ctypes.c_void_p(FAKE), ws, None, None) == 1
    name = ctypes.c_char_p()
    assert lib.mhcPreExecutorPath(exe, ctypes.byref(name)) == 0
    assert name.value in (b"split", b"fused", b"strip", b"rows")
    assert lib.mhcPreExecutorDestroy(exe) == 0
    assert lib.mhcPreExecutorDestroy(None) == 1


def test_status_strings(lib):
    assert lib.mhcPreStatusString(0) == b"success"
    assert lib.mhcPreStatusString(5) == b"workspace too small"
    assert lib.mhcPreStatusString(12345) == b"unknown status"


def test_phase1_is_thread_safe(pkg, lib):
    """Concurrent phase-1 calls with different shapes each get their own answer
    (the reference's tiling cache is an unlocked global, mhc_pre.cpp:51)."""
    shapes = [(1, S, n, D) for S in (3, 17, 64) for n in (4, 6, 8) for D in (16, 64, 256)]
    expected = {s: _call(pkg, lib, _descs(pkg, *s)) for s in shapes}
    errors = []

    def worker(seed):
        for i in range(40):
            s = shapes[(seed * 7 + i) % len(shapes)]
            got = _call(pkg, lib, _descs(pkg, *s))
            if got != expected[s]:
                errors.append((s, got, expected[s]))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors


def _path(pkg, lib, d, env=None):
    import os

    mk = lambda v: None if v is None else ctypes.byref(pkg.make_tensor(*v))
    ws = ctypes.c_uint64(0)
    exe = ctypes.c_void_p(None)
    if env is not None:
        os.environ["MHCPRE_FORCE_PATH"] = env
    try:
        st = lib.mhcPreGetWorkspaceSize(mk(d["x"]), mk(d["phi"]), mk(d["alpha"]), mk(d["bias"]),
                                        mk(d["gamma"]), ctypes.c_float(1e-6), ctypes.c_float(1e-6),
                                        mk(d["hIn"]), mk(d["hPost"]), mk(d["hRes"]),
                                        ctypes.byref(ws), ctypes.byref(exe))
    finally:
        os.environ.pop("MHCPRE_FORCE_PATH", None)
    assert st == 0
    name = ctypes.c_char_p()
    assert lib.mhcPreExecutorPath(exe, ctypes.byref(name)) == 0
    lib.mhcPreExecutorDestroy(exe)
    return name.value.decode()


@pytest.mark.parametrize("n,D,S,want", [
    (4, 7168, 4096, "strip"),  # 28 slices of 256 columns, one team per XCD
    (4, 7680, 8192, "strip"),  # 30 slices and 2 reducers per XCD
    (4, 7936, 8192, "strip"),  # 31 or more slices: teams across XCDs
    (4, 7936, 1025, "strip"),
    (4, 8192, 8192, "strip"),
    (4, 8192, 512, "strip"),
    (4, 8192, 256, "rows"),    # small batches stay on the rows path
    (4, 12288, 8192, "strip"),
    (4, 16384, 4096, "strip"), # 64 slices, the widest team
    (4, 16640, 4096, "rows"),  # 65 slices: rows
    (4, 64, 4096, "split"),    # n = 4, not a strip width: split for K <= 8704 from T = 2048
    (4, 64, 2047, "rows"),
    (4, 2176, 2048, "strip"),  # D % 64 == 0: strip, the last slice two strips wide
    (4, 192, 8192, "strip"),   # one slice, three strips
    (4, 128, 8192, "split"),   # one slice of two strips: not a strip width
    (4, 2240, 2048, "strip"),
    (4, 2272, 2048, "strip"),  # D % 64 == 32: strip, the last strip half live
    (4, 2256, 2048, "split"),  # D % 32 != 0: K % 128 != 0, split
    (4, 7104, 8192, "strip"),
    (4, 7072, 8192, "strip"),
    (4, 7056, 8192, "split"),  # D % 32 != 0
    (4, 48, 64, "split"),      # n = 4, D % 64 != 0
    (4, 5120, 128, "rows"),    # small n = 4 batch: T <= 128 at every width
    (4, 256, 128, "rows"),
    (4, 7168, 128, "rows"),
    (4, 7168, 64, "rows"),
    (4, 5632, 1, "rows"),
    (4, 4096, 160, "rows"),    # T <= 160 up to D = 6144
    (4, 6144, 160, "rows"),
    (4, 7168, 129, "rows"),    # T <= 256 on the wide small-batch GEMM while T * D <= 9 * 2^17
    (4, 7168, 192, "strip"),
    (4, 7168, 256, "strip"),
    (4, 4096, 256, "rows"),
    (4, 5120, 224, "rows"),
    (4, 5120, 256, "strip"),
    (4, 6144, 192, "rows"),
    (4, 6144, 224, "strip"),
    (4, 7936, 256, "rows"),    # ... or at 31 or more slices
    (4, 16384, 256, "rows"),
    (4, 16384, 257, "strip"),
    (4, 7168, 257, "strip"),
    (4, 3584, 161, "strip"),   # T <= 256 below D = 4096: rows while T * D <= 2^19
    (4, 2048, 256, "rows"),
    (4, 3072, 192, "strip"),
    (4, 2048, 257, "strip"),   # T <= 1024: rows while T * D <= 3 * 2^17
    (4, 768, 512, "rows"),
    (4, 1024, 512, "strip"),
    (4, 256, 1024, "rows"),
    (4, 256, 1025, "strip"),
    (4, 256, 4095, "strip"),
    (4, 256, 4096, "strip"),   # one slice per team: strip at every longer batch
    (4, 256, 32768, "strip"),
    (4, 512, 8192, "strip"),
    (4, 512, 1024, "strip"),
    (4, 5696, 64, "rows"),     # not a strip width: rows, not fused
    (8, 7168, 64, "rows"),     # n = 8, K % 128 == 0
    (8, 8192, 5472, "rows"),
    (6, 1024, 16, "rows"),     # K = 6144
    (6, 1024, 2048, "split"),  # K <= 9216 from T = 1024
    (6, 1024, 1024, "split"),
    (6, 1024, 8192, "split"),
    (6, 512, 4096, "split"),
    (6, 1536, 1024, "split"),  # K = 9216
    (6, 1024, 512, "rows"),
    (8, 1024, 1024, "split"),
    (8, 1024, 4096, "split"),
    (8, 1024, 512, "split"),   # n = 8, K <= 8192: from T = 512
    (8, 1024, 511, "rows"),
    (8, 1024, 256, "rows"),
    (8, 1024, 2049, "split"),
    (6, 2048, 512, "rows"),    # K = 12288: rows at every T
    (6, 2048, 1024, "rows"),
    (6, 2048, 8192, "rows"),
    (8, 1536, 1024, "rows"),
    (8, 1536, 512, "rows"),
    (8, 2048, 1024, "rows"),   # K = 16384
    (6, 48, 16, "split"),      # K = 288: not a multiple of 128
    (8, 16, 16, "rows"),       # K = 128
])
def test_path_selection(pkg, lib, n, D, S, want):
    assert _path(pkg, lib, _descs(pkg, S=S, n=n, D=D)) == want


def test_forced_paths(pkg, lib):
    d = _descs(pkg, S=64, n=8, D=1024)
    assert _path(pkg, lib, d, env="split") == "split"
    assert _path(pkg, lib, d, env="rows") == "rows"
    assert _path(pkg, lib, _descs(pkg, S=64, n=4, D=7168), env="strip") == "strip"
    # A path the shape cannot take is ignored.
    assert _path(pkg, lib, _descs(pkg, S=16, n=6, D=48), env="rows") == "split"


def test_no_alloc_rejects_workspaces_beyond_the_builtin_scratch(pkg, lib):
    """mhcPreNoAlloc checks the executor's workspace size against its 64 MiB
    built-in array before any HIP call: a plan that needs more (the rows
    path's partial sums of 131072 rows at n=8, D=16384) is rejected with
    MHC_STATUS_SCRATCH_TOO_SMALL, and a NULL executor with
    MHC_STATUS_NULL_ARGUMENT."""
    T, n, D = 131072, 8, 16384
    d = _descs(pkg, B=1, S=T, n=n, D=D)
    mk = lambda v: None if v is None else ctypes.byref(pkg.make_tensor(*v))
    ws, exe = ctypes.c_uint64(0), ctypes.c_void_p(None)
    st = lib.mhcPreGetWorkspaceSize(mk(d["x"]), mk(d["phi"]), mk(d["alpha"]), mk(d["bias"]),
                                    mk(d["gamma"]), ctypes.c_float(1e-6), ctypes.c_float(1e-6),
                                    mk(d["hIn"]), mk(d["hPost"]), mk(d["hRes"]),
                                    ctypes.byref(ws), ctypes.byref(exe))
    assert st == 0 and ws.value > 64 << 20
    try:
        assert lib.mhcPreNoAlloc(exe, None) == code(pkg, "MHC_STATUS_SCRATCH_TOO_SMALL")
    finally:
        lib.mhcPreExecutorDestroy(exe)
    assert lib.mhcPreNoAlloc(None, None) == code(pkg, "MHC_STATUS_NULL_ARGUMENT")
    assert lib.mhcPreStatusString(code(pkg, "MHC_STATUS_SCRATCH_TOO_SMALL")) != b"unknown status"


def test_stream_probe_rejects_bad_arguments_before_any_launch(pkg, lib):
    """mhcPreStreamProbe (a measurement aid) validates before it touches the
    device: NULL buffers with nonzero sizes, sizes off the block granularity,
    misaligned buffers and out-of-range grids are refused, and an empty
    request succeeds without a launch."""
    probe = lib.mhcPreStreamProbe
    vp = ctypes.c_void_p
    assert probe(None, 4096, vp(FAKE), 1024, 0, None) == code(pkg, "MHC_STATUS_NULL_ARGUMENT")
    assert probe(vp(FAKE), 4096, None, 1024, 0, None) == code(pkg, "MHC_STATUS_NULL_ARGUMENT")
    assert probe(vp(FAKE), 4000, vp(FAKE), 1024, 0, None) == code(pkg, "MHC_STATUS_INVALID_SHAPE")
    assert probe(vp(FAKE), 4096, vp(FAKE), 1000, 0, None) == code(pkg, "MHC_STATUS_INVALID_SHAPE")
    assert probe(vp(FAKE), 4096, vp(FAKE), 1024, -1, None) == code(pkg, "MHC_STATUS_INVALID_SHAPE")
    assert probe(vp(FAKE), 4096, vp(FAKE), 1024, 70000, None) == code(pkg, "MHC_STATUS_INVALID_SHAPE")
    assert probe(vp(FAKE + 4), 4096, vp(FAKE), 1024, 0, None) == code(pkg, "MHC_STATUS_MISALIGNED")
    assert probe(None, 0, None, 0, 0, None) == code(pkg, "MHC_STATUS_SUCCESS")
