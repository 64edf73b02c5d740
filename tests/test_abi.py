"""The C-ABI library loads on the host and exports every entry point include/cufk_hip.h
declares; status paths that return before any device work behave as documented.  No kernel
is launched here."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "cufk_hip.h"
LIB = ROOT / "cufk_amd" / "libcufk_hip.so"

OK, ERR_DTYPE, ERR_POINTS, ERR_SHAPE, ERR_STEPS, ERR_NULL, ERR_STRIDE = 0, 1, 2, 3, 4, 5, 6


@pytest.fixture(scope="module")
def lib():
    lib = ctypes.CDLL(str(LIB))
    i64, vp = ctypes.c_int64, ctypes.c_void_p
    lib.cufk_reconstruct_fwd.argtypes = [ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, i64, i64, vp]
    lib.cufk_reconstruct_bwd.argtypes = [ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, vp]
    lib.cufk_reconstruct_fwd_flagged.argtypes = [ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, vp]
    lib.cufk_reconstruct_bwd_saved.argtypes = [ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, vp]
    lib.cufk_torsion_fwd.argtypes = [ctypes.c_int, vp, i64, vp, vp, i64, i64, vp]
    lib.cufk_torsion_bwd.argtypes = [ctypes.c_int, vp, i64, vp, vp, vp, i64, vp, i64, i64, vp]
    lib.cufk_reconstruct_bwd_anchored.argtypes = [ctypes.c_int] + [vp] * 16 + [i64, i64, vp]
    lib.cufk_reconstruct_bwd_anchored_noalloc.argtypes = [ctypes.c_int] + [vp] * 15 + [i64, i64, vp]
    lib.cufk_reconstruct_superposed_fwd.argtypes = [ctypes.c_int, ctypes.c_int] + [vp] * 11 + [i64, i64, vp]
    lib.cufk_reconstruct_superposed_bwd.argtypes = [ctypes.c_int, ctypes.c_int] + [vp] * 14 + [i64, i64, vp]
    lib.cufk_torsion_loss_fwd.argtypes = [ctypes.c_int, ctypes.c_int, vp, i64, vp, vp, vp, vp, vp, i64, i64, vp]
    lib.cufk_torsion_loss_bwd.argtypes = [ctypes.c_int, ctypes.c_int, vp, i64, vp, vp, vp, vp, vp, i64, vp, i64, i64, vp]
    lib.cufk_reconstruct_loss_fwd.argtypes = [ctypes.c_int] + [vp] * 10 + [i64, i64, vp]
    lib.cufk_reconstruct_loss_bwd.argtypes = [ctypes.c_int] + [vp] * 13 + [i64, i64, vp]
    lib.cufk_reconstruct_long_fwd.argtypes = [ctypes.c_int] + [vp] * 8 + [i64, i64, i64, vp]
    lib.cufk_reconstruct_long_bwd.argtypes = [ctypes.c_int] + [vp] * 13 + [i64, i64, i64, vp]
    for name in ("cufk_long_state_doubles", "cufk_long_work_doubles"):
        getattr(lib, name).argtypes = [i64, i64, i64]
        getattr(lib, name).restype = i64
    lib.cufk_reconstruct_shadow_floats.argtypes = [i64, i64]
    lib.cufk_reconstruct_shadow_floats.restype = i64
    lib.cufk_reconstruct_fwd_shadow.argtypes = [ctypes.c_int] + [vp] * 9 + [i64, i64, vp]
    lib.cufk_reconstruct_bwd_shadow.argtypes = [ctypes.c_int] + [vp] * 12 + [i64, i64, vp]
    lib.cufk_long_segment_steps.argtypes = [i64, i64]
    lib.cufk_long_segment_steps.restype = i64
    lib.cufk_error_string.restype = ctypes.c_char_p
    lib.cufk_version.restype = ctypes.c_char_p
    return lib


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(cufk_\w+)\s*\(", text, re.M)))


def test_header_declares_the_entry_points():
    assert declared_functions() == [
        "cufk_error_string",
        "cufk_long_segment_steps",
        "cufk_long_state_doubles",
        "cufk_long_work_doubles",
        "cufk_max_steps",
        "cufk_reconstruct_bwd",
        "cufk_reconstruct_bwd_anchored",
        "cufk_reconstruct_bwd_anchored_noalloc",
        "cufk_reconstruct_bwd_saved",
        "cufk_reconstruct_bwd_shadow",
        "cufk_reconstruct_fwd",
        "cufk_reconstruct_fwd_flagged",
        "cufk_reconstruct_fwd_shadow",
        "cufk_reconstruct_long_bwd",
        "cufk_reconstruct_long_bwd_anchored",
        "cufk_reconstruct_long_fwd",
        "cufk_reconstruct_loss_bwd",
        "cufk_reconstruct_loss_bwd_anchored",
        "cufk_reconstruct_loss_fwd",
        "cufk_reconstruct_shadow_floats",
        "cufk_reconstruct_superposed_bwd",
        "cufk_reconstruct_superposed_fwd",
        "cufk_torsion_bwd",
        "cufk_torsion_fwd",
        "cufk_torsion_loss_bwd",
        "cufk_torsion_loss_fwd",
        "cufk_version",
    ]


def test_every_declared_symbol_is_exported(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_status_strings(lib):
    assert lib.cufk_error_string(OK) == b"success"
    assert lib.cufk_error_string(ERR_POINTS) == b"point_count must be >= 4"
    assert lib.cufk_error_string(ERR_SHAPE) == b"shape exceeds int32 kernel limits"
    assert lib.cufk_error_string(ERR_DTYPE) == b"unsupported dtype"
    assert lib.cufk_error_string(999) == b"unknown status"
    assert lib.cufk_version() == b"0.1.0"


ERR_DEVICE, ERR_DIRECTION = 8, 12


def test_max_steps(lib):
    # Argument checks come before the device query; no device index below 0 or past the
    # present devices is supported (this host may have no GPU at all: then none is).
    assert lib.cufk_max_steps(9, 0, 0) == -ERR_DTYPE
    assert lib.cufk_max_steps(0, 2, 0) == -ERR_DIRECTION
    assert lib.cufk_max_steps(0, -1, 0) == -ERR_DIRECTION
    for dtype in range(4):
        for direction in range(2):
            assert lib.cufk_max_steps(dtype, direction, -1) == -ERR_DEVICE
            assert lib.cufk_max_steps(dtype, direction, 4096) == -ERR_DEVICE
            assert lib.cufk_max_steps(dtype, direction, 0) in (2048, -ERR_DEVICE)
    assert lib.cufk_error_string(ERR_DIRECTION) == b"direction must be CUFK_FORWARD or CUFK_BACKWARD"
    assert lib.cufk_error_string(ERR_DEVICE) == b"device query failed"


def test_reconstruct_status_paths(lib):
    p = ctypes.c_void_p(1)  # never dereferenced: every call below returns before device work
    null = None
    f = lib.cufk_reconstruct_fwd
    assert f(9, p, p, p, p, p, p, p, 4, 10, null) == ERR_DTYPE
    assert f(0, p, p, p, p, p, p, p, 4, 3, null) == ERR_POINTS
    assert f(0, p, p, p, p, p, p, p, 4, 2052, null) == ERR_STEPS
    assert f(0, p, p, p, p, p, p, p, -1, 10, null) == ERR_SHAPE
    assert f(0, p, p, p, p, p, p, p, 2**31, 10, null) == ERR_SHAPE
    assert f(0, p, p, p, p, p, p, p, 0, 10, null) == OK  # empty batch: nothing to launch
    assert f(0, null, p, p, p, p, p, p, 4, 10, null) == ERR_NULL
    b = lib.cufk_reconstruct_bwd
    assert b(0, p, p, p, p, p, p, p, p, p, p, 4, 2052, null) == ERR_STEPS
    assert b(0, p, p, p, p, p, p, p, null, p, p, 4, 10, null) == ERR_NULL
    assert b(0, p, p, p, p, p, p, p, p, p, p, 0, 10, null) == OK
    ff = lib.cufk_reconstruct_fwd_flagged
    assert ff(9, p, p, p, p, p, p, p, p, 4, 10, null) == ERR_DTYPE
    assert ff(0, p, p, p, p, p, p, p, null, 0, 10, null) == OK
    assert ff(0, p, p, p, p, p, p, null, p, 4, 10, null) == ERR_NULL
    bs = lib.cufk_reconstruct_bwd_saved
    assert bs(0, p, p, p, p, p, p, p, null, p, p, p, p, 4, 10, null) == ERR_NULL  # flags are required
    assert bs(0, p, p, p, p, p, p, p, p, p, p, p, p, 4, 3, null) == ERR_POINTS
    assert bs(0, p, p, p, p, p, p, p, p, p, p, p, p, 0, 10, null) == OK


def test_shadow_sizes_and_status_paths(lib):
    n = lib.cufk_reconstruct_shadow_floats
    assert n(16384, 1026) == 16384 * 1026 * 3
    assert n(4095, 100) == 4095 * 100 * 3  # below the packed batch: one chain per workgroup
    assert n(4096, 131) == 0 and n(131072, 64) == 0  # packed forward: the backward recomputes
    assert n(4096, 132) == 4096 * 132 * 3
    assert n(0, 10) == 0
    assert n(4, 3) == -1 and n(4, 2052) == -1 and n(-1, 10) == -1
    p = ctypes.c_void_p(1)
    null = None
    f = lib.cufk_reconstruct_fwd_shadow
    #        dtype L  A  D  p0 d0 n0 xyz pos flags
    for dtype in (0, 1, 9):  # float32 and float64 keep their own output
        assert f(dtype, p, p, p, p, p, p, p, p, p, 4, 10, null) == ERR_DTYPE
    assert f(3, p, p, p, p, p, p, p, p, p, 4, 2052, null) == ERR_STEPS
    assert f(3, p, p, p, p, p, p, p, null, p, 4, 10, null) == ERR_NULL  # positions are written
    assert f(2, p, p, p, p, p, p, p, p, null, 4, 10, null) == ERR_NULL  # and flags
    assert f(3, p, p, p, p, p, p, null, p, p, 4, 10, null) == ERR_NULL
    assert f(3, p, p, p, p, p, p, p, null, null, 0, 10, null) == OK
    b = lib.cufk_reconstruct_bwd_shadow
    #        dtype L  A  D  p0 d0 n0 pos flags g  gL gA gD
    assert b(0, p, p, p, p, p, p, p, p, p, p, p, p, 4, 10, null) == ERR_DTYPE
    assert b(2, p, p, p, p, p, p, null, p, p, p, p, p, 4, 10, null) == ERR_NULL
    assert b(2, p, p, p, p, p, p, p, p, null, p, p, p, 4, 10, null) == ERR_NULL
    assert b(3, p, p, p, p, p, p, p, p, p, p, p, p, 4, 3, null) == ERR_POINTS
    assert b(3, p, p, p, p, p, p, null, null, p, p, p, p, 0, 10, null) == OK


def test_torsion_status_paths(lib):
    p = ctypes.c_void_p(1)
    null = None
    f = lib.cufk_torsion_fwd
    assert f(0, p, 14, null, p, 2, 10, null) == ERR_NULL  # constants are required
    assert f(0, p, -1, p, p, 2, 10, null) == ERR_STRIDE
    assert f(0, p, 14, p, p, 2, 2052, null) == ERR_STEPS
    assert f(0, p, 14, p, p, 0, 10, null) == OK
    b = lib.cufk_torsion_bwd
    assert b(0, p, 14, p, p, p, -3, p, 2, 10, null) == ERR_STRIDE
    # Gradient rows (14 values at N = 10) must not overlap: a shorter row stride is refused
    # for two chains or more; one chain has no second row to overlap (the stride check passes
    # and the missing gradient pointer is what is refused).  Overlapping raw rows are only read.
    assert b(0, p, 14, p, p, p, 13, p, 2, 10, null) == ERR_STRIDE
    assert b(0, p, 14, p, p, p, 0, p, 2, 10, null) == ERR_STRIDE
    assert b(0, p, 3, p, p, null, 14, p, 2, 10, null) == ERR_NULL
    assert b(0, p, 14, p, p, null, 3, p, 1, 10, null) == ERR_NULL
    assert b(0, p, 14, p, p, null, 0, p, 1, 10, null) == ERR_NULL
    assert lib.cufk_error_string(ERR_STRIDE) == b"negative row stride, or gradient row stride shorter than the row"
    assert b(3, p, 14, p, p, p, 14, p, 2, 3, null) == ERR_POINTS


ERR_SEGMENT = 9


def test_long_sizes_and_default_segments(lib):
    seg = lib.cufk_long_segment_steps
    assert seg(4096, 2049) == 2048  # 4096 chains x 1 segment already fill the grid
    assert seg(1, 100000) == 256  # 1 chain: halved down to the 256-step floor (391 segments)
    assert seg(64, 131072) == 2048  # 64 x 64 segments
    assert seg(16, 65536) == 1024  # 16 x 32 = 512 < 1024 at 2048; 16 x 64 at 1024
    assert seg(0, 10) == 256 and seg(4, 3) == 0 and seg(-1, 10) == 0
    # 24 doubles per (chain, segment), its flag bytes in whole 16-byte units, then room for
    # the local positions as (chains, points, 3) doubles.
    assert lib.cufk_long_state_doubles(3, 5003, 1000) == 3 * 5 * 24 + 2 + 3 * 5003 * 3
    assert lib.cufk_long_work_doubles(3, 5003, 1000) == 3 * 5 * 12
    assert lib.cufk_long_state_doubles(3, 5004, 1000) == 3 * 6 * 24 + 4 + 3 * 5004 * 3
    assert lib.cufk_long_state_doubles(3, 5004, 0) == -1
    assert lib.cufk_long_state_doubles(3, 5004, 2049) == -1
    assert lib.cufk_long_state_doubles(3, 3, 16) == -1
    assert lib.cufk_long_state_doubles(2, 2**31 // 3 + 1, 2048) == -1  # in-row offsets past int32


def test_long_status_paths(lib):
    p = ctypes.c_void_p(1)
    null = None
    f = lib.cufk_reconstruct_long_fwd
    assert f(9, p, p, p, p, p, p, p, p, 4, 10, 4, null) == ERR_DTYPE
    assert f(0, p, p, p, p, p, p, p, p, 4, 3, 4, null) == ERR_POINTS
    assert f(0, p, p, p, p, p, p, p, p, 4, 10, 0, null) == ERR_SEGMENT
    assert f(0, p, p, p, p, p, p, p, p, 4, 10, 2049, null) == ERR_SEGMENT
    assert f(0, p, p, p, p, p, p, p, null, 4, 10, 4, null) == ERR_NULL  # state is required
    assert f(0, p, p, p, p, p, p, p, p, 0, 10, 4, null) == OK
    assert f(0, p, p, p, p, p, p, p, p, 2**20, 2**20, 1, null) == ERR_SHAPE  # grid past 32 bits
    b = lib.cufk_reconstruct_long_bwd
    assert b(0, p, p, p, p, p, p, p, p, p, null, p, p, p, 4, 10, 4, null) == ERR_NULL  # work is required
    assert b(0, p, p, p, p, p, p, p, p, p, p, p, p, p, 4, 10, 0, null) == ERR_SEGMENT
    assert b(0, p, p, p, p, p, p, p, p, p, p, p, p, p, 0, 10, 4, null) == OK
    assert lib.cufk_error_string(ERR_SEGMENT) == b"segment length must be in [1, 2048] local transforms"


def test_loss_status_paths(lib):
    p = ctypes.c_void_p(1)
    null = None
    f = lib.cufk_reconstruct_loss_fwd
    assert f(9, p, p, p, p, p, p, p, p, p, p, 4, 10, null) == ERR_DTYPE
    assert f(0, p, p, p, p, p, p, p, p, p, p, 4, 2052, null) == ERR_STEPS
    assert f(0, p, p, p, p, p, p, null, p, p, p, 4, 10, null) == ERR_NULL  # target is required
    assert f(0, p, p, p, p, p, p, p, p, null, p, 4, 10, null) == ERR_NULL  # flags are written
    assert f(0, p, p, p, p, p, p, p, p, p, p, 0, 10, null) == OK
    b = lib.cufk_reconstruct_loss_bwd
    assert b(0, p, p, p, p, p, p, p, p, p, p, null, p, p, 4, 10, null) == ERR_NULL  # gradients are required
    assert b(0, p, p, p, p, p, p, p, p, p, null, p, p, p, 4, 3, null) == ERR_POINTS  # grad_loss may be null
    assert b(0, p, p, p, p, p, p, p, p, p, null, p, p, p, 0, 10, null) == OK


def test_anchored_status_paths(lib):
    p = ctypes.c_void_p(1)
    null = None
    f = lib.cufk_reconstruct_bwd_anchored
    #        dtype L  A  D  p0 d0 n0 xyz flags g  gL gA gD work gp0 gd0 gn0
    assert f(9, p, p, p, p, p, p, p, p, p, p, p, p, p, p, p, p, 4, 10, null) == ERR_DTYPE
    assert f(0, p, p, p, p, p, p, p, p, p, p, p, p, p, p, p, p, 4, 2052, null) == ERR_STEPS
    assert f(0, p, p, p, p, p, p, p, null, p, p, p, p, p, p, p, p, 4, 10, null) == ERR_NULL  # xyz needs its flags
    assert f(0, p, p, p, p, p, p, p, p, p, p, p, p, null, p, p, p, 4, 10, null) == ERR_NULL  # scratch is required
    assert f(0, p, p, p, p, p, p, p, p, p, p, p, p, p, null, p, p, 4, 10, null) == ERR_NULL  # anchor gradients too


ERR_SCRATCH = 10


def test_anchored_noalloc_status_paths(lib):
    """The allocation-free anchored backward checks its arguments before it looks up its static
    scratch on the device: no GPU is touched by these calls."""
    p = ctypes.c_void_p(1)
    null = None
    f = lib.cufk_reconstruct_bwd_anchored_noalloc
    #        dtype L  A  D  p0 d0 n0 xyz flags g  gL gA gD gp0 gd0 gn0
    assert f(9, p, p, p, p, p, p, p, p, p, p, p, p, p, p, p, 4, 10, null) == ERR_DTYPE
    assert f(0, p, p, p, p, p, p, p, p, p, p, p, p, p, p, p, 4, 2052, null) == ERR_STEPS
    assert f(0, p, p, p, p, p, p, p, p, p, p, p, p, p, p, p, 65537, 10, null) == ERR_SCRATCH
    assert f(0, p, p, p, p, p, p, p, p, p, p, p, p, p, p, p, 65537, 3, null) == ERR_POINTS
    assert lib.cufk_error_string(ERR_SCRATCH).startswith(b"batch exceeds the 65536 chains")


ERR_LOSS = 11


def test_fused_loss_status_paths(lib):
    """Loss kinds, shapes and pointers are checked before any device work."""
    p = ctypes.c_void_p(1)
    null = None
    f = lib.cufk_reconstruct_superposed_fwd
    #        dtype kind L  A  D  p0 d0 n0 tgt xyz flags loss rec
    assert f(0, 0, p, p, p, p, p, p, p, p, p, p, p, 4, 10, null) == ERR_LOSS  # squared distance: reconstruct_loss
    assert f(0, 3, p, p, p, p, p, p, p, p, p, p, p, 4, 10, null) == ERR_LOSS
    assert f(9, 2, p, p, p, p, p, p, p, p, p, p, p, 4, 10, null) == ERR_DTYPE
    assert f(0, 2, p, p, p, p, p, p, p, p, p, p, null, 4, 10, null) == ERR_NULL  # the record is required
    assert f(0, 1, p, p, p, p, p, p, p, p, p, p, p, 4, 3, null) == ERR_POINTS
    assert f(0, 1, p, p, p, p, p, p, p, p, p, p, null, 0, 10, null) == OK  # empty batch: nothing to do
    b = lib.cufk_reconstruct_superposed_bwd
    #        dtype kind L  A  D  p0 d0 n0 xyz flags tgt rec gl gL gA gD
    assert b(0, 2, p, p, p, p, p, p, p, p, p, null, null, p, p, p, 4, 10, null) == ERR_NULL
    assert b(0, 2, p, p, p, p, p, p, p, p, p, p, null, p, p, p, 4, 2052, null) == ERR_STEPS
    t = lib.cufk_torsion_loss_fwd
    #        dtype kind raw stride consts tgt xyz loss rec
    assert t(0, 4, p, 10, p, p, p, p, p, 4, 8, null) == ERR_LOSS
    assert t(0, 0, p, -1, p, p, p, p, null, 4, 8, null) == ERR_STRIDE
    assert t(0, 2, p, 10, p, p, p, p, null, 4, 8, null) == ERR_NULL  # superposed kinds need the record
    tb = lib.cufk_torsion_loss_bwd
    #         dtype kind raw stride xyz tgt rec gl graw gstride consts
    assert tb(0, 1, p, 10, p, p, null, null, p, 10, p, 4, 8, null) == ERR_NULL
    assert tb(0, 0, p, 10, p, p, null, null, p, -2, p, 4, 8, null) == ERR_STRIDE
    assert tb(0, 0, p, 10, p, p, null, null, p, 9, p, 4, 8, null) == ERR_STRIDE  # rows of 10 would overlap
    assert tb(0, 0, p, 10, p, p, null, null, null, 9, p, 1, 8, null) == ERR_NULL  # one chain: stride accepted
    assert lib.cufk_error_string(ERR_LOSS) == b"unknown or unsupported loss kind"


def declared_parameter_counts():
    text = HEADER.read_text()
    counts = {}
    for m in re.finditer(r"^\s*(?:int|int64_t|const char\*)\s+(cufk_\w+)\s*\((.*?)\);", text, re.M | re.S):
        params = m.group(2).strip()
        counts[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return counts


def _documented_argtypes():
    """The `lib.NAME.argtypes = [...]` lines of the integration notes, evaluated with placeholders."""
    import types

    ns = {"vp": "p", "i64": "i", "ctypes": types.SimpleNamespace(c_int="c", c_void_p="p", c_int64="i")}
    out = {}
    for m in re.finditer(r"^lib\.(cufk_\w+)\.argtypes = (.+)$", (ROOT / "INTEGRATION.md").read_text(), re.M):
        out[m.group(1)] = eval(m.group(2), {}, dict(ns))  # noqa: S307 - the repository's own documentation
    return out


def test_documented_ctypes_bindings_match_the_header():
    """Every argtypes list the integration notes give has as many entries as the header's
    declaration has parameters (a count that has drifted once is now pinned)."""
    declared = declared_parameter_counts()
    documented = _documented_argtypes()
    assert len(documented) >= 10
    for name, types_ in documented.items():
        assert len(types_) == declared[name], (name, len(types_), declared[name])


def test_test_bindings_match_the_header(lib):
    declared = declared_parameter_counts()
    for name, n in declared.items():
        fn = getattr(lib, name)
        if fn.argtypes is not None:
            assert len(fn.argtypes) == n, (name, len(fn.argtypes), n)


def test_documented_c_snippet_compiles(tmp_path):
    """The C example of the integration notes, wrapped in a function, compiles against the
    header with gcc (syntax and types only; nothing is linked or run)."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no host C compiler")
    body = re.search(r"```c\n(.*?)```", (ROOT / "INTEGRATION.md").read_text(), re.S).group(1)
    include, rest = body.split("\n", 1)
    src = tmp_path / "snippet.c"
    src.write_text("#include <math.h>\n#include <stdint.h>\n#include <stdio.h>\n" + include + "\n"
                   "int demo(const void* d_raw, int64_t raw_stride, void* d_xyz, int64_t B, int64_t N, void* stream) {\n"
                   + rest + "\nreturn rc;\n}\n")
    proc = subprocess.run([gcc, "-std=c11", "-Wall", "-Werror", "-fsyntax-only", f"-I{ROOT / 'include'}", str(src)],
                          capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
