"""The C-ABI library: it loads, exports every function `include/attnres_hip.h`
declares with the argument list the ctypes binding uses, and rejects invalid
arguments on the host with the documented status codes before any device
work.  Runs without a GPU (no valid call is made)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from attnres import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "attnres_hip.h"

_C_TYPES = {
    "void*": ctypes.c_void_p, "const void*": ctypes.c_void_p, "float*": ctypes.c_void_p,
    "const float*": ctypes.c_void_p, "int8_t*": ctypes.c_void_p, "const int8_t*": ctypes.c_void_p,
    "const void* const*": ctypes.c_void_p, "void* const*": ctypes.c_void_p,
    "const int64_t*": ctypes.c_void_p, "const uint8_t*": ctypes.c_void_p, "int64_t": ctypes.c_int64,
    "float": ctypes.c_float, "float* const*": ctypes.c_void_p, "int": ctypes.c_int,
    "const attnres_gather_read*": ctypes.c_void_p,
}


def _declarations() -> dict[str, list[str]]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    found = {}
    for match in re.finditer(r"\b(?:int|int64_t|const char\*)\s+(attnres_hip_\w+)\s*\(([^)]*)\)\s*;", text):
        name, params = match.group(1), match.group(2).strip()
        if params in ("", "void"):
            found[name] = []
            continue
        types = []
        for param in params.split(","):
            words = " ".join(param.split())
            types.append(re.sub(r"\s*\b\w+$", "", words).replace(" *", "*"))
        found[name] = types
    return found


def test_header_declares_the_bound_functions():
    assert set(_declarations()) == set(_native.SIGNATURES)


@pytest.mark.parametrize("name", sorted(_native.SIGNATURES))
def test_binding_matches_header_argument_list(name):
    declared = [_C_TYPES[t] for t in _declarations()[name]]
    assert _native.SIGNATURES[name][1] == declared


def test_library_loads_and_exports_every_symbol():
    lib = _native.load()
    for name in _declarations():
        assert hasattr(lib, name), name
    import attnres

    assert lib.attnres_hip_version().decode() == attnres.__version__


def test_workspace_size_is_shape_only_and_rejects_bad_shapes():
    lib = _native.load()
    assert lib.attnres_hip_dq_workspace_elems(16384, 2048, 2048) > 2048
    assert (lib.attnres_hip_dq_workspace_elems(16384, 2048, 2048)
            == lib.attnres_hip_dq_workspace_elems(16384, 2048, 2048))
    assert lib.attnres_hip_dq_workspace_elems(0, 2048, 2048) == -1
    assert lib.attnres_hip_dq_workspace_elems(16, 8193, 16) == -1
    assert lib.attnres_hip_dq_workspace_elems(16, 64, 65) == -1


_FAKE = 0x1000  # never dereferenced: every call below fails host-side checks


def _forward(**overrides):
    args = dict(values=_FAKE, source_stride=64, row_stride=64, n_sources=3, n_tokens=4,
                width=64, query=_FAKE, rank=16, eps=2.0**-23, scale=1.0, out=_FAKE,
                out_refine=_FAKE, logit=_FAKE, inv_rms=_FAKE, stats=_FAKE, stream=None)
    args.update(overrides)
    return _native.load().attnres_hip_packed_forward(*args.values())


@pytest.mark.parametrize("override,status", [
    ({"values": None}, _native.ERR_NULL_POINTER),
    ({"out": None}, _native.ERR_NULL_POINTER),
    ({"n_sources": 0}, _native.ERR_SHAPE),
    ({"n_sources": 130}, _native.ERR_SHAPE),
    ({"n_tokens": 0}, _native.ERR_SHAPE),
    ({"width": 8193}, _native.ERR_SHAPE),
    ({"rank": 65}, _native.ERR_SHAPE),
    ({"rank": 0}, _native.ERR_SHAPE),
    ({"row_stride": -1}, _native.ERR_STRIDE),
    ({"eps": 0.0}, _native.ERR_SCALAR),
    ({"eps": float("nan")}, _native.ERR_SCALAR),
    ({"scale": float("inf")}, _native.ERR_SCALAR),
])
def test_packed_forward_rejects_invalid_arguments(override, status):
    assert _forward(**override) == status
    assert _native.load().attnres_hip_last_error().decode()


def test_backward_rejects_a_short_workspace():
    lib = _native.load()
    need = lib.attnres_hip_dq_workspace_elems(4, 64, 16)
    status = lib.attnres_hip_packed_backward(
        _FAKE, 64, 64, 3, 4, 64, _FAKE, 16, 1.0, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE,
        _FAKE, _FAKE, _FAKE, need - 1, None)
    assert status == _native.ERR_WORKSPACE
    assert b"workspace" in lib.attnres_hip_last_error()


def test_source_list_rejects_null_entries():
    lib = _native.load()
    pointers = (ctypes.c_void_p * 2)(_FAKE, None)
    strides = (ctypes.c_int64 * 2)(64, 64)
    status = lib.attnres_hip_sources_forward(
        pointers, strides, 2, 4, 64, _FAKE, 16, 2.0**-23, 1.0, _FAKE, _FAKE, _FAKE, _FAKE,
        _FAKE, None)
    assert status == _native.ERR_NULL_POINTER


def test_status_is_raised_with_the_library_message():
    _forward(width=9000)
    with pytest.raises(ValueError, match="width"):
        _native.check(_native.ERR_SHAPE, "attnres packed forward")


def test_accumulating_backward_needs_its_flags_and_checks_like_the_plain_one():
    """The accumulate entry points take the plain backward's arguments plus a
    host array of flags; a missing array and the plain checks fail on the
    host (no device work)."""
    lib = _native.load()
    need = lib.attnres_hip_dq_workspace_elems(4, 64, 16)
    flags = (ctypes.c_uint8 * 3)(1, 0, 1)
    common = (_FAKE, 16, 1.0, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE)
    status = lib.attnres_hip_packed_backward_accumulate(
        _FAKE, 64, 64, 3, 4, 64, *common, _FAKE, _FAKE, _FAKE, need, None, None)
    assert status == _native.ERR_NULL_POINTER
    assert b"accumulate" in lib.attnres_hip_last_error()
    status = lib.attnres_hip_packed_backward_accumulate(
        _FAKE, 64, 64, 3, 4, 64, *common, _FAKE, _FAKE, _FAKE, need - 1, flags, None)
    assert status == _native.ERR_WORKSPACE
    pointers = (ctypes.c_void_p * 3)(_FAKE, _FAKE, _FAKE)
    strides = (ctypes.c_int64 * 3)(64, 64, 64)
    status = lib.attnres_hip_sources_backward_accumulate(
        pointers, strides, 3, 4, 64, *common, pointers, _FAKE, _FAKE, need, None, None)
    assert status == _native.ERR_NULL_POINTER
    status = lib.attnres_hip_sources_backward_accumulate(
        pointers, strides, 0, 4, 64, *common, pointers, _FAKE, _FAKE, need, flags, None)
    assert status == _native.ERR_SHAPE


def test_save_recompute_policy_matches_the_header_and_the_ops():
    """Reads of at most ATTNRES_RECOMPUTE_MAX_SOURCES sources save no
    refinement (the reference recomputes for S <= 3, fla_full_sources.py:146-161;
    the register-resident backward pays up to 6 here), and neither do reads of
    at most ATTNRES_KEYRES_MAX_SOURCES whose key is the last 512 or 1024
    elements of a 2048- or 4096-wide row (the key-resident backward).  The
    library and the ops agree on every shape class."""
    from attnres import _ops

    lib = _native.load()
    text = HEADER.read_text()
    assert f"#define ATTNRES_RECOMPUTE_MAX_SOURCES {_ops.RECOMPUTE_MAX_SOURCES}" in text
    assert f"#define ATTNRES_KEYRES_MAX_SOURCES {_ops.KEYRES_MAX_SOURCES}" in text
    assert f"#define ATTNRES_KEYRES_FULL_MAX_SOURCES {_ops.KEYRES_FULL_MAX_SOURCES}" in text
    assert _ops.RECOMPUTE_MAX_SOURCES == 6 and _ops.KEYRES_MAX_SOURCES == 16 and _ops.KEYRES_FULL_MAX_SOURCES == 12
    for count in range(1, 130):
        assert bool(lib.attnres_hip_saves_refinement(count)) == (count > 6)
    key_resident = {(2048, 512), (2048, 1024), (4096, 512), (4096, 1024)}
    full_key = {(2048, 2048)}
    widths = (1, 8, 64, 100, 512, 1000, 1024, 1536, 2040, 2048, 2056, 3072, 4096, 5000, 8192)
    for width in widths:
        for rank in sorted({1, 8, 256, 511, 512, 513, 768, 1024, 1536, 2048, 3072, width // 2, width} - {0}):
            if rank > width:
                continue
            for count in (1, 6, 7, 9, 12, 13, 16, 17, 25, 129):
                expected = count > 6 and not ((count <= 16 and (width, rank) in key_resident) or
                                              (count <= 12 and (width, rank) in full_key))
                assert _ops.saves_refinement(count, width, rank) == expected, (count, width, rank)
                assert bool(lib.attnres_hip_saves_refinement_for(count, width, rank)) == expected, (count, width, rank)


def test_backward_without_the_refinement_is_for_small_reads_only():
    """out_refine = NULL selects the recompute kernel: more than 6 sources is a
    shape error, and the accumulating entry points still need the refinement;
    both are rejected on the host."""
    lib = _native.load()
    need = lib.attnres_hip_dq_workspace_elems(4, 64, 16)
    stats = (_FAKE, _FAKE, _FAKE)
    status = lib.attnres_hip_packed_backward(
        _FAKE, 64, 64, 7, 4, 64, _FAKE, 16, 1.0, None, None, _FAKE, *stats, _FAKE, _FAKE, _FAKE, need, None)
    assert status == _native.ERR_SHAPE
    assert b"n_sources <= 6" in lib.attnres_hip_last_error()
    # the key-resident backward: 16 sources of 4096-wide rows with a 1024 key pass
    # the checks up to the workspace; 17 sources, or a key of 768, do not
    need_wide = lib.attnres_hip_dq_workspace_elems(4, 4096, 1024)
    for count, rank, expected in ((16, 1024, _native.ERR_WORKSPACE), (17, 1024, _native.ERR_SHAPE),
                                  (16, 768, _native.ERR_SHAPE)):
        status = lib.attnres_hip_packed_backward(
            _FAKE, 4096 * 4, 4096, count, 4, 4096, _FAKE, rank, 1.0, None, None, _FAKE, *stats, _FAKE, _FAKE, _FAKE,
            lib.attnres_hip_dq_workspace_elems(4, 4096, rank) - 1 if rank == 1024 else need_wide, None)
        assert status == expected, (count, rank)
    status = lib.attnres_hip_packed_backward(  # small read: checks pass up to the workspace
        _FAKE, 64, 64, 6, 4, 64, _FAKE, 16, 1.0, None, None, _FAKE, *stats, _FAKE, _FAKE, _FAKE, need - 1, None)
    assert status == _native.ERR_WORKSPACE
    pointers = (ctypes.c_void_p * 7)(*[_FAKE] * 7)
    strides = (ctypes.c_int64 * 7)(*[64] * 7)
    status = lib.attnres_hip_sources_backward(
        pointers, strides, 7, 4, 64, _FAKE, 16, 1.0, None, None, _FAKE, *stats, pointers, _FAKE, _FAKE, need, None)
    assert status == _native.ERR_SHAPE
    flags = (ctypes.c_uint8 * 3)(0, 0, 0)
    status = lib.attnres_hip_packed_backward_accumulate(
        _FAKE, 64, 64, 3, 4, 64, _FAKE, 16, 1.0, None, None, _FAKE, *stats, _FAKE, _FAKE, _FAKE, need, flags, None)
    assert status == _native.ERR_NULL_POINTER


def test_partial_sum_checks_its_arguments_on_the_host():
    lib = _native.load()
    assert lib.attnres_hip_partial_sum(None, _FAKE, 0, 16, _FAKE, _FAKE, None) == _native.ERR_NULL_POINTER
    assert lib.attnres_hip_partial_sum(_FAKE, _FAKE, 2, 16, _FAKE, _FAKE, None) == _native.ERR_SHAPE
    assert b"dtype" in lib.attnres_hip_last_error()
    assert lib.attnres_hip_partial_sum(_FAKE, _FAKE, 0, 0, _FAKE, _FAKE, None) == _native.ERR_SHAPE
    text = HEADER.read_text()
    assert "#define ATTNRES_DTYPE_F32 0" in text and "#define ATTNRES_DTYPE_BF16 1" in text
    from attnres import shared

    assert f"#define ATTNRES_MAX_GATHER_READS {shared._MAX_GATHER_READS}" in text


def test_list_f32_accumulating_backward_checks_like_the_others():
    lib = _native.load()
    need = lib.attnres_hip_dq_workspace_elems(4, 64, 16)
    pointers = (ctypes.c_void_p * 3)(_FAKE, _FAKE, _FAKE)
    strides = (ctypes.c_int64 * 3)(64, 64, 64)
    flags = (ctypes.c_uint8 * 3)(0, 1, 0)
    common = (_FAKE, 16, 1.0, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE)
    status = lib.attnres_hip_sources_backward_accumulate_f32(
        pointers, strides, 3, 4, 64, *common, pointers, _FAKE, _FAKE, need, None, None)
    assert status == _native.ERR_NULL_POINTER
    assert b"accumulate_f32" in lib.attnres_hip_last_error()
    status = lib.attnres_hip_sources_backward_accumulate_f32(
        pointers, strides, 3, 4, 64, *common, pointers, _FAKE, _FAKE, need - 1, flags, None)
    assert status == _native.ERR_WORKSPACE


def test_gather_read_struct_matches_the_header():
    """attnres_gather_read: three pointers and three int64, in the header's
    order (the ctypes mirror attnres.shared._GatherRead)."""
    from attnres.shared import _GatherRead

    body = re.search(r"typedef struct attnres_gather_read \{(.*?)\} attnres_gather_read;", HEADER.read_text(), re.S)
    fields = re.findall(r"^\s*[\w\s\*]+?\b(\w+);", re.sub(r"/\*.*?\*/", "", body.group(1), flags=re.S), re.M)
    assert fields == [name for name, _ in _GatherRead._fields_]
    assert ctypes.sizeof(_GatherRead) == 6 * 8
    # the source bank passes the table as an int64 array of the same bytes
    from array import array

    rows = [(0x7F0000001000, 0x7F0000002000, 0x7F0000003000, 5, 2, 384), (16, 32, 48, 1, 0, 1)]
    table = (_GatherRead * 2)(*rows)
    packed = array("q", [field for row in rows for field in row])
    assert bytes(table) == packed.tobytes()


def test_coefficient_backward_and_gather_check_on_the_host():
    from attnres.shared import _GatherRead

    lib = _native.load()
    need = lib.attnres_hip_dq_workspace_elems(4, 64, 16)
    stats = (_FAKE, _FAKE, _FAKE)
    status = lib.attnres_hip_packed_backward_coef(
        _FAKE, 64, 64, 3, 4, 64, _FAKE, 16, 1.0, _FAKE, None, _FAKE, *stats, _FAKE, _FAKE, _FAKE, need, None)
    assert status == _native.ERR_NULL_POINTER  # the coefficient backward needs the saved refinement
    status = lib.attnres_hip_packed_backward_coef(
        _FAKE, 64, 64, 3, 4, 64, _FAKE, 16, 1.0, _FAKE, _FAKE, _FAKE, *stats, None, _FAKE, _FAKE, need, None)
    assert status == _native.ERR_NULL_POINTER
    pointers = (ctypes.c_void_p * 3)(_FAKE, _FAKE, _FAKE)
    strides = (ctypes.c_int64 * 3)(64, 64, 64)
    status = lib.attnres_hip_sources_backward_coef(
        pointers, strides, 3, 4, 64, _FAKE, 16, 1.0, _FAKE, _FAKE, _FAKE, *stats, _FAKE, _FAKE, _FAKE, need - 1,
        None)
    assert status == _native.ERR_WORKSPACE
    reads = (_GatherRead * 2)()
    for entry in reads:
        entry.grad_out = entry.query_row = entry.coef = _FAKE
        entry.n_sources, entry.position, entry.rank = 3, 1, 16
    reads[1].position = 3
    assert lib.attnres_hip_bank_gather(_FAKE, 64, 4, 64, reads, 2, _FAKE, 0, 0, None) == _native.ERR_SHAPE
    assert b"position" in lib.attnres_hip_last_error()
    reads[1].position, reads[1].coef = 2, None
    assert lib.attnres_hip_bank_gather(_FAKE, 64, 4, 64, reads, 2, _FAKE, 0, 0, None) == _native.ERR_NULL_POINTER
    from array import array

    packed = array("q", bytes(reads))  # the source bank's form of the table: the same checks apply
    packed[3 + 6] = 4  # read 1: n_sources 3 -> 4, so position 2 is in range but coef is still NULL
    assert lib.attnres_hip_bank_gather(_FAKE, 64, 4, 64, packed.buffer_info()[0], 2, _FAKE, 0, 0,
                                       None) == _native.ERR_NULL_POINTER
    assert lib.attnres_hip_bank_gather(_FAKE, 64, 4, 64, reads, 0, _FAKE, 0, 0, None) == _native.ERR_SHAPE
    # BF16 output: a known element type, written by one launch (every case fails before any launch)
    reads[1].coef = _FAKE
    assert lib.attnres_hip_bank_gather(_FAKE, 64, 4, 64, reads, 2, _FAKE, 7, 0, None) == _native.ERR_SHAPE
    assert b"grad_dtype" in lib.attnres_hip_last_error()
    bf16 = 1
    assert lib.attnres_hip_bank_gather(_FAKE, 64, 4, 64, reads, 2, _FAKE, bf16, 1, None) == _native.ERR_SHAPE
    assert b"one launch" in lib.attnres_hip_last_error()
    reads[1].rank = 32
    assert lib.attnres_hip_bank_gather(_FAKE, 64, 4, 64, reads, 2, _FAKE, bf16, 0, None) == _native.ERR_SHAPE
    many = (_GatherRead * 49)(*[(_FAKE, _FAKE, _FAKE, 3, 0, 16)] * 49)
    assert lib.attnres_hip_bank_gather(_FAKE, 64, 4, 64, many, 49, _FAKE, bf16, 0, None) == _native.ERR_SHAPE
    assert b"at most 48 reads" in lib.attnres_hip_last_error()


def test_workspace_holds_the_widest_backward_grid():
    """The dq workspace holds one partial row per workgroup of the widest
    backward variant plus the total: for 2048 < D <= 4096 the recompute kernel
    runs one token per workgroup, elsewhere the geometry's groups share one."""
    lib = _native.load()
    assert lib.attnres_hip_dq_workspace_elems(100, 3000, 257) == (100 + 1) * 257
    assert lib.attnres_hip_dq_workspace_elems(100, 2048, 2048) == (25 + 1) * 2048    # 4 groups of 64 lanes
    assert lib.attnres_hip_dq_workspace_elems(100, 1024, 1024) == (13 + 1) * 1024    # 8 groups of 32 lanes
    assert lib.attnres_hip_dq_workspace_elems(100, 8192, 8192) == (100 + 1) * 8192   # a workgroup per token
    assert lib.attnres_hip_dq_workspace_elems(10**6, 4096, 64) == (2048 + 1) * 64    # the persistent-grid cap


def test_no_alloc_backward_checks_arguments_on_the_host():
    """The no-allocation backward rejects bad shapes and null pointers before
    any runtime call (so also on a machine without a GPU)."""
    lib = _native.load()
    args = [None, 0, 0, 2, 4, 64, None, 65, 1.0, None, None, None, None, None, None, None, None, None]
    assert lib.attnres_hip_packed_backward_noalloc(*args) == _native.ERR_SHAPE
    assert b"rank" in lib.attnres_hip_last_error()
    args[7] = 64
    assert lib.attnres_hip_packed_backward_noalloc(*args) == _native.ERR_NULL_POINTER
    assert b"attnres_hip_packed_backward_noalloc" in lib.attnres_hip_last_error()


def test_no_alloc_backward_runs_every_check_before_touching_the_device():
    """The recompute, stride and scale checks of the no-allocation backward
    name that entry point and run before it looks up its device scratch, so
    they return their own codes on a machine without a GPU (a device lookup
    would fail with ATTNRES_ERR_LAUNCH instead)."""
    lib = _native.load()
    fake = ctypes.c_void_p(16)
    # S = 7 without out_refine: the recompute kernel takes at most 6 sources
    args = [fake, 0, 64, 7, 4, 64, fake, 64, 1.0, None, None, fake, fake, fake, fake, fake, fake, None]
    assert lib.attnres_hip_packed_backward_noalloc(*args) == _native.ERR_SHAPE
    assert b"attnres_hip_packed_backward_noalloc" in lib.attnres_hip_last_error()
    args[3] = 2  # a small read may recompute; now a negative row stride
    args[2] = -64
    assert lib.attnres_hip_packed_backward_noalloc(*args) == _native.ERR_STRIDE
    assert b"attnres_hip_packed_backward_noalloc" in lib.attnres_hip_last_error()
    args[2] = 64
    args[8] = float("nan")
    assert lib.attnres_hip_packed_backward_noalloc(*args) == _native.ERR_SCALAR
