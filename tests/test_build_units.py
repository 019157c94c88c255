"""The library's translation units (fast-attnres_amd/build_native.py), on the
CPU: every row geometry of the dispatch table is compiled for gfx950 with the
packed-FP32 VALU ops disabled; the 4096-wide geometry is built in two parts,
its unmasked forwards and gather (default scheduler) and its backwards and
masked forwards (iterative-minreg); one more unit
holds the 2048-wide token-block and whole-row key-resident backwards built
with the max-ilp scheduler.  A unit dropped from the list would leave
launchers undefined in the shared library, which the loader reports only on
the GPU box; the last test checks the built library for that here.
"""

from __future__ import annotations

import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "fast-attnres_amd"))

import build_native  # noqa: E402

PACKED_FP32_OFF = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _units():
    units = {}
    for cmd, obj in build_native.compile_commands():
        units[obj.name] = cmd
    return units


def _has_sequence(cmd, seq):
    return any(cmd[i:i + len(seq)] == seq for i in range(len(cmd) - len(seq) + 1))


def test_geometries_match_the_dispatch_table():
    header = (ROOT / "fast-attnres_amd" / "csrc" / "attnres_internal.h").read_text()
    line = re.search(r"#define ATTNRES_FOR_EACH_GEOMETRY\(X\)(.*)", header).group(1)
    table = tuple((int(g), int(c)) for g, c in re.findall(r"X\((\d+),\s*(\d+)\)", line))
    assert table == build_native.GEOMETRIES


def test_every_geometry_has_its_units():
    units = _units()
    assert "attnres_hip.o" in units
    for lanes, chunks in build_native.GEOMETRIES:
        stem = f"attnres_kernels_g{lanes}_c{chunks}"
        defines = [f"-DATTNRES_LANES={lanes}", f"-DATTNRES_CHUNKS={chunks}"]
        if (lanes, chunks) in build_native.SPLIT_GEOMETRIES:
            assert f"{stem}.o" not in units
            forward, backward = units[f"{stem}_part1.o"], units[f"{stem}_part2.o"]
            assert all(d in forward for d in defines) and "-DATTNRES_UNIT_PART=1" in forward
            assert all(d in backward for d in defines) and "-DATTNRES_UNIT_PART=2" in backward
            assert not any(a.startswith("-amdgpu-sched-strategy") for a in forward)
            assert _has_sequence(backward, build_native.SPLIT_GEOMETRIES[(lanes, chunks)])
        else:
            cmd = units[f"{stem}.o"]
            assert all(d in cmd for d in defines)
            assert not any(a.startswith("-DATTNRES_UNIT_PART") or a.startswith("-amdgpu-sched-strategy") for a in cmd)
    max_ilp = units["attnres_kernels_max_ilp.o"]
    assert "-DATTNRES_MAX_ILP_UNIT" in max_ilp
    assert _has_sequence(max_ilp, ["-mllvm", "-amdgpu-sched-strategy=max-ilp"])
    assert not any(a.startswith("-DATTNRES_LANES") for a in max_ilp)
    assert build_native.SPLIT_GEOMETRIES[(64, 8)] == ["-mllvm", "-amdgpu-sched-strategy=iterative-minreg"]


def test_every_unit_targets_gfx950_without_packed_fp32():
    for name, cmd in _units().items():
        assert f"--offload-arch={build_native.ARCH}" in cmd and build_native.ARCH == "gfx950", name
        assert _has_sequence(cmd, PACKED_FP32_OFF), name
        assert "-O3" in cmd, name


def test_built_library_leaves_no_attnres_symbol_undefined():
    lib = build_native.OUTPUT
    nm = shutil.which("nm")
    if not lib.exists() or nm is None:
        pytest.skip("library not built or nm missing")
    undefined = subprocess.run([nm, "-C", "--undefined-only", str(lib)], capture_output=True, text=True,
                               check=True).stdout
    assert not [line for line in undefined.splitlines() if "attnres_hip" in line]
    defined = subprocess.run([nm, "-C", "--defined-only", str(lib)], capture_output=True, text=True,
                             check=True).stdout
    for launcher in ("launch_bwd_block<64, 4, 4, true", "launch_bwd_keyres_chunks<64, 4, 4, true",
                     "launch_bwd_geometry<64, 8", "launch_fwd_geometry<64, 8",
                     "launch_fwd<64, 8, false, true"):
        assert launcher in defined, launcher


def test_scheduler_units_hold_the_only_definitions():
    """Template instances are weak symbols: if a default-scheduler unit also
    instantiated a launcher that a scheduler unit provides, the linker would
    keep either copy without a word.  The default units must only reference
    them (nm 'U'), the scheduler units define them."""
    nm = shutil.which("nm")
    build = build_native.BUILD_DIR
    pairs = {
        "attnres_kernels_g64_c8_part1.o": ("attnres_kernels_g64_c8_part2.o", "launch_fwd<64, 8, false, "),
        "attnres_kernels_g64_c4.o": ("attnres_kernels_max_ilp.o", "launch_bwd_block<64, 4, 4, true, "),
    }
    if nm is None or not all((build / a).exists() and (build / b).exists() for a, (b, _) in pairs.items()):
        pytest.skip("objects not built or nm missing")

    def symbol_lines(obj, needle):
        out = subprocess.run([nm, "-C", str(build / obj)], capture_output=True, text=True, check=True).stdout
        return [line for line in out.splitlines() if needle in line]

    for plain, (scheduled, needle) in pairs.items():
        plain_lines, scheduled_lines = symbol_lines(plain, needle), symbol_lines(scheduled, needle)
        assert plain_lines and all(line.split()[0] == "U" for line in plain_lines), plain
        assert scheduled_lines and all(line.split()[1] in ("W", "T") for line in scheduled_lines), scheduled
