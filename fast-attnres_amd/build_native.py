"""Build the gfx950 HIP library `attnres/_lib/libattnres_hip.so` in-tree.

    python fast-attnres_amd/build_native.py [-v]

Translation units, compiled in parallel by hipcc and linked into one shared
library:

* `csrc/attnres_hip.hip`: the C ABI (`include/attnres_hip.h`), host-side
  argument checks, dispatch and the dq reduction kernels;
* `csrc/attnres_kernels.hip`, once per row geometry (lanes per token group,
  16-byte chunks per lane) listed in GEOMETRIES.

Packed-FP32 VALU ops are disabled (``-target-feature -packed-fp32-ops``); the
compiler still emits ordinary FP32 FMAs, v_dot2_f32_bf16 and the gfx950 BF16
conversions.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
BUILD_DIR = HERE / "_build"
OUTPUT = HERE / "attnres" / "_lib" / "libattnres_hip.so"
ARCH = "gfx950"
# (lanes, chunks) per translation unit; must match ATTNRES_FOR_EACH_GEOMETRY
# in csrc/attnres_internal.h.
GEOMETRIES = ((16, 1), (32, 1), (32, 2), (32, 4), (64, 4), (64, 8), (256, 4))
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    for candidate in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found (ROCm is required to build the extension)")


def compile_commands() -> list[tuple[list[str], Path]]:
    """(hipcc command, object path) for every translation unit."""
    units = [(CSRC / "attnres_hip.hip", [], BUILD_DIR / "attnres_hip.o")]
    for lanes, chunks in GEOMETRIES:
        units.append((CSRC / "attnres_kernels.hip",
                      [f"-DATTNRES_LANES={lanes}", f"-DATTNRES_CHUNKS={chunks}"],
                      BUILD_DIR / f"attnres_kernels_g{lanes}_c{chunks}.o"))
    return [([hipcc(), f"--offload-arch={ARCH}", *FLAGS, *defines, f"-I{INCLUDE}", f"-I{CSRC}",
              "-c", str(source), "-o", str(obj)], obj)
            for source, defines, obj in units]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        errors = [line for line in result.stderr.splitlines()
                  if "packed-fp32-ops" not in line and line.strip()]
        raise RuntimeError("hipcc failed:\n" + "\n".join(errors))


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile the library (always, even if one exists) and return its path."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    OUTPUT.parent.mkdir(parents=True, exist_ok=True)
    commands = compile_commands()
    workers = jobs or min(len(commands), os.cpu_count() or 1, 16)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        for future in [pool.submit(_run, cmd, verbose) for cmd, _ in commands]:
            future.result()
    temporary = OUTPUT.with_suffix(".so.tmp")
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC",
          *[str(obj) for _, obj in commands], "-o", str(temporary)], verbose)
    os.replace(temporary, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(f"built {path}")
