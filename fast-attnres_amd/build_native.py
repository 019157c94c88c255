"""Build the gfx950 HIP library `attnres/_lib/libattnres_hip.so` in-tree.

    python fast-attnres_amd/build_native.py

Runs hipcc once on `csrc/attnres_hip.hip` (kernels and C ABI in one
translation unit).  Packed-FP32 VALU ops are disabled
(``-target-feature -packed-fp32-ops``); the compiler still emits ordinary
FP32 FMAs and the gfx950 BF16 conversions.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SOURCE = HERE / "csrc" / "attnres_hip.hip"
INCLUDE = HERE.parent / "include"
OUTPUT = HERE / "attnres" / "_lib" / "libattnres_hip.so"
ARCH = "gfx950"


def hipcc() -> str:
    for candidate in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found (ROCm is required to build the extension)")


def command(output: Path = OUTPUT) -> list[str]:
    return [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{INCLUDE}", str(SOURCE), "-o", str(output),
    ]


def build(verbose: bool = False) -> Path:
    """Compile the library (always, even if one exists) and return its path."""
    OUTPUT.parent.mkdir(parents=True, exist_ok=True)
    temporary = OUTPUT.with_suffix(".so.tmp")
    cmd = command(temporary)
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    errors = [line for line in result.stderr.splitlines()
              if "packed-fp32-ops" not in line and line.strip()]
    if result.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(errors))
    os.replace(temporary, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(f"built {path}")
