"""Build the gfx950 HIP library `attnres/_lib/libattnres_hip.so` in-tree.

    python fast-attnres_amd/build_native.py [-v]

Translation units, compiled in parallel by hipcc and linked into one shared
library:

* `csrc/attnres_hip.hip`: the C ABI (`include/attnres_hip.h`), host-side
  argument checks, dispatch and the dq reduction kernels;
* `csrc/attnres_kernels.hip`, once per row geometry (lanes per token group,
  16-byte chunks per lane) listed in GEOMETRIES, the (64, 8) geometry in two
  parts (1: unmasked forwards and gather; 2: backwards and masked forwards)
  whose part 2 is scheduled with LLVM's iterative-minreg strategy, and once
  more for the (64, 4) token-block and whole-row key-resident backwards,
  scheduled with the max-ilp strategy;

and, against PyTorch's headers and libraries, the eager autograd nodes
`csrc/attnres_autograd.cpp` -> `attnres/_lib/_autograd.so` (host C++, no
device code; linked to the library above with an `$ORIGIN` run path).

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
# geometries built as two units (ATTNRES_UNIT_PART 1: forwards and gather;
# 2: backwards, and for (64, 8) the masked forwards), with extra flags for
# part 2: the (64, 8) backwards (streaming, key-resident, recompute) are
# 0.4-1.2% faster with the iterative-minreg scheduler and its masked forwards
# 1-2%, its unmasked forwards are not (MI355X, backward us, default -> minreg:
# S = 16, D = 4096, R = 1024: 777.7 / 786.7 -> 772.7 / 777.5; S = 25, R = D:
# 1287.9 -> 1282.8; S = 25, R = 1024: 1277.8 -> 1267.3; forwards: see
# launch_fwd)
SPLIT_GEOMETRIES = {(64, 8): ["-mllvm", "-amdgpu-sched-strategy=iterative-minreg"]}
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
AUTOGRAD_SOURCE = CSRC / "attnres_autograd.cpp"
AUTOGRAD_OBJECT = BUILD_DIR / "attnres_autograd.o"
AUTOGRAD_OUTPUT = HERE / "attnres" / "_lib" / "_autograd.so"
ROCM_INCLUDE = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "include"


def hipcc() -> str:
    for candidate in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found (ROCm is required to build the extension)")


def compile_commands() -> list[tuple[list[str], Path]]:
    """(hipcc command, object path) for every translation unit."""
    units = [(CSRC / "attnres_hip.hip", [], BUILD_DIR / "attnres_hip.o")]
    for lanes, chunks in GEOMETRIES:
        defines = [f"-DATTNRES_LANES={lanes}", f"-DATTNRES_CHUNKS={chunks}"]
        stem = f"attnres_kernels_g{lanes}_c{chunks}"
        if (lanes, chunks) in SPLIT_GEOMETRIES:
            units.append((CSRC / "attnres_kernels.hip", [*defines, "-DATTNRES_UNIT_PART=1"],
                          BUILD_DIR / f"{stem}_part1.o"))
            units.append((CSRC / "attnres_kernels.hip",
                          [*defines, "-DATTNRES_UNIT_PART=2", *SPLIT_GEOMETRIES[(lanes, chunks)]],
                          BUILD_DIR / f"{stem}_part2.o"))
        else:
            units.append((CSRC / "attnres_kernels.hip", defines, BUILD_DIR / f"{stem}.o"))
    # the (64, 4) token-block and whole-row key-resident backwards, with LLVM's
    # max-ilp machine scheduler (1-1.5% faster there, slower for the forwards;
    # see launch_bwd_block and launch_bwd_keyres_chunks)
    units.append((CSRC / "attnres_kernels.hip",
                  ["-DATTNRES_MAX_ILP_UNIT", "-mllvm", "-amdgpu-sched-strategy=max-ilp"],
                  BUILD_DIR / "attnres_kernels_max_ilp.o"))
    return [([hipcc(), f"--offload-arch={ARCH}", *FLAGS, *defines, f"-I{INCLUDE}", f"-I{CSRC}",
              "-c", str(source), "-o", str(obj)], obj)
            for source, defines, obj in units]


def _torch_flags() -> tuple[list[str], list[str]]:
    """Compile and link flags of a PyTorch C++ extension module named
    `_autograd` (the same ones `torch.utils.cpp_extension` uses on ROCm)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    compile_flags = ["-O2", "-std=c++17", "-fPIC", "-DTORCH_EXTENSION_NAME=_autograd", "-DTORCH_API_INCLUDE_EXTENSION_H",
                     f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}", "-D__HIP_PLATFORM_AMD__=1",
                     "-DUSE_ROCM=1", f"-I{INCLUDE}", f"-I{ROCM_INCLUDE}"]
    for path in (*cpp_extension.include_paths(), sysconfig.get_paths()["include"]):
        compile_flags += ["-isystem", path]
    link_flags = [f"-L{lib}" for lib in cpp_extension.library_paths()]
    link_flags += ["-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch", "-ltorch_python"]
    return compile_flags, link_flags


def cxx() -> str:
    for candidate in (os.environ.get("CXX"), shutil.which("c++"), shutil.which("g++")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("no C++ compiler found for the autograd extension")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        errors = [line for line in result.stderr.splitlines()
                  if "packed-fp32-ops" not in line and line.strip()]
        raise RuntimeError(f"{Path(cmd[0]).name} failed:\n" + "\n".join(errors))


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile the library (always, even if one exists) and return its path."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    OUTPUT.parent.mkdir(parents=True, exist_ok=True)
    commands = compile_commands()
    compile_flags, link_flags = _torch_flags()
    autograd = [cxx(), *compile_flags, "-c", str(AUTOGRAD_SOURCE), "-o", str(AUTOGRAD_OBJECT)]
    workers = jobs or min(len(commands) + 1, os.cpu_count() or 1, 16)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        futures = [pool.submit(_run, autograd, verbose)]  # the longest unit (PyTorch headers) first
        futures += [pool.submit(_run, cmd, verbose) for cmd, _ in commands]
        for future in futures:
            future.result()
    temporary = OUTPUT.with_suffix(".so.tmp")
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC",
          *[str(obj) for _, obj in commands], "-o", str(temporary)], verbose)
    os.replace(temporary, OUTPUT)
    temporary = AUTOGRAD_OUTPUT.with_suffix(".so.tmp")
    _run([cxx(), "-shared", str(AUTOGRAD_OBJECT), "-o", str(temporary), f"-L{OUTPUT.parent}", "-lattnres_hip",
          "-Wl,-rpath,$ORIGIN", *link_flags], verbose)
    os.replace(temporary, AUTOGRAD_OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(f"built {path}")
