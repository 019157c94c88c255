"""ctypes binding of the C ABI in `include/attnres_hip.h`, and the loader of
the eager autograd nodes.

The shared library `_lib/libattnres_hip.so` is built in-tree from
`csrc/attnres_hip.hip` by `build_native.py` (hipcc, gfx950), and so is
`_lib/_autograd.so` (`csrc/attnres_autograd.cpp`, a PyTorch C++ extension
linked to that library).  There is no fallback: if either is missing or does
not load, every operator call raises, so a GPU run can never silently take
another path.
"""

from __future__ import annotations

import ctypes
import importlib.util
import threading
from pathlib import Path
from types import ModuleType

LIBRARY_NAME = "libattnres_hip.so"
LIBRARY_PATH = Path(__file__).resolve().parent / "_lib" / LIBRARY_NAME
AUTOGRAD_PATH = Path(__file__).resolve().parent / "_lib" / "_autograd.so"

# Status codes of `enum attnres_status`.
OK = 0
ERR_NULL_POINTER = 1
ERR_SHAPE = 2
ERR_STRIDE = 3
ERR_SCALAR = 4
ERR_WORKSPACE = 5
ERR_LAUNCH = 6

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# name -> (restype, argtypes); one entry per declaration in attnres_hip.h.
SIGNATURES = {
    "attnres_hip_version": (ctypes.c_char_p, []),
    "attnres_hip_last_error": (ctypes.c_char_p, []),
    "attnres_hip_saves_refinement": (ctypes.c_int, [_i64]),
    "attnres_hip_saves_refinement_for": (ctypes.c_int, [_i64, _i64, _i64]),
    "attnres_hip_dq_workspace_elems": (_i64, [_i64, _i64, _i64]),
    "attnres_hip_packed_forward": (ctypes.c_int, [
        _c_void_p, _i64, _i64, _i64, _i64, _i64, _c_void_p, _i64, _f32, _f32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "attnres_hip_packed_backward": (ctypes.c_int, [
        _c_void_p, _i64, _i64, _i64, _i64, _i64, _c_void_p, _i64, _f32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p]),
    "attnres_hip_packed_backward_noalloc": (ctypes.c_int, [
        _c_void_p, _i64, _i64, _i64, _i64, _i64, _c_void_p, _i64, _f32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _c_void_p, _c_void_p, _c_void_p]),
    "attnres_hip_sources_forward": (ctypes.c_int, [
        _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _f32, _f32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "attnres_hip_sources_backward": (ctypes.c_int, [
        _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _f32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p]),
    "attnres_hip_packed_backward_accumulate": (ctypes.c_int, [
        _c_void_p, _i64, _i64, _i64, _i64, _i64, _c_void_p, _i64, _f32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p]),
    "attnres_hip_packed_backward_accumulate_f32": (ctypes.c_int, [
        _c_void_p, _i64, _i64, _i64, _i64, _i64, _c_void_p, _i64, _f32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p]),
    "attnres_hip_sources_backward_accumulate": (ctypes.c_int, [
        _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _f32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p]),
    "attnres_hip_sources_backward_accumulate_f32": (ctypes.c_int, [
        _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _f32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p]),
    "attnres_hip_packed_backward_coef": (ctypes.c_int, [
        _c_void_p, _i64, _i64, _i64, _i64, _i64, _c_void_p, _i64, _f32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p]),
    "attnres_hip_sources_backward_coef": (ctypes.c_int, [
        _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _f32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p]),
    "attnres_hip_bank_gather": (ctypes.c_int, [_c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _c_void_p, ctypes.c_int,
                                               ctypes.c_int, _c_void_p]),
    "attnres_hip_partial_sum": (ctypes.c_int, [_c_void_p, _c_void_p, ctypes.c_int, _i64, _c_void_p, _c_void_p,
                                               _c_void_p]),
}

_lock = threading.Lock()
_library: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load (once) and return the native library, or raise RuntimeError."""
    global _library
    if _library is not None:
        return _library
    with _lock:
        if _library is None:
            path = LIBRARY_PATH
            if not path.is_file():
                raise RuntimeError(
                    f"attnres HIP extension not built: {path} is missing "
                    "(run `python fast-attnres_amd/build_native.py`)")
            try:
                library = ctypes.CDLL(str(path))
            except OSError as error:
                raise RuntimeError(f"attnres HIP extension failed to load: {error}") from error
            for name, (restype, argtypes) in SIGNATURES.items():
                function = getattr(library, name)
                function.restype = restype
                function.argtypes = argtypes
            _library = library
    return _library


_autograd: ModuleType | None = None


def load_autograd() -> ModuleType:
    """Load (once) and return the eager autograd nodes (`packed_read`,
    `sources_read`), or raise RuntimeError.  The HIP library is loaded first:
    the module links it, and both then share one copy of its state."""
    global _autograd
    if _autograd is not None:
        return _autograd
    load()
    with _lock:
        if _autograd is None:
            if not AUTOGRAD_PATH.is_file():
                raise RuntimeError(
                    f"attnres autograd extension not built: {AUTOGRAD_PATH} is missing "
                    "(run `python fast-attnres_amd/build_native.py`)")
            import torch  # noqa: F401  (the module links PyTorch's libraries)

            spec = importlib.util.spec_from_file_location("attnres._autograd", AUTOGRAD_PATH)
            try:
                module = importlib.util.module_from_spec(spec)
                spec.loader.exec_module(module)
            except ImportError as error:
                raise RuntimeError(f"attnres autograd extension failed to load: {error}") from error
            _autograd = module
    return _autograd


def check(status: int, what: str) -> None:
    """Raise for a non-OK status, with the library's own message."""
    if status == OK:
        return
    message = (load().attnres_hip_last_error() or b"").decode(errors="replace")
    if status in (ERR_SHAPE, ERR_STRIDE, ERR_SCALAR, ERR_WORKSPACE):
        raise ValueError(f"{what}: {message}")
    raise RuntimeError(f"{what}: {message} (status {status})")


__all__ = ["AUTOGRAD_PATH", "LIBRARY_PATH", "SIGNATURES", "check", "load", "load_autograd"]
