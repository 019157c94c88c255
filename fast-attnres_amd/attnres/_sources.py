"""Argument validation shared by the packed and source-list containers.

Behaviour (exception classes, message substrings, check order) follows the
reference's `src/attnres/api.py:9-27` and `src/attnres/_sources.py:16-93`,
so code written against the reference sees the same errors.  Nothing here
copies, stacks or makes tensors contiguous.
"""

from __future__ import annotations

import math
from numbers import Real

import torch

_EPS = 2**-23
_MAX_SOURCES = 129
_MAX_WIDTH = 8192


def check_scalar(value, name: str, *, positive: bool = False) -> float:
    """Accept real Python/NumPy scalars only (not bool, str or tensors)."""
    if type(value) is not float and (isinstance(value, bool) or not isinstance(value, Real)):
        raise TypeError(f"{name} must be a real scalar")
    number = float(value)
    if not math.isfinite(number):
        raise ValueError(f"{name} must be finite" + (" and positive" if positive else ""))
    if positive and number <= 0.0:
        raise ValueError(f"{name} must be finite and positive")
    return number


def check_packed(values: torch.Tensor, query, eps, scale) -> tuple[float, float]:
    """Validate a packed ``[S, ..., D]`` call (reference `api.py:9-27`).

    Device placement is checked last so that numeric options are rejected
    before a CPU tensor is (reference `tests/test_api.py:53-60`).
    """
    if not isinstance(query, torch.Tensor):
        raise TypeError("query must be a tensor")
    shape = values.shape
    if len(shape) < 2 or query.ndim != 1:
        raise ValueError("expected values [S,...,D] and query [R]")
    if not 1 <= shape[0] <= _MAX_SOURCES or not 1 <= shape[-1] <= _MAX_WIDTH:
        raise ValueError(
            f"supported envelope is 1<=S<={_MAX_SOURCES} and 1<=D<={_MAX_WIDTH}")
    if min(shape) < 1 or not 1 <= query.numel() <= shape[-1]:
        raise ValueError("dimensions must be positive and 1<=R<=D")
    if values.dtype != torch.bfloat16:
        raise TypeError("values must use BF16 storage")
    if query.dtype != torch.bfloat16:
        raise TypeError("query must use BF16 storage")
    if query.device != values.device:
        raise TypeError("query must be on the values device")
    eps_value = check_scalar(eps, "eps", positive=True)
    scale_value = check_scalar(scale, "scale")
    if not values.is_cuda:
        raise RuntimeError("attnres requires CUDA (ROCm/HIP) device tensors")
    return eps_value, scale_value


def check_sources(values, query, eps, scale) -> tuple[tuple[torch.Tensor, ...], float, float]:
    """Validate an ordered list/tuple of ``S`` sources ``[..., D]``.

    Mirrors reference `_sources.validate_sources` (`_sources.py:37-93`):
    returns the caller's own tensor objects in order (a repeated source stays
    repeated), never a packed copy.
    """
    if not isinstance(query, torch.Tensor):
        raise TypeError("query must be a tensor")
    if query.ndim != 1:
        raise ValueError("query must have 1 dimensions")
    if any(int(size) < 1 for size in query.shape):
        raise ValueError("query dimensions must be positive")
    if query.dtype != torch.bfloat16:
        raise TypeError("query must use BF16 storage")
    if not isinstance(values, (list, tuple)):
        raise TypeError("values must be a tensor or a list/tuple of tensors")
    sources = tuple(values)
    if not 1 <= len(sources) <= _MAX_SOURCES:
        raise ValueError(f"supported source envelope is 1<=S<={_MAX_SOURCES}")
    if any(not isinstance(source, torch.Tensor) for source in sources):
        raise TypeError("values must contain only tensors")
    first = sources[0]
    if first.ndim < 1:
        raise ValueError("each source must have shape [...,D]")
    if any(int(size) < 1 for size in first.shape):
        raise ValueError("source dimensions must be positive")
    width = int(first.shape[-1])
    if not 1 <= width <= _MAX_WIDTH:
        raise ValueError(f"supported value envelope is 1<=D<={_MAX_WIDTH}")
    if first.dtype != torch.bfloat16:
        raise TypeError("values must use BF16 storage")
    if query.device != first.device:
        raise TypeError("query must be on the values device")
    for index, source in enumerate(sources):
        if source.ndim < 1:
            raise ValueError(f"source {index} must have shape [...,D]")
        if tuple(source.shape) != tuple(first.shape):
            raise ValueError("all source tensors must have the same logical shape")
        if source.dtype != first.dtype or source.device != first.device:
            raise TypeError("all source tensors must match the first source dtype/device")
    if not 1 <= int(query.shape[-1]) <= width:
        raise ValueError("query rank must satisfy 1<=R<=D")
    eps_value = check_scalar(eps, "eps", positive=True)
    scale_value = check_scalar(scale, "scale")
    return sources, eps_value, scale_value


def check_query(query, width: int, device: torch.device, eps, scale) -> tuple[float, float]:
    """Validate the query and options of a read over sources already known
    to be valid BF16 ``[..., D]`` rows on ``device`` (a source bank's own
    slots); the query checks and messages are those of ``check_sources``."""
    if not isinstance(query, torch.Tensor):
        raise TypeError("query must be a tensor")
    if query.ndim != 1:
        raise ValueError("query must have 1 dimensions")
    if query.dtype != torch.bfloat16:
        raise TypeError("query must use BF16 storage")
    if query.device != device:
        raise TypeError("query must be on the values device")
    if not 1 <= int(query.shape[0]) <= width:
        raise ValueError("query rank must satisfy 1<=R<=D")
    return check_scalar(eps, "eps", positive=True), check_scalar(scale, "scale")


__all__ = ["check_packed", "check_query", "check_scalar", "check_sources"]
