"""Public functional entry point: ``attnres(values, query, *, eps, scale)``.

Same signature, container forms and error behaviour as the reference's
`src/attnres/api.py:30-62`.  Device work runs in hand-written gfx950 HIP
kernels reached through the C ABI in `include/attnres_hip.h`; the kernel
modules are imported lazily so CPU-only installs can validate arguments
without loading the native library.
"""

from __future__ import annotations

import torch
from torch import Tensor

from ._sources import _EPS, check_packed, check_sources


def attnres(
    values: Tensor | list[Tensor] | tuple[Tensor, ...],
    query: Tensor,
    *,
    eps: float = _EPS,
    scale: float = 1.0,
) -> Tensor:
    """Mix S depth sources with a static query over implicit tail keys.

    ``values`` is a packed ``[S, ..., D]`` BF16 tensor or an ordered
    list/tuple of ``S`` BF16 tensors ``[..., D]``.  ``query`` is BF16
    ``[R]``, ``1 <= R <= D``; the key of every source is its last ``R``
    coordinates, RMS-normalised with ``eps``.  The softmax over sources of
    ``scale * <key, query>`` weights the full-width values; the result is a
    BF16 ``[..., D]`` tensor.  ``R == D`` is standard AttnRes, ``R < D`` is
    sliced low-rank AttnRes.  Internal arithmetic is FP32; first-order
    gradients flow to values and query.
    """
    if isinstance(values, torch.Tensor):
        eps_value, scale_value = check_packed(values, query, eps, scale)
        from ._ops import packed_attnres

        return packed_attnres(values, query, eps_value, scale_value)

    sources, eps_value, scale_value = check_sources(values, query, eps, scale)
    if not sources[0].is_cuda:
        raise RuntimeError("attnres requires CUDA (ROCm/HIP) device tensors")
    from ._ops import sources_attnres

    return sources_attnres(sources, query, eps_value, scale_value)


__all__ = ["attnres"]
