"""Trainable static query for AttnRes reads.

API parity with the reference's `src/attnres/modules.py:22-38`
(`LearnedQuery(rank, *, init_std=0.02)`, BF16 parameter, ``forward()``
returns it as BF16).
"""

from __future__ import annotations

import math
import operator

import torch
from torch import nn


def _as_index(value, name: str) -> int:
    if isinstance(value, bool):
        raise TypeError(f"{name} must be an integer")
    try:
        return operator.index(value)
    except TypeError as error:
        raise TypeError(f"{name} must be an integer") from error


class LearnedQuery(nn.Module):
    """One learned BF16 query vector ``[rank]`` for an AttnRes read."""

    def __init__(self, rank: int, *, init_std: float = 0.02) -> None:
        super().__init__()
        rank = _as_index(rank, "rank")
        init_std = float(init_std)
        if rank < 1:
            raise ValueError("rank must be positive")
        if not (math.isfinite(init_std) and init_std > 0):
            raise ValueError("init_std must be finite and positive")
        self.query = nn.Parameter(torch.empty(rank, dtype=torch.bfloat16))
        with torch.no_grad():
            self.query.normal_(mean=0.0, std=init_std)

    def forward(self) -> torch.Tensor:
        return self.query.to(dtype=torch.bfloat16)


__all__ = ["LearnedQuery"]
