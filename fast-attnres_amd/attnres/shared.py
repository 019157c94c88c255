"""Several reads of one ordered list of sources, with the source gradients
summed inside the backward kernels.

Autograd sums the gradients of a tensor used by several reads with separate
add kernels after each read's backward: for a source of N x D BF16 elements
every further read costs a pass that reads two gradient buffers and writes a
third.  ``SharedSources`` instead gives every read of the same sources one set
of gradient buffers: the first backward writes them, each later backward
adds its dv in the kernel (``attnres_hip_sources_backward_accumulate``: one
extra read of the buffer, no add kernel), and the sources receive the sums
once every read's backward has run.

    bank = SharedSources(sources)             # ordered list of BF16 [..., D] tensors
    out_a = bank.read(query_a)                # same result as attnres(sources, query_a)
    out_b = bank.read(query_b, scale=0.5)
    loss(out_a, out_b).backward()             # sources get d/d(source) summed over both reads

The ordering uses a token: the reads take a zero-size tensor produced from
the sources by one autograd node, so autograd runs that node's backward --
which hands the summed buffers to the sources -- only after every read that
received a gradient.  Each backward pass starts a fresh sum.  Eager mode only
(the bank holds state between the reads' backward calls); first-order
gradients, like the read itself.

The reference has no counterpart: its shared sources' gradients are summed
by autograd (the Block-schedule reads of `benchmarks/model.py:306-338`).
"""

from __future__ import annotations

import ctypes
from typing import Sequence

import torch
from torch import Tensor

from . import _native
from ._ops import _contiguous, _dq_workspace, _source_table, _stream, sources_forward
from ._sources import _EPS, check_sources


class SharedSources:
    """An ordered list of BF16 sources read by several queries (see module doc)."""

    def __init__(self, sources: Sequence[Tensor]) -> None:
        if not isinstance(sources, (list, tuple)) or not sources:
            raise TypeError("sources must be a non-empty list or tuple of tensors")
        first = sources[0]
        if not isinstance(first, Tensor):
            raise TypeError("values must contain only tensors")
        probe = torch.empty(1, device=first.device, dtype=torch.bfloat16)
        checked, _, _ = check_sources(tuple(sources), probe, _EPS, 1.0)
        if not checked[0].is_cuda:
            raise RuntimeError("attnres requires CUDA (ROCm/HIP) device tensors")
        self.sources = checked
        self._grads: list[Tensor] | None = None
        self._token = _Gather.apply(self, *checked)

    def __len__(self) -> int:
        return len(self.sources)

    def read(self, query: Tensor, *, eps: float = _EPS, scale: float = 1.0) -> Tensor:
        """``attnres(sources, query, eps=eps, scale=scale)`` with the source
        gradients summed in the kernels across this bank's reads."""
        _, eps_value, scale_value = check_sources(self.sources, query, eps, scale)
        return _Read.apply(self, self._token, query, eps_value, scale_value)

    # ------------------------------------------------------------ backward

    def _backward(self, query: Tensor, out: Tensor, out_refine: Tensor, grad_out: Tensor,
                  logit: Tensor, inv_rms: Tensor, stats: Tensor, scale: float) -> Tensor:
        """One read's backward: dv into the shared buffers (written by the
        first read of this pass, accumulated by the others); returns dq."""
        lib = _native.load()
        first = self.sources[0]
        count, width = len(self.sources), int(first.shape[-1])
        tokens = out.numel() // width
        rank = query.numel()
        device = first.device
        accumulate = self._grads is not None
        if self._grads is None:
            self._grads = [torch.empty(first.shape, device=device, dtype=torch.bfloat16) for _ in range(count)]
        flags = (ctypes.c_uint8 * count)(*([1 if accumulate else 0] * count))
        grad_pointers = (ctypes.c_void_p * count)(*[grad.data_ptr() for grad in self._grads])
        prepared, pointers, row_strides = _source_table(list(self.sources))
        grad_query = torch.empty((rank,), device=device, dtype=torch.bfloat16)
        workspace = _dq_workspace(lib, tokens, width, rank, device)
        grad_out = _contiguous(grad_out.to(torch.bfloat16))
        with torch.cuda.device(device):
            status = lib.attnres_hip_sources_backward_accumulate(
                pointers, row_strides, count, tokens, width, query.data_ptr(), rank, scale,
                _contiguous(out).data_ptr(), _contiguous(out_refine).data_ptr(), grad_out.data_ptr(),
                _contiguous(logit).data_ptr(), _contiguous(inv_rms).data_ptr(), _contiguous(stats).data_ptr(),
                grad_pointers, grad_query.data_ptr(), workspace.data_ptr(), workspace.numel(), flags,
                _stream(device))
        del prepared
        _native.check(status, "attnres shared-source backward")
        return grad_query

    def _take_grads(self) -> list[Tensor] | None:
        grads, self._grads = self._grads, None
        return grads


class _Gather(torch.autograd.Function):
    """The bank's autograd node: its backward hands the summed gradients to
    the sources after every read's backward."""

    @staticmethod
    def forward(ctx, bank: SharedSources, *sources: Tensor) -> Tensor:
        ctx.bank = bank
        return sources[0].new_empty((0,))

    @staticmethod
    def backward(ctx, _token_grad):
        grads = ctx.bank._take_grads()
        count = len(ctx.bank.sources)
        if grads is None:
            return (None,) * (count + 1)
        return (None, *[g if need else None for g, need in zip(grads, ctx.needs_input_grad[1:])])


class _Read(torch.autograd.Function):
    @staticmethod
    def forward(ctx, bank: SharedSources, token: Tensor, query: Tensor, eps: float, scale: float) -> Tensor:
        query = _contiguous(query)
        out, out_refine, logit, inv_rms, stats = sources_forward(list(bank.sources), query, eps, scale)
        ctx.bank = bank
        ctx.scale = scale
        ctx.token_device = token.device
        ctx.save_for_backward(query, out, out_refine, logit, inv_rms, stats)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        query, out, out_refine, logit, inv_rms, stats = ctx.saved_tensors
        grad_query = ctx.bank._backward(query, out, out_refine, grad_out, logit, inv_rms, stats, ctx.scale)
        token_grad = torch.empty((0,), device=ctx.token_device)
        return None, token_grad, grad_query if ctx.needs_input_grad[2] else None, None, None


__all__ = ["SharedSources"]
