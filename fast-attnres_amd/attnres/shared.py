"""Several reads of shared sources, with the source gradients summed inside
the backward kernels: ``SharedSources`` (a fixed list read by several
queries) and ``SourceBank`` (sources appended one at a time and read as
prefixes, the residual stream of a Full-schedule model).

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
received a gradient.  Each backward pass (autograd graph task) starts a
fresh sum, also after a pass that stopped short of the sources (e.g.
``torch.autograd.grad`` with respect to the queries only).  Eager mode only
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
from ._ops import _contiguous, _dq_workspace, _source_table, _stream, packed_forward_impl, sources_forward_impl
from ._sources import _EPS, _MAX_SOURCES, _MAX_WIDTH, check_packed, check_sources


def _pass_id() -> int:
    """The running backward pass: autograd's graph-task id (-1 outside one)."""
    return torch._C._current_graph_task_id()


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
        self._pass = -1
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
        current = _pass_id()
        accumulate = self._grads is not None and self._pass == current
        if not accumulate:  # first read of this pass (an earlier pass may have left its sums untaken)
            self._grads = [torch.empty(first.shape, device=device, dtype=torch.bfloat16) for _ in range(count)]
            self._pass = current
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
        return grads if self._pass == _pass_id() else None


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
        # always saved: the accumulating kernels read the refinement
        out, out_refine, logit, inv_rms, stats = sources_forward_impl(list(bank.sources), query, eps, scale, True)
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


class SourceBank:
    """Sources appended one at a time and read as prefixes: the residual stream
    of a Full-schedule model, where read i sees every source pushed before it.

        bank = SourceBank(capacity=2 * layers + 1)
        bank.push(embedding)                      # any float dtype, shape [..., D]
        x = bank.read(query_0)                    # attnres over the 1 source so far (BF16 out)
        bank.push(sublayer(x.to(dtype)))
        x = bank.read(query_1)                    # over 2 sources, ...

    Each source is converted to BF16 once, into slot i of one packed
    ``[capacity, ..., D]`` BF16 buffer, so a read is the prefix view
    ``buffer[:count]`` (no per-read conversion or stack).  In the backward every
    read adds its FP32 dv for its prefix into one FP32 ``[capacity, ..., D]``
    buffer in the kernel (``attnres_hip_packed_backward_accumulate_f32``: the
    first contribution to a slot writes it); slot i's sum is handed to source i
    (in its dtype) once every read that saw it has run its backward -- source
    i's autograd node produced the token those reads take as inputs.  The sums
    are FP32 without BF16 rounding of the per-read dv.  Eager mode only; one
    bank per forward pass.
    """

    def __init__(self, capacity: int) -> None:
        if isinstance(capacity, bool) or not isinstance(capacity, int) or not 1 <= capacity <= _MAX_SOURCES:
            raise ValueError(f"capacity must be an integer in 1..{_MAX_SOURCES}")
        self.capacity = capacity
        self._values: Tensor | None = None
        self._tokens: list[Tensor] = []
        self._grads: Tensor | None = None
        self._written: list[bool] = []
        self._pass = -1

    def __len__(self) -> int:
        return len(self._tokens)

    def push(self, source: Tensor) -> None:
        """Append ``source`` (``[..., D]``, any float dtype, on the GPU) as the next slot."""
        if not isinstance(source, Tensor) or not source.is_floating_point():
            raise TypeError("a source must be a floating-point tensor")
        if not source.is_cuda:
            raise RuntimeError("attnres requires CUDA (ROCm/HIP) device tensors")
        if len(self._tokens) == self.capacity:
            raise ValueError("the source bank is full")
        if self._values is None:
            if source.ndim < 1 or source.numel() == 0 or not 1 <= source.shape[-1] <= _MAX_WIDTH:
                raise ValueError("each source must have shape [...,D]")
            self._values = torch.empty((self.capacity, *source.shape), device=source.device, dtype=torch.bfloat16)
        elif source.shape != self._values.shape[1:] or source.device != self._values.device:
            raise ValueError("all source tensors must have the same logical shape and device")
        self._written.append(False)
        self._tokens.append(_Push.apply(self, len(self._tokens), source))

    def read(self, query: Tensor, *, count: int | None = None, eps: float = _EPS, scale: float = 1.0) -> Tensor:
        """``attnres(first `count` sources, query)`` (all pushed so far by default), BF16."""
        count = len(self._tokens) if count is None else count
        if isinstance(count, bool) or not isinstance(count, int) or not 1 <= count <= len(self._tokens):
            raise ValueError("count must select 1..len(bank) pushed sources")
        values = self._values[:count]
        eps_value, scale_value = check_packed(values, query, eps, scale)
        return _BankRead.apply(self, count, query, eps_value, scale_value, *self._tokens[:count])

    def _backward(self, count: int, query: Tensor, out: Tensor, out_refine: Tensor, grad_out: Tensor,
                  logit: Tensor, inv_rms: Tensor, stats: Tensor, scale: float) -> Tensor:
        lib = _native.load()
        values = self._values[:count]
        width = int(values.shape[-1])
        tokens = values[0].numel() // width
        rank = query.numel()
        device = values.device
        current = _pass_id()
        if self._pass != current:
            # first read of this pass: a fresh buffer, so sums handed out by an earlier pass
            # (views of its buffer) stay valid and a pass that stopped short leaves nothing behind
            self._grads = torch.empty(self._values.shape, device=device, dtype=torch.float32)
            self._written = [False] * len(self._written)
            self._pass = current
        flags = (ctypes.c_uint8 * count)(*[1 if written else 0 for written in self._written[:count]])
        grad_query = torch.empty((rank,), device=device, dtype=torch.bfloat16)
        workspace = _dq_workspace(lib, tokens, width, rank, device)
        grad_out = _contiguous(grad_out.to(torch.bfloat16))
        with torch.cuda.device(device):
            status = lib.attnres_hip_packed_backward_accumulate_f32(
                values.data_ptr(), tokens * width, width, count, tokens, width, query.data_ptr(), rank, scale,
                _contiguous(out).data_ptr(), _contiguous(out_refine).data_ptr(), grad_out.data_ptr(),
                _contiguous(logit).data_ptr(), _contiguous(inv_rms).data_ptr(), _contiguous(stats).data_ptr(),
                self._grads.data_ptr(), grad_query.data_ptr(), workspace.data_ptr(), workspace.numel(), flags,
                _stream(device))
        _native.check(status, "attnres source-bank backward")
        for slot in range(count):
            self._written[slot] = True
        return grad_query

    def _take(self, slot: int, dtype: torch.dtype) -> Tensor | None:
        """Slot `slot`'s FP32 sum in `dtype` (a view of this pass's buffer when FP32)."""
        if self._pass != _pass_id() or not self._written[slot]:
            return None
        self._written[slot] = False
        return self._grads[slot].to(dtype)


class _Push(torch.autograd.Function):
    @staticmethod
    def forward(ctx, bank: SourceBank, slot: int, source: Tensor) -> Tensor:
        bank._values[slot].copy_(source.detach())
        ctx.bank, ctx.slot, ctx.dtype = bank, slot, source.dtype
        return source.new_empty((0,))

    @staticmethod
    def backward(ctx, _token_grad):
        return None, None, ctx.bank._take(ctx.slot, ctx.dtype)


class _BankRead(torch.autograd.Function):
    @staticmethod
    def forward(ctx, bank: SourceBank, count: int, query: Tensor, eps: float, scale: float,
                *tokens: Tensor) -> Tensor:
        query = _contiguous(query)
        values = bank._values[:count]
        flat = values.reshape(count, -1, values.shape[-1])  # a view: the bank is contiguous
        out, out_refine, logit, inv_rms, stats = packed_forward_impl(flat, query, eps, scale, True)
        ctx.bank, ctx.count, ctx.scale = bank, count, scale
        ctx.token_device = tokens[0].device
        ctx.save_for_backward(query, out, out_refine, logit, inv_rms, stats)
        return out.reshape(values.shape[1:])

    @staticmethod
    def backward(ctx, grad_out):
        query, out, out_refine, logit, inv_rms, stats = ctx.saved_tensors
        grad_query = ctx.bank._backward(ctx.count, query, out, out_refine, grad_out, logit, inv_rms, stats,
                                        ctx.scale)
        empty = torch.empty((0,), device=ctx.token_device)
        return (None, None, grad_query if ctx.needs_input_grad[2] else None, None, None,
                *([empty] * ctx.count))


__all__ = ["SharedSources", "SourceBank"]
