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

The autograd nodes hold the buffers and the per-pass bookkeeping in a state
object that holds no token, so the buffers are freed with the graph, without
waiting for Python's cycle collector (a node that held the bank itself would
close a cycle bank -> token -> node -> bank).

The reference has no counterpart: its shared sources' gradients are summed
by autograd (the Block-schedule reads of `benchmarks/model.py:306-338`).
"""

from __future__ import annotations

import ctypes
from array import array
from typing import Sequence

import torch
from torch import Tensor

from . import _native
from ._ops import (_contiguous, _dq_workspace, _on_device, _source_table, _stream, packed_forward_impl,
                   sources_forward_impl)
from ._sources import _EPS, _MAX_SOURCES, _MAX_WIDTH, check_query, check_sources

_DTYPE_F32, _DTYPE_BF16 = 0, 1  # attnres_hip.h ATTNRES_DTYPE_*
_MAX_GATHER_READS = 48  # attnres_hip.h ATTNRES_MAX_GATHER_READS
# A BF16 source's gathered gradient is stored as BF16 by the gather itself
# when one launch covers its reads (else FP32, converted afterwards).
_BF16_GATHER = True


class _GatherRead(ctypes.Structure):
    """attnres_hip.h ``attnres_gather_read``."""

    _fields_ = [("grad_out", ctypes.c_void_p), ("query_row", ctypes.c_void_p), ("coef", ctypes.c_void_p),
                ("n_sources", ctypes.c_int64), ("position", ctypes.c_int64), ("rank", ctypes.c_int64)]


# A gather's read table is passed as an int64 array of the same layout (six
# 8-byte fields per read), filled without per-field ctypes attribute writes.
assert ctypes.sizeof(_GatherRead) == 6 * 8 and _GatherRead.position.offset == 4 * 8


_GRAPH_TASK_ID = getattr(torch._C, "_current_graph_task_id", None)


def _pass_id() -> int:
    """The running backward pass: autograd's graph-task id (-1 outside one).
    No public torch API tells one backward pass from the next; a torch build
    without this query cannot run shared-source reads and says so."""
    if _GRAPH_TASK_ID is None:
        raise RuntimeError("SharedSources and SourceBank need torch._C._current_graph_task_id, "
                           "which this torch build does not provide")
    return _GRAPH_TASK_ID()


class _SharedState:
    """The sources and this pass's gradient sums, used by the nodes of a
    ``SharedSources``."""

    def __init__(self, sources: tuple[Tensor, ...]) -> None:
        self.sources = sources
        self._grads: list[Tensor] | None = None
        self._pass = -1

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
        with _on_device(device):
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
        self._state = _SharedState(checked)
        self._token = _Gather.apply(self._state, *checked)

    @property
    def sources(self) -> tuple[Tensor, ...]:
        return self._state.sources

    def __len__(self) -> int:
        return len(self.sources)

    def read(self, query: Tensor, *, eps: float = _EPS, scale: float = 1.0) -> Tensor:
        """``attnres(sources, query, eps=eps, scale=scale)`` with the source
        gradients summed in the kernels across this bank's reads."""
        _, eps_value, scale_value = check_sources(self.sources, query, eps, scale)
        if not _needs_gradients(query, self._token):  # the forward alone: nothing saved
            return sources_forward_impl(list(self.sources), _contiguous(query), eps_value, scale_value, False,
                                        pooled=True)[0]
        return _Read.apply(self._state, self._token, query, eps_value, scale_value)


class _Gather(torch.autograd.Function):
    """The bank's autograd node: its backward hands the summed gradients to
    the sources after every read's backward."""

    @staticmethod
    def forward(ctx, bank: _SharedState, *sources: Tensor) -> Tensor:
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
    def forward(ctx, bank: _SharedState, token: Tensor, query: Tensor, eps: float, scale: float) -> Tensor:
        query = _contiguous(query)
        # always saved: the accumulating kernels read the refinement
        out, out_refine, logit, inv_rms, stats = sources_forward_impl(list(bank.sources), query, eps, scale, True,
                                                                      pooled=True)
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


class _BankState:
    """The slot buffer and this pass's gradient bookkeeping, used by the
    nodes of a ``SourceBank``."""

    def __init__(self, capacity: int, gradients: str) -> None:
        self.capacity = capacity
        self.gradients = gradients
        self._values: Tensor | None = None
        self._flat: Tensor | None = None  # _values viewed as [capacity, tokens, width]
        self._width = self._tokens = self._base = 0
        self._device: torch.device | None = None
        self._grads: Tensor | None = None
        self._written: list[bool] = [False] * capacity
        self._pending: list[list[tuple[tuple, int]]] = [[] for _ in range(capacity)]
        self._pass = -1

    def _allocate(self, source: Tensor) -> None:
        self._values = torch.empty((self.capacity, *source.shape), device=source.device, dtype=torch.bfloat16)
        self._width = int(source.shape[-1])
        self._tokens = source.numel() // self._width
        self._device = source.device
        self._flat = self._values.view(self.capacity, self._tokens, self._width)
        self._base = self._values.data_ptr()

    def _slot_ptr(self, slot: int) -> int:
        """Device address of slot ``slot``'s BF16 rows (the buffer is contiguous)."""
        return self._base + slot * self._tokens * self._width * 2

    def _sources(self, slots: tuple[int, ...]) -> list[Tensor]:
        return [self._values[i] for i in slots]

    def _prefix(self, slots: tuple[int, ...]) -> bool:
        return slots == tuple(range(len(slots)))

    def _backward(self, slots: tuple[int, ...], query: Tensor, out: Tensor, out_refine: Tensor, grad_out: Tensor,
                  logit: Tensor, inv_rms: Tensor, stats: Tensor, scale: float) -> Tensor:
        current = _pass_id()
        if self._pass != current:
            # first read of this pass: nothing left from an earlier pass (one that stopped short
            # of the sources) is used, and sums handed out earlier stay valid (fresh buffers)
            self._grads = None
            self._written = [False] * self.capacity
            self._pending = [[] for _ in range(self.capacity)]
            self._pass = current
        if self.gradients == "gather":
            return self._backward_coef(slots, query, out, out_refine, grad_out, logit, inv_rms, stats, scale)
        lib = _native.load()
        count = len(slots)
        width, tokens, device = self._width, self._tokens, self._device
        rank = query.numel()
        if self._grads is None:
            self._grads = torch.empty(self._values.shape, device=device, dtype=torch.float32)
        flags = (ctypes.c_uint8 * count)(*[1 if self._written[i] else 0 for i in slots])
        grad_query = torch.empty((rank,), device=device, dtype=torch.bfloat16)
        workspace = _dq_workspace(lib, tokens, width, rank, device)
        grad_out = _contiguous(grad_out.to(torch.bfloat16))
        saved = (_contiguous(out).data_ptr(), _contiguous(out_refine).data_ptr(), grad_out.data_ptr(),
                 _contiguous(logit).data_ptr(), _contiguous(inv_rms).data_ptr(), _contiguous(stats).data_ptr())
        with _on_device(device):
            if self._prefix(slots):
                status = lib.attnres_hip_packed_backward_accumulate_f32(
                    self._values.data_ptr(), tokens * width, width, count, tokens, width, query.data_ptr(), rank,
                    scale, *saved, self._grads.data_ptr(), grad_query.data_ptr(), workspace.data_ptr(),
                    workspace.numel(), flags, _stream(device))
            else:
                pointers = (ctypes.c_void_p * count)(*[self._slot_ptr(i) for i in slots])
                strides = (ctypes.c_int64 * count)(*([width] * count))
                sums = (ctypes.c_void_p * count)(*[self._grads[i].data_ptr() for i in slots])
                status = lib.attnres_hip_sources_backward_accumulate_f32(
                    pointers, strides, count, tokens, width, query.data_ptr(), rank, scale, *saved, sums,
                    grad_query.data_ptr(), workspace.data_ptr(), workspace.numel(), flags, _stream(device))
        _native.check(status, "attnres source-bank backward")
        for i in slots:
            self._written[i] = True
        return grad_query

    def _backward_coef(self, slots: tuple[int, ...], query: Tensor, out: Tensor, out_refine: Tensor,
                       grad_out: Tensor, logit: Tensor, inv_rms: Tensor, stats: Tensor, scale: float) -> Tensor:
        """First stage of the gathered gradients: dq and the dv coefficients now;
        the read's dO and coefficients are kept for the slots' gathers."""
        lib = _native.load()
        count = len(slots)
        width, tokens, device = self._width, self._tokens, self._device
        rank = query.numel()
        grad_query = torch.empty((rank,), device=device, dtype=torch.bfloat16)
        coef = torch.empty((3, count, tokens), device=device, dtype=torch.float32)
        workspace = _dq_workspace(lib, tokens, width, rank, device)
        grad_out = _contiguous(grad_out.to(torch.bfloat16))
        saved = (_contiguous(out).data_ptr(), _contiguous(out_refine).data_ptr(), grad_out.data_ptr(),
                 _contiguous(logit).data_ptr(), _contiguous(inv_rms).data_ptr(), _contiguous(stats).data_ptr())
        with _on_device(device):
            if self._prefix(slots):
                status = lib.attnres_hip_packed_backward_coef(
                    self._values.data_ptr(), tokens * width, width, count, tokens, width, query.data_ptr(), rank,
                    scale, *saved, coef.data_ptr(), grad_query.data_ptr(), workspace.data_ptr(), workspace.numel(),
                    _stream(device))
            else:
                pointers = (ctypes.c_void_p * count)(*[self._slot_ptr(i) for i in slots])
                strides = (ctypes.c_int64 * count)(*([width] * count))
                status = lib.attnres_hip_sources_backward_coef(
                    pointers, strides, count, tokens, width, query.data_ptr(), rank, scale, *saved, coef.data_ptr(),
                    grad_query.data_ptr(), workspace.data_ptr(), workspace.numel(), _stream(device))
        _native.check(status, "attnres source-bank coefficient backward")
        if rank == width:
            query_row = query
        else:  # the query is aligned to the row's last R elements, zeros before
            query_row = torch.zeros((width,), device=device, dtype=torch.bfloat16)
            query_row[width - rank:] = query.reshape(-1)
        # the tensors stay referenced until the slots' gathers are enqueued
        record = ((grad_out, query_row, coef), (grad_out.data_ptr(), query_row.data_ptr(), coef.data_ptr(), count),
                  rank)
        for position, slot in enumerate(slots):
            self._pending[slot].append((record, position))
        return grad_query

    def _take(self, slot: int, dtype: torch.dtype) -> Tensor | None:
        """Slot `slot`'s gradient for this pass, or None: gathered (in BF16
        when ``dtype`` is BF16 and one gather launch covers the slot's reads,
        else FP32), or a view of the FP32 accumulated sums."""
        if self._pass != _pass_id():
            return None
        if self.gradients == "accumulate":
            if not self._written[slot]:
                return None
            self._written[slot] = False
            return self._grads[slot]
        pending, self._pending[slot] = self._pending[slot], []
        if not pending:
            return None
        lib = _native.load()
        width, tokens, device = self._width, self._tokens, self._device
        reads = array("q")  # attnres_gather_read[len(pending)]
        for (_, head, rank), position in pending:
            reads.extend(head)
            reads.append(position)
            reads.append(rank)
        rank0 = pending[0][0][2]
        bf16 = (_BF16_GATHER and dtype == torch.bfloat16 and len(pending) <= _MAX_GATHER_READS
                and all(rank == rank0 for (_, _, rank), _ in pending))
        grad = torch.empty(self._values.shape[1:], device=device, dtype=torch.bfloat16 if bf16 else torch.float32)
        with _on_device(device):
            status = lib.attnres_hip_bank_gather(self._slot_ptr(slot), width, tokens, width,
                                                 reads.buffer_info()[0], len(pending), grad.data_ptr(),
                                                 _DTYPE_BF16 if bf16 else _DTYPE_F32, 0,
                                                 _stream(device))
        _native.check(status, "attnres source-bank gather")
        return grad


class SourceBank:
    """Sources kept in numbered slots of one packed BF16 buffer and read as
    slot lists: the residual stream of a Full- or Block-schedule model.

    Full schedule (read i sees every source pushed before it)::

        bank = SourceBank(capacity=2 * layers + 1)
        bank.push(embedding)                      # slot 0; any float dtype, shape [..., D]
        x = bank.read(query_0)                    # attnres over slot 0 (BF16 out)
        bank.push(sublayer(x.to(dtype)))          # slot 1
        x = bank.read(query_1)                    # over slots 0..1, ...

    Block schedule (a read sees the completed blocks, slots 0..k-1, plus the
    running partial sum of the current block in some other slot)::

        bank.push(embedding, slot=0)
        bank.push(first_emitted, slot=p)          # the partial starts as one output
        x = bank.read(query, count=1, tail=p)     # attnres(embedding, partial)
        partial = bank.push_sum(partial, emitted, slot=q)   # partial + emitted, one pass

    Each source is converted to BF16 once, into its slot, so a read passes
    slot rows (the prefix view ``buffer[:count]``, or a list of slot pointers
    when a tail slot is added) with no per-read conversion or stack.
    ``push_sum`` adds the block's partial and the new output and writes the
    sum (in their dtype, returned) and its BF16 copy (into the slot) in one
    kernel (``attnres_hip_partial_sum``).

    Gradients (``gradients="gather"``, the default): a read's backward writes
    no dv rows, only its dq and the per-token coefficients of its dv
    (``attnres_hip_{packed,sources}_backward_coef``), and keeps its BF16 dO.
    Slot i's gradient is formed once, when the slot's push node runs its
    backward, by ``attnres_hip_bank_gather``: one FP32 pass over the dO rows
    of the reads that saw slot i.  The ordering uses one chain of zero-size
    tokens: every push node takes the token of the push before it, and a
    read takes the latest token, so a push node's backward runs after that
    of every read made after the push (those that saw the slot among them),
    and a read has one token input however many slots it reads.  ``gradients="accumulate"`` instead adds
    every read's FP32 dv into one FP32 ``[capacity, ..., D]`` buffer in the
    backward kernel (``attnres_hip_{packed,sources}_backward_accumulate_f32``:
    a read-modify-write of the sum per read).  Either way the sums are FP32
    without BF16 rounding of the per-read dv, and reach the source in its
    dtype.  Eager mode only; one bank per forward pass.
    """

    def __init__(self, capacity: int, *, gradients: str = "gather") -> None:
        if isinstance(capacity, bool) or not isinstance(capacity, int) or not 1 <= capacity <= _MAX_SOURCES:
            raise ValueError(f"capacity must be an integer in 1..{_MAX_SOURCES}")
        if gradients not in ("gather", "accumulate"):
            raise ValueError("gradients must be 'gather' or 'accumulate'")
        self.capacity = capacity
        self.gradients = gradients
        self._state = _BankState(capacity, gradients)
        self._pushed: list[bool] = [False] * capacity
        self._token: Tensor | None = None  # the latest push's token

    def __len__(self) -> int:
        """Number of pushed slots."""
        return sum(self._pushed)

    def _claim(self, source: Tensor, slot: int | None) -> int:
        if not isinstance(source, Tensor) or not source.is_floating_point():
            raise TypeError("a source must be a floating-point tensor")
        if not source.is_cuda:
            raise RuntimeError("attnres requires CUDA (ROCm/HIP) device tensors")
        if slot is None:
            free = [i for i, pushed in enumerate(self._pushed) if not pushed]
            if not free:
                raise ValueError("the source bank is full")
            slot = free[0]
        if isinstance(slot, bool) or not isinstance(slot, int) or not 0 <= slot < self.capacity:
            raise ValueError(f"slot must be an integer in 0..{self.capacity - 1}")
        if self._pushed[slot]:
            raise ValueError(f"slot {slot} already holds a source")
        state = self._state
        if state._values is None:
            if source.ndim < 1 or source.numel() == 0 or not 1 <= source.shape[-1] <= _MAX_WIDTH:
                raise ValueError("each source must have shape [...,D]")
            state._allocate(source)
        elif source.shape != state._values.shape[1:] or source.device != state._values.device:
            raise ValueError("all source tensors must have the same logical shape and device")
        return slot

    def push(self, source: Tensor, *, slot: int | None = None) -> int:
        """Store ``source`` (``[..., D]``, any float dtype, on the GPU) in
        ``slot`` (default: the lowest free one); returns the slot."""
        slot = self._claim(source, slot)
        self._token = _Push.apply(self._state, slot, source, self._token)
        self._pushed[slot] = True
        return slot

    def push_sum(self, prev: Tensor, emitted: Tensor, *, slot: int | None = None) -> Tensor:
        """``prev + emitted`` (FP32 or BF16, same shape and dtype), returned in
        that dtype and stored as BF16 in ``slot`` -- one kernel for the
        Block schedule's partial sum and its BF16 copy."""
        if not isinstance(prev, Tensor) or not isinstance(emitted, Tensor):
            raise TypeError("push_sum takes two tensors")
        if prev.shape != emitted.shape or prev.dtype != emitted.dtype or prev.device != emitted.device:
            raise ValueError("push_sum needs tensors of one shape, dtype and device")
        if prev.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError("push_sum supports float32 and bfloat16 tensors")
        slot = self._claim(emitted, slot)
        partial, self._token = _PushSum.apply(self._state, slot, prev, emitted, self._token)
        self._pushed[slot] = True
        return partial

    def read(self, query: Tensor, *, count: int | None = None, tail: int | None = None, eps: float = _EPS,
             scale: float = 1.0) -> Tensor:
        """``attnres`` over slots ``0..count-1`` (default: every pushed slot,
        which must then be ``0..len-1``) followed by slot ``tail`` if given; BF16."""
        if count is None:
            if tail is not None:
                raise ValueError("a read with a tail slot needs count")
            count = len(self)
        if isinstance(count, bool) or not isinstance(count, int) or not 0 <= count <= self.capacity:
            raise ValueError("count must be a number of leading slots")
        if not all(self._pushed[:count]):
            raise ValueError("count must select pushed slots 0..count-1")
        slots = list(range(count))
        if tail is not None:
            if isinstance(tail, bool) or not isinstance(tail, int) or not count <= tail < self.capacity \
                    or not self._pushed[tail]:
                raise ValueError("tail must be a pushed slot after the leading ones")
            slots.append(tail)
        if not slots:
            raise ValueError("a read needs at least one source")
        # the slots were checked at their push: BF16 rows [..., D] on one device
        state = self._state
        eps_value, scale_value = check_query(query, state._width, state._device, eps, scale)
        if not _needs_gradients(query, self._token):  # the forward alone: nothing saved
            query = _contiguous(query)
            if state._prefix(tuple(slots)):
                out = packed_forward_impl(state._flat[:len(slots)], query, eps_value, scale_value, False, pooled=True)[0]
            else:
                out = sources_forward_impl(state._sources(tuple(slots)), query, eps_value, scale_value, False,
                                           pooled=True)[0]
            return out.reshape(state._values.shape[1:])
        return _BankRead.apply(self._state, tuple(slots), query, eps_value, scale_value, self._token)


def _needs_gradients(query: Tensor, token: Tensor | None) -> bool:
    """Whether autograd will want this read's gradients: grad mode on and the
    query or the sources (through the container's token) requiring grad.
    Otherwise a read runs the forward alone, with no refinement bytes or
    saved state, and the same output bits."""
    return torch.is_grad_enabled() and (query.requires_grad or (token is not None and token.requires_grad))


def _token_input_grad(ctx, index: int) -> Tensor | None:
    """The zero-size gradient of a token input (None when it has none)."""
    return torch.empty((0,), device=ctx.token_device) if ctx.needs_input_grad[index] else None


class _Push(torch.autograd.Function):
    """Copy a source into its slot; the new token follows ``previous`` (the
    token of the push before, None for the first)."""

    @staticmethod
    def forward(ctx, bank: _BankState, slot: int, source: Tensor, previous: Tensor | None) -> Tensor:
        bank._values[slot].copy_(source.detach())
        ctx.bank, ctx.slot, ctx.dtype, ctx.token_device = bank, slot, source.dtype, source.device
        return source.new_empty((0,))

    @staticmethod
    def backward(ctx, _token_grad):
        grad = ctx.bank._take(ctx.slot, ctx.dtype)
        return None, None, None if grad is None else grad.to(ctx.dtype), _token_input_grad(ctx, 3)


class _PushSum(torch.autograd.Function):
    """partial = prev + emitted, with its BF16 copy written into the slot by
    the same kernel; the gradient of both inputs is that of the partial plus
    the slot's summed read gradient."""

    @staticmethod
    def forward(ctx, bank: _BankState, slot: int, prev: Tensor, emitted: Tensor, previous: Tensor | None):
        lib = _native.load()
        prev, emitted = _contiguous(prev.detach()), _contiguous(emitted.detach())
        partial = torch.empty_like(emitted)
        dtype = _DTYPE_F32 if emitted.dtype == torch.float32 else _DTYPE_BF16
        with _on_device(emitted.device):
            status = lib.attnres_hip_partial_sum(prev.data_ptr(), emitted.data_ptr(), dtype, emitted.numel(),
                                                 partial.data_ptr(), bank._slot_ptr(slot),
                                                 _stream(emitted.device))
        _native.check(status, "attnres partial sum")
        ctx.bank, ctx.slot, ctx.dtype, ctx.token_device = bank, slot, emitted.dtype, emitted.device
        return partial, emitted.new_empty((0,))

    @staticmethod
    def backward(ctx, grad_partial, _token_grad):
        grad = ctx.bank._take(ctx.slot, ctx.dtype)
        if grad is not None:
            grad = grad.to(ctx.dtype) if grad_partial is None else grad_partial + grad.to(ctx.dtype)
        else:
            grad = grad_partial
        return None, None, grad, grad, _token_input_grad(ctx, 4)


class _BankRead(torch.autograd.Function):
    @staticmethod
    def forward(ctx, bank: _BankState, slots: tuple[int, ...], query: Tensor, eps: float, scale: float,
                token: Tensor) -> Tensor:
        query = _contiguous(query)
        shape = bank._values.shape[1:]
        if bank._prefix(slots):
            flat = bank._flat[:len(slots)]
            out, out_refine, logit, inv_rms, stats = packed_forward_impl(flat, query, eps, scale, True, pooled=True)
        else:
            out, out_refine, logit, inv_rms, stats = sources_forward_impl(bank._sources(slots), query, eps, scale,
                                                                         True, pooled=True)
        # always saved: the accumulating kernels read the refinement
        ctx.bank, ctx.slots, ctx.scale = bank, slots, scale
        ctx.token_device = token.device
        ctx.save_for_backward(query, out, out_refine, logit, inv_rms, stats)
        return out.reshape(shape)

    @staticmethod
    def backward(ctx, grad_out):
        query, out, out_refine, logit, inv_rms, stats = ctx.saved_tensors
        grad_query = ctx.bank._backward(ctx.slots, query, out, out_refine, grad_out, logit, inv_rms, stats,
                                        ctx.scale)
        return None, None, grad_query if ctx.needs_input_grad[2] else None, None, None, _token_input_grad(ctx, 5)


__all__ = ["SharedSources", "SourceBank"]
