"""torch.library operators for the HIP read, their fake (meta) kernels and autograd.

Four opaque ops in the ``attnres_hip`` namespace stand where the reference
registers ``attnres::_fixed_tail_forward_with_aux`` / ``_fixed_tail_backward``
(packed, `src/attnres/_kernels/fixed_tail.py:902-1094`) and
``attnres::_fixed_tail_sources_forward_with_aux`` / ``_fixed_tail_sources_backward``
(list, `src/attnres/_kernels/fixed_tail_sources.py:78-183`):

* ``packed_forward(values[S,N,D], query[R], eps, scale)``
  -> ``(out[N,D] bf16, out_refine[N,D] int8, logit[N,S] f32, inv_rms[N,S] f32,
  stats[2,N] f32)``
* ``packed_backward(values, query, out, out_refine, grad_out, logit, inv_rms,
  stats, scale)`` -> ``(grad_values[S,N,D] bf16, grad_query[R] bf16)``
* ``sources_forward(sources: list, query, eps, scale)`` -> same five tensors,
  ``out`` shaped like one source
* ``sources_backward(sources, query, out, out_refine, grad_out, logit, inv_rms,
  stats, scale)`` -> ``[grad_source_0, ..., grad_source_{S-1}, grad_query]``

and two more for reads that need no gradient (grad mode off, or no input
requiring grad), which return the output alone and store no refinement or
saved state: ``packed_forward_out`` and ``sources_forward_out``.

In eager mode (not under dynamo tracing, plain tensors) ``packed_attnres``
and ``sources_attnres`` call the C++ autograd nodes of
``csrc/attnres_autograd.cpp`` (``_native.load_autograd``): the same C ABI
launches, saved state and gradients as the ops' registered autograd, without
the op dispatcher or Python in the node's forward and backward, which cost tens
of microseconds per read; under ``torch.compile`` they call the ops.

Every output and workspace is allocated with ``torch.empty`` on the caller's
device (here, or by those nodes); the kernels run on the current stream and the C ABI never
allocates or synchronises, so the ops are safe under ``torch.compile``
(opaque custom ops with fake kernels) and HIP/CUDA graph capture.

Saved for backward: the inputs, the small statistics and -- for reads of
more than ``RECOMPUTE_MAX_SOURCES`` sources -- the BF16 output plus one
refinement byte per element (together the FP32 mix to ulp/512, for
``delta = <dO, o>``).  Smaller reads save neither: ``out_refine`` is
``[0, D]`` and their backward derives delta from the value rows it reads
anyway; so do reads of up to ``KEYRES_MAX_SOURCES`` sources whose key is the
last 512 or 1024 elements of a 2048- or 4096-wide row, and of up to
``KEYRES_FULL_MAX_SOURCES`` with the whole 2048-wide row as key
(`keyres_key_chunks`: the key-resident backward holds the key coordinates of a
token's rows until delta is complete).  The reference makes the same structural choice
(`fla_full_sources._should_save_mixed`, `fla_full_sources.py:146-161`:
recompute for S <= 3) but saves an FP32 copy of the output for larger reads
(`fixed_tail.py:917-919`): four extra bytes per element written in the
forward and read in the backward instead of one.  Here the threshold is 6:
the recompute backward holds a token's rows in registers, and up to six
rows that is faster than writing and re-reading the refinement.
"""

from __future__ import annotations

import contextlib
import ctypes
import math
from typing import Any

import torch
from torch import Tensor

from . import _native

_F32 = torch.float32
_BF16 = torch.bfloat16

# Save/recompute policy (attnres_hip.h ATTNRES_RECOMPUTE_MAX_SOURCES,
# ATTNRES_KEYRES_MAX_SOURCES; attnres_hip_saves_refinement_for).
RECOMPUTE_MAX_SOURCES = 6
KEYRES_MAX_SOURCES = 16       # key of 512 or 1024 of a 2048- or 4096-wide row
KEYRES_FULL_MAX_SOURCES = 12  # the whole 2048-wide row as key
_KEY_COLUMN = 512  # elements per chunk column of a 64-lane row (64 lanes x 8)


def keyres_key_chunks(width: int, rank: int) -> int:
    """Chunk columns of the key when the key-resident backward applies to a
    read of this width and rank: rows of 2048 or 4096 elements (64-lane
    groups, every chunk in range) whose key is their last 512 or 1024
    elements (1 or 2 columns), or whole rows of 2048 (4 columns); 0 otherwise."""
    if not 1024 < width <= 4096:
        return 0
    chunks = 4 if width <= 2048 else 8
    if width != chunks * _KEY_COLUMN or rank % _KEY_COLUMN:
        return 0
    key_chunks = rank // _KEY_COLUMN
    if key_chunks == chunks:
        return key_chunks if chunks == 4 else 0
    return key_chunks if key_chunks <= 2 else 0


def saves_refinement(sources: int, width: int, rank: int) -> bool:
    """Whether a read saves its output refinement for the backward (else the
    backward takes delta from the value rows: every read of at most
    ``RECOMPUTE_MAX_SOURCES`` sources, and reads whose key the key-resident
    backward holds, up to ``KEYRES_MAX_SOURCES`` sources for a partial key and
    ``KEYRES_FULL_MAX_SOURCES`` for the whole row).  Reference
    `fla_full_sources._should_save_mixed`, `fla_full_sources.py:146-161`, keys
    on the source count alone."""
    if sources <= RECOMPUTE_MAX_SOURCES:
        return False
    key_chunks = keyres_key_chunks(width, rank)
    limit = KEYRES_FULL_MAX_SOURCES if key_chunks == 4 else KEYRES_MAX_SOURCES
    return not (key_chunks > 0 and sources <= limit)


def _refine_rows(sources: int, tokens: int, width: int, rank: int) -> int:
    return tokens if saves_refinement(sources, width, rank) else 0


def _pointer(tensor: Tensor) -> int | None:
    return tensor.data_ptr() if tensor.numel() else None
_OP_TAGS = (torch.Tag.flexible_layout,) if hasattr(torch.Tag, "flexible_layout") else ()


# ------------------------------------------------------------------ layouts

def row_stride(tensor: Tensor) -> int | None:
    """Element stride between consecutive rows of ``tensor[..., D]`` flattened
    to ``[rows, D]``, or None when the rows are not evenly spaced or a row is
    not unit-stride.  Size-1 dimensions place no constraint; a single row
    reports 0.  (Same flattening rule as the reference's
    `fla_full_sources._affine_row_stride`, `fla_full_sources.py:164-178`, plus
    the unit feature stride the 16-byte loads rely on.)"""
    if tensor.shape[-1] > 1 and tensor.stride(-1) != 1:
        return None
    stride: int | None = None
    rows = 1
    for size, step in zip(reversed(tensor.shape[:-1]), reversed(tensor.stride()[:-1])):
        if size == 1:
            continue
        if stride is None:
            stride = int(step)
        elif int(step) != rows * stride:
            return None
        rows *= int(size)
    return 0 if stride is None else stride


def prepare_rows(tensor: Tensor) -> tuple[Tensor, int]:
    """The tensor itself when its rows are addressable, else a contiguous copy."""
    stride = row_stride(tensor)
    if stride is None:
        tensor = tensor.contiguous()
        stride = row_stride(tensor)
        assert stride is not None
    return tensor, stride


def _unit_feature_stride(values: Tensor) -> Tensor:
    if values.shape[-1] > 1 and values.stride(-1) != 1:
        return values.contiguous()
    return values


def _contiguous(tensor: Tensor) -> Tensor:
    return tensor if tensor.is_contiguous() else tensor.contiguous()


# torch's raw current-stream query skips building a Python Stream object (a
# few microseconds per launch); builds without it use the public Stream.
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    """The current stream's handle on ``device``."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(device.index)
    return torch.cuda.current_stream(device).cuda_stream


_NO_SWITCH = contextlib.nullcontext()


def _on_device(device: torch.device):
    """``torch.cuda.device(device)``, or nothing when it is the current device."""
    return _NO_SWITCH if device.index == torch.cuda.current_device() else torch.cuda.device(device)


def _rows_of(shape) -> int:
    return math.prod(int(size) for size in shape[:-1]) if len(shape) > 1 else 1


def _dq_workspace(lib, n_tokens: int, width: int, rank: int, device) -> Tensor:
    elems = int(lib.attnres_hip_dq_workspace_elems(n_tokens, width, rank))
    if elems < 0:
        raise ValueError("attnres backward: shape outside the supported envelope")
    return torch.empty((elems,), device=device, dtype=_F32)


def _pool_layout(tokens: int, sources: int, width: int, save: bool) -> tuple[int, int, int]:
    """``(head, block, size)`` of a pooled saved state: the refinement bytes
    ``[N, D]`` (when saved) at offset 0, then from the 16-byte aligned byte
    offset ``head`` logit ``[N, S]``, 1/rms ``[N, S]`` (``block`` = N*S floats
    each) and stats ``[2, N]`` in FP32; ``size`` bytes in all."""
    head = ((tokens * width if save else 0) + 15) // 16 * 16
    block = tokens * sources
    return head, block, head + 4 * (2 * block + 2 * tokens)


def _saved_state(tokens: int, sources: int, width: int, save: bool, device,
                 pooled: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """out_refine ``[N, D]`` int8 (``[0, D]`` when not saved), logit ``[N, S]``,
    inv_rms ``[N, S]`` and stats ``[2, N]`` (FP32).  ``pooled``: views of one
    byte allocation (``_pool_layout``), for callers that keep them together
    (not for custom-op outputs, which must not alias each other); a small read
    then pays one allocation here instead of four."""
    refine_rows = tokens if save else 0
    if not pooled:
        return (torch.empty((refine_rows, width), device=device, dtype=torch.int8),
                torch.empty((tokens, sources), device=device, dtype=_F32),
                torch.empty((tokens, sources), device=device, dtype=_F32),
                torch.empty((2, tokens), device=device, dtype=_F32))
    head, block, size = _pool_layout(tokens, sources, width, save)
    pool = torch.empty((size,), device=device, dtype=torch.uint8)
    floats = pool[head:].view(_F32)
    return (pool[:refine_rows * width].view(torch.int8).view(refine_rows, width),
            floats[:block].view(tokens, sources), floats[block:2 * block].view(tokens, sources),
            floats[2 * block:].view(2, tokens))


def _state_addresses(out_refine: Tensor, logit: Tensor, inv_rms: Tensor,
                     stats: Tensor) -> tuple[int | None, int, int, int]:
    return (_pointer(_contiguous(out_refine)), _contiguous(logit).data_ptr(), _contiguous(inv_rms).data_ptr(),
            _contiguous(stats).data_ptr())


# ------------------------------------------------------------------ packed

def _packed_forward_launch(values: Tensor, query: Tensor, eps: float, scale: float, out: Tensor,
                           state: tuple[int | None, int, int, int]) -> None:
    """``attnres_hip_packed_forward`` into ``out`` and the saved state at
    ``state`` = (out_refine or None, logit, inv_rms, stats) addresses."""
    sources, tokens, width = (int(size) for size in values.shape)
    device = values.device
    with _on_device(device):
        status = _native.load().attnres_hip_packed_forward(
            values.data_ptr(), values.stride(0), values.stride(1), sources, tokens, width,
            query.data_ptr(), query.numel(), eps, scale, out.data_ptr(), *state, _stream(device))
    _native.check(status, "attnres packed forward")


def packed_forward_impl(values: Tensor, query: Tensor, eps: float, scale: float,
                        save: bool, pooled: bool = False) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """The packed forward launch; ``save`` chooses whether the refinement is
    stored (``out_refine`` ``[N, D]``) or not (``[0, D]``); ``pooled`` as for
    ``_saved_state``."""
    values = _unit_feature_stride(values)
    query = _contiguous(query)
    sources, tokens, width = (int(size) for size in values.shape)
    out = torch.empty((tokens, width), device=values.device, dtype=_BF16)
    state = _saved_state(tokens, sources, width, save, values.device, pooled)
    _packed_forward_launch(values, query, eps, scale, out, _state_addresses(*state))
    return (out, *state)


@torch.library.custom_op("attnres_hip::packed_forward", mutates_args=(),
                         device_types="cuda", tags=_OP_TAGS)
def packed_forward(values: Tensor, query: Tensor, eps: float,
                   scale: float) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    return packed_forward_impl(values, query, eps, scale,
                               saves_refinement(int(values.shape[0]), int(values.shape[2]), query.numel()))


@packed_forward.register_fake
def _packed_forward_fake(values, query, eps, scale):
    sources, tokens, width = values.shape
    return (values.new_empty((tokens, width)),
            values.new_empty((_refine_rows(sources, tokens, width, query.numel()), width), dtype=torch.int8),
            values.new_empty((tokens, sources), dtype=_F32),
            values.new_empty((tokens, sources), dtype=_F32),
            values.new_empty((2, tokens), dtype=_F32))


@torch.library.custom_op("attnres_hip::packed_forward_out", mutates_args=(),
                         device_types="cuda", tags=_OP_TAGS)
def packed_forward_out(values: Tensor, query: Tensor, eps: float, scale: float) -> Tensor:
    """The packed forward of a read that needs no gradient: the output alone.
    No refinement bytes are stored (the C ABI takes ``out_refine = NULL`` at
    any S); the statistics the kernels write live in scratch freed on
    return.  The output is ``packed_forward``'s, bit for bit."""
    return packed_forward_impl(values, query, eps, scale, False, pooled=True)[0]


@packed_forward_out.register_fake
def _packed_forward_out_fake(values, query, eps, scale):
    return values.new_empty((values.shape[1], values.shape[2]))


def _packed_backward_launch(values: Tensor, query: Tensor, out: Tensor | None, grad_out: Tensor,
                            state: tuple[int | None, int, int, int], scale: float) -> tuple[Tensor, Tensor]:
    """``attnres_hip_packed_backward`` with the saved state at ``state``
    addresses (out_refine None: nothing saved, delta from the value rows; then
    ``out`` is not read)."""
    lib = _native.load()
    values = _unit_feature_stride(values)
    query = _contiguous(query)
    grad_out = _contiguous(grad_out.to(_BF16))
    refine = state[0]
    sources, tokens, width = (int(size) for size in values.shape)
    rank = query.numel()
    device = values.device
    grad_values = torch.empty((sources, tokens, width), device=device, dtype=_BF16)
    grad_query = torch.empty((rank,), device=device, dtype=_BF16)
    workspace = _dq_workspace(lib, tokens, width, rank, device)
    with _on_device(device):
        status = lib.attnres_hip_packed_backward(
            values.data_ptr(), values.stride(0), values.stride(1), sources, tokens, width,
            query.data_ptr(), rank, scale, None if refine is None else _contiguous(out).data_ptr(), refine,
            grad_out.data_ptr(), *state[1:], grad_values.data_ptr(), grad_query.data_ptr(),
            workspace.data_ptr(), workspace.numel(), _stream(device))
    _native.check(status, "attnres packed backward")
    return grad_values, grad_query


def packed_backward_impl(values: Tensor, query: Tensor, out: Tensor, out_refine: Tensor,
                         grad_out: Tensor, logit: Tensor, inv_rms: Tensor, stats: Tensor,
                         scale: float) -> tuple[Tensor, Tensor]:
    """The packed backward launch (dv rows and dq); an empty ``out_refine``
    means nothing was saved (delta from the value rows)."""
    return _packed_backward_launch(values, query, out, grad_out,
                                   _state_addresses(out_refine, logit, inv_rms, stats), scale)


@torch.library.custom_op("attnres_hip::packed_backward", mutates_args=(),
                         device_types="cuda", tags=_OP_TAGS)
def packed_backward(values: Tensor, query: Tensor, out: Tensor, out_refine: Tensor,
                    grad_out: Tensor, logit: Tensor, inv_rms: Tensor, stats: Tensor,
                    scale: float) -> tuple[Tensor, Tensor]:
    return packed_backward_impl(values, query, out, out_refine, grad_out, logit, inv_rms, stats, scale)


@packed_backward.register_fake
def _packed_backward_fake(values, query, out, out_refine, grad_out, logit, inv_rms, stats,
                          scale):
    return (values.new_empty(values.shape),
            query.new_empty(query.shape))


def _packed_setup_context(ctx: Any, inputs: tuple, output: tuple) -> None:
    values, query, _eps, scale = inputs
    out, out_refine, logit, inv_rms, stats = output
    ctx.mark_non_differentiable(out_refine, logit, inv_rms, stats)
    ctx.set_materialize_grads(False)
    # recompute policy: the output is not needed (the empty refinement stands in)
    saved_out = out if out_refine.numel() else out_refine
    ctx.save_for_backward(values, query, saved_out, out_refine, logit, inv_rms, stats)
    ctx.scale = float(scale)


def _packed_autograd(ctx: Any, grad_out, *_aux_grads):
    if grad_out is None:
        return None, None, None, None
    values, query, out, out_refine, logit, inv_rms, stats = ctx.saved_tensors
    grad_values, grad_query = packed_backward(
        values, query, out, out_refine, grad_out, logit, inv_rms, stats, ctx.scale)
    return (grad_values if ctx.needs_input_grad[0] else None,
            grad_query if ctx.needs_input_grad[1] else None, None, None)


packed_forward.register_autograd(_packed_autograd, setup_context=_packed_setup_context)


def _needs_grad(query: Tensor, *sources: Tensor) -> bool:
    """Whether autograd will want gradients of this read (grad mode on and an
    input that requires grad); traced as a guarded constant under dynamo."""
    return torch.is_grad_enabled() and (query.requires_grad or any(s.requires_grad for s in sources))


def _eager(*tensors: Tensor) -> bool:
    """An eager call: not under dynamo tracing, and only plain tensors or
    parameters (no fake or functional tensors of a compiler's tracing)."""
    return not torch.compiler.is_compiling() and all(type(t) in (Tensor, torch.nn.Parameter) for t in tensors)


def packed_attnres(values: Tensor, query: Tensor, eps: float, scale: float) -> Tensor:
    """Packed ``[S, ..., D]`` adapter (reference `fixed_tail.fused_attnres`,
    `fixed_tail.py:1097-1135`): flatten the batch axes to ``[S, N, D]`` as a
    view when the layout allows it (a copy only otherwise), call the op and
    restore the batch shape.  The eager node does the flattening inside, so
    autograd records no view nodes around it."""
    query = _contiguous(query)
    if _eager(values, query):
        return _native.load_autograd().packed_read(values, query, eps, scale)
    sources, width = int(values.shape[0]), int(values.shape[-1])
    flat = values.reshape(sources, -1, width)
    if width > 1 and flat.stride(2) != 1:
        flat = flat.contiguous()
    if not _needs_grad(query, values):
        return packed_forward_out(flat, query, eps, scale).reshape(values.shape[1:])
    return packed_forward(flat, query, eps, scale)[0].reshape(values.shape[1:])


# -------------------------------------------------------------------- list

def _source_table(sources: list[Tensor]) -> tuple[list[Tensor], Any, Any]:
    prepared, strides = [], []
    for source in sources:
        tensor, stride = prepare_rows(source)
        prepared.append(tensor)
        strides.append(stride)
    count = len(prepared)
    pointers = (ctypes.c_void_p * count)(*[tensor.data_ptr() for tensor in prepared])
    row_strides = (ctypes.c_int64 * count)(*strides)
    return prepared, pointers, row_strides


def _sources_forward_launch(sources: list[Tensor], query: Tensor, eps: float, scale: float, out: Tensor,
                            state: tuple[int | None, int, int, int]) -> None:
    """``attnres_hip_sources_forward`` into ``out`` and the saved state at
    ``state`` addresses (as ``_packed_forward_launch``)."""
    first = sources[0]
    count, tokens, width = len(sources), _rows_of(first.shape), int(first.shape[-1])
    device = first.device
    prepared, pointers, row_strides = _source_table(sources)
    with _on_device(device):
        status = _native.load().attnres_hip_sources_forward(
            pointers, row_strides, count, tokens, width, query.data_ptr(), query.numel(),
            eps, scale, out.data_ptr(), *state, _stream(device))
    del prepared  # copies (if any) stay alive until the launch is enqueued
    _native.check(status, "attnres source-list forward")


def sources_forward_impl(sources: list[Tensor], query: Tensor, eps: float, scale: float,
                         save: bool, pooled: bool = False) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """The source-list forward launch; ``save`` and ``pooled`` as for
    ``packed_forward_impl``."""
    first = sources[0]
    query = _contiguous(query)
    count, tokens, width = len(sources), _rows_of(first.shape), int(first.shape[-1])
    out = torch.empty(first.shape, device=first.device, dtype=_BF16)
    state = _saved_state(tokens, count, width, save, first.device, pooled)
    _sources_forward_launch(sources, query, eps, scale, out, _state_addresses(*state))
    return (out, *state)


@torch.library.custom_op("attnres_hip::sources_forward", mutates_args=(),
                         device_types="cuda", tags=_OP_TAGS)
def sources_forward(sources: list[Tensor], query: Tensor, eps: float,
                    scale: float) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    return sources_forward_impl(sources, query, eps, scale,
                                saves_refinement(len(sources), int(sources[0].shape[-1]), query.numel()))


@torch.library.custom_op("attnres_hip::sources_forward_out", mutates_args=(),
                         device_types="cuda", tags=_OP_TAGS)
def sources_forward_out(sources: list[Tensor], query: Tensor, eps: float, scale: float) -> Tensor:
    """The source-list forward of a read that needs no gradient (as
    ``packed_forward_out``)."""
    return sources_forward_impl(sources, query, eps, scale, False, pooled=True)[0]


@sources_forward_out.register_fake
def _sources_forward_out_fake(sources, query, eps, scale):
    return sources[0].new_empty(sources[0].shape)


@sources_forward.register_fake
def _sources_forward_fake(sources, query, eps, scale):
    first = sources[0]
    count, tokens = len(sources), _rows_of(first.shape)
    return (first.new_empty(first.shape),
            first.new_empty((_refine_rows(count, tokens, int(first.shape[-1]), query.numel()), int(first.shape[-1])),
                            dtype=torch.int8),
            first.new_empty((tokens, count), dtype=_F32),
            first.new_empty((tokens, count), dtype=_F32),
            first.new_empty((2, tokens), dtype=_F32))


def _sources_backward_launch(sources: list[Tensor], query: Tensor, out: Tensor | None, grad_out: Tensor,
                             state: tuple[int | None, int, int, int], scale: float) -> list[Tensor]:
    """``attnres_hip_sources_backward`` with the saved state at ``state``
    addresses (as ``_packed_backward_launch``): one dv buffer per list
    position, then dq."""
    lib = _native.load()
    first = sources[0]
    query = _contiguous(query)
    grad_out = _contiguous(grad_out.to(_BF16))
    refine = state[0]
    count, tokens, width = len(sources), _rows_of(first.shape), int(first.shape[-1])
    rank = query.numel()
    device = first.device
    prepared, pointers, row_strides = _source_table(sources)
    grads = [torch.empty(first.shape, device=device, dtype=_BF16) for _ in range(count)]
    grad_pointers = (ctypes.c_void_p * count)(*[grad.data_ptr() for grad in grads])
    grad_query = torch.empty((rank,), device=device, dtype=_BF16)
    workspace = _dq_workspace(lib, tokens, width, rank, device)
    with _on_device(device):
        status = lib.attnres_hip_sources_backward(
            pointers, row_strides, count, tokens, width, query.data_ptr(), rank, scale,
            None if refine is None else _contiguous(out).data_ptr(), refine, grad_out.data_ptr(), *state[1:],
            grad_pointers, grad_query.data_ptr(), workspace.data_ptr(), workspace.numel(), _stream(device))
    del prepared
    _native.check(status, "attnres source-list backward")
    return [*grads, grad_query]


def sources_backward_impl(sources: list[Tensor], query: Tensor, out: Tensor, out_refine: Tensor,
                          grad_out: Tensor, logit: Tensor, inv_rms: Tensor, stats: Tensor,
                          scale: float) -> list[Tensor]:
    """The source-list backward launch: one dv buffer per list position, then dq."""
    return _sources_backward_launch(sources, query, out, grad_out,
                                    _state_addresses(out_refine, logit, inv_rms, stats), scale)


@torch.library.custom_op("attnres_hip::sources_backward", mutates_args=(),
                         device_types="cuda", tags=_OP_TAGS)
def sources_backward(sources: list[Tensor], query: Tensor, out: Tensor, out_refine: Tensor,
                     grad_out: Tensor, logit: Tensor, inv_rms: Tensor, stats: Tensor,
                     scale: float) -> list[Tensor]:
    return sources_backward_impl(sources, query, out, out_refine, grad_out, logit, inv_rms, stats, scale)


@sources_backward.register_fake
def _sources_backward_fake(sources, query, out, out_refine, grad_out, logit, inv_rms, stats,
                           scale):
    return [source.new_empty(source.shape)
            for source in sources] + [query.new_empty(query.shape)]


def _sources_setup_context(ctx: Any, inputs: tuple, output: tuple) -> None:
    sources, query, _eps, scale = inputs
    out, out_refine, logit, inv_rms, stats = output
    ctx.mark_non_differentiable(out_refine, logit, inv_rms, stats)
    ctx.set_materialize_grads(False)
    saved_out = out if out_refine.numel() else out_refine
    ctx.save_for_backward(*sources, query, saved_out, out_refine, logit, inv_rms, stats)
    ctx.count = len(sources)
    ctx.scale = float(scale)


def _sources_autograd(ctx: Any, grad_out, *_aux_grads):
    count = ctx.count
    if grad_out is None:
        return [None] * count, None, None, None
    saved = ctx.saved_tensors
    sources = list(saved[:count])
    query, out, out_refine, logit, inv_rms, stats = saved[count:]
    grads = sources_backward(sources, query, out, out_refine, grad_out, logit, inv_rms, stats,
                             ctx.scale)
    return list(grads[:count]), grads[count], None, None


sources_forward.register_autograd(_sources_autograd, setup_context=_sources_setup_context)


def sources_attnres(sources: tuple[Tensor, ...], query: Tensor, eps: float,
                    scale: float) -> Tensor:
    """Ordered source-list adapter (reference `fixed_tail_sources.source_attnres`,
    `fixed_tail_sources.py:186-195`): the list is passed through unpacked."""
    query = _contiguous(query)
    if _eager(query, *sources):
        return _native.load_autograd().sources_read(query, eps, scale, list(sources))
    if not _needs_grad(query, *sources):
        return sources_forward_out(list(sources), query, eps, scale)
    return sources_forward(list(sources), query, eps, scale)[0]


__all__ = [
    "KEYRES_FULL_MAX_SOURCES", "KEYRES_MAX_SOURCES", "RECOMPUTE_MAX_SOURCES", "keyres_key_chunks", "packed_attnres", "packed_backward", "packed_backward_impl", "packed_forward",
    "packed_forward_impl", "packed_forward_out", "prepare_rows", "row_stride", "saves_refinement", "sources_attnres",
    "sources_backward", "sources_backward_impl", "sources_forward", "sources_forward_impl", "sources_forward_out",
]
