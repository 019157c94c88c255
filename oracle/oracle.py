"""CPU FP32 oracle of the AttnRes read -- TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s CPU-baseline leg
may import this module, and only as the checker (or the timed CPU
baseline).  The product path (`fast-attnres_amd/attnres`) never imports it;
it has no CPU fallback.

Restates the reference's validation oracle, `validation/oracle.py:5-19`,
whose semantics define correctness for this operator:

* BF16 inputs only (FP32/FP64 are rejected, `validation/oracle.py:9-10`);
* autocast is disabled, so results do not depend on an enclosing autocast
  region (`validation/oracle.py:11`);
* a list/tuple of sources is stacked along a new leading axis;
* the value and the key are promoted to FP32 SEPARATELY (one ``.float()`` of
  the whole value, one of its last-R slice), so in autograd the value
  gradient arrives as two BF16 contributions (direct + key path) that are
  summed in BF16 -- the "double-rounded" tail gradient that
  `validation/REVISIONS.md:19-26` fixes as the contract;
* the key is normalised first, then dotted with the query, then scaled
  (normalise-then-dot, `validation/oracle.py:16-17`);
* softmax over the source axis, FP32 mix, one BF16 rounding of the output.

The parity bar for the HIP kernels is the reference's own gate,
``rtol = atol = 0.05`` on outputs and first-order gradients
(`validation/protocol.json:12-15`, `validation/comparison.py:5-12`).

Besides the BF16 gate, the kernels are measured in BF16 ulps against
`oracle_float64`: the same operations in float64 with no rounding, which
isolates the kernels' own rounding from the oracle's (its double-rounded
tail gradient can sit several ulps from the exact value where the two parts
cancel).

Parity status of each function here (all pinned; `tests/test_oracle_pinning.py`):

* `oracle`, `oracle_with_grads`: float64 brute force and finite differences
  (`oracle/exact.py`), the closed-form known-answer cases of the reference's
  tests (equal logits, zero scale, zero keys, single source), planted-mistake
  mutants;
* `oracle_float64`, `exact_with_grads`: the same brute force and finite
  differences at float64 tolerances (1e-12 forward), and agreement with
  `oracle` to one BF16 rounding;
* `oracle_chunks`, `chunked_with_grads`: bitwise equal to the unchunked `oracle_with_grads`
  for the output and value gradient, the query gradient within FP32 order;
  equal to `exact_with_grads` in float64 to 1e-12;
* `softmax_statistics`: float64 values of the logits, 1/rms, max and 1/sum.
"""

from __future__ import annotations

import torch

EPS = 2**-23
BF16_TOLERANCE = {"rtol": 0.05, "atol": 0.05}


def _packed(values) -> torch.Tensor:
    if isinstance(values, (list, tuple)):
        return torch.stack(tuple(values))
    return values


def _mix(value: torch.Tensor, key: torch.Tensor, query: torch.Tensor, eps: float, scale: float) -> torch.Tensor:
    """The read's arithmetic on already-promoted tensors (`validation/oracle.py:16-19`):
    normalise the key, dot with the query, scale, softmax over the source
    axis, mix the values.  Runs in the dtype of its arguments."""
    inv_rms = torch.rsqrt(key.square().mean(-1, keepdim=True) + eps)
    logit = (key * inv_rms * query).sum(-1) * scale
    weight = logit.softmax(0)
    return (weight.unsqueeze(-1) * value).sum(0)


def _promoted(packed: torch.Tensor, rank: int, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """Value and key promoted SEPARATELY (`validation/oracle.py:14-15`)."""
    return packed.to(dtype), packed[..., packed.shape[-1] - rank:].to(dtype)


def oracle(values, query, *, eps: float = EPS, scale: float = 1.0) -> torch.Tensor:
    """BF16 AttnRes read with FP32 internal arithmetic; differentiable.

    ``values``: BF16 ``[S, ..., D]`` or a list/tuple of ``S`` BF16 ``[..., D]``;
    ``query``: BF16 ``[R]``.  Returns BF16 ``[..., D]``.
    """
    tensors = [*values, query] if isinstance(values, (list, tuple)) else [values, query]
    if any(tensor.dtype != torch.bfloat16 for tensor in tensors):
        raise TypeError("the oracle requires BF16 tensors")
    with torch.autocast(device_type=query.device.type, enabled=False):
        value, key = _promoted(_packed(values), query.numel(), torch.float32)
        return _mix(value, key, query.float(), eps, scale).to(torch.bfloat16)


def oracle_float64(values, query, *, eps: float = EPS, scale: float = 1.0) -> torch.Tensor:
    """The same read in float64 with no final rounding: the reference value the
    kernels' BF16 results are measured against in BF16 ulps.

    Same operations and order as `oracle` (`_mix`), on float64 tensors.  Pass
    float64 leaves (BF16 inputs converted exactly) to get float64 gradients
    without the BF16 roundings of the oracle's autograd."""
    tensors = [*values, query] if isinstance(values, (list, tuple)) else [values, query]
    if any(tensor.dtype != torch.float64 for tensor in tensors):
        raise TypeError("oracle_float64 takes float64 tensors")
    with torch.autocast(device_type=query.device.type, enabled=False):
        packed = _packed(values)
        return _mix(packed, packed[..., packed.shape[-1] - query.numel():], query, eps, scale)


def oracle_with_grads(values, query, grad_out, *, eps: float = EPS, scale: float = 1.0):
    """Output and first-order gradients (values, query) of `oracle` for one
    upstream gradient, with fresh leaves so the caller's tensors are untouched.

    For a list input the value gradient is returned per source position."""
    if isinstance(values, (list, tuple)):
        leaves = [v.detach().clone().requires_grad_(True) for v in values]
        inputs = leaves
    else:
        leaves = [values.detach().clone().requires_grad_(True)]
        inputs = leaves[0]
    q = query.detach().clone().requires_grad_(True)
    out = oracle(inputs, q, eps=eps, scale=scale)
    grads = torch.autograd.grad(out, (*leaves, q), grad_out)
    grad_values = list(grads[:-1]) if isinstance(values, (list, tuple)) else grads[0]
    return out.detach(), grad_values, grads[-1]


def exact_with_grads(values, query, grad_out, *, eps: float = EPS, scale: float = 1.0):
    """`oracle_float64` output and gradients for BF16 inputs: the inputs are
    converted to float64 leaves (exactly), so the value gradient is the float64
    sum of its direct and key parts, with no rounding anywhere.  Returns float64
    ``(out, grad_values, grad_query)``; for a list input the value gradient is
    returned per source position."""
    if isinstance(values, (list, tuple)):
        leaves = [v.detach().double().requires_grad_(True) for v in values]
        inputs = leaves
    else:
        leaves = [values.detach().double().requires_grad_(True)]
        inputs = leaves[0]
    q = query.detach().double().requires_grad_(True)
    out = oracle_float64(inputs, q, eps=eps, scale=scale)
    grads = torch.autograd.grad(out, (*leaves, q), grad_out.detach().double())
    grad_values = list(grads[:-1]) if isinstance(values, (list, tuple)) else grads[0]
    return out.detach(), grad_values, grads[-1]


def oracle_chunks(values, query, grad_out, *, eps: float = EPS, scale: float = 1.0, chunk: int = 2048,
                  exact: bool = False):
    """The read over token chunks, one chunk at a time (for reads too large to
    hold whole): yields ``(start, stop, out, grad_value_rows, grad_query_part)``.

    ``values``: BF16 ``[S, N, D]`` or a list of ``S`` BF16 ``[N, D]`` (any
    device; chunks are moved to the CPU); ``grad_out``: ``[N, D]``.  Each chunk
    runs `oracle`'s own graph (``_promoted`` + ``_mix`` + the BF16 rounding),
    or `oracle_float64`'s when ``exact``.  The output and value-gradient rows
    of a chunk are exactly those of the whole read (tokens are independent);
    ``grad_query_part`` is the chunk's UNROUNDED query gradient (FP32 before
    the oracle's BF16 cast; float64 when ``exact``), to be summed over chunks.
    ``grad_value_rows`` is ``[S, n, D]`` (packed) or a list of ``[n, D]``."""
    listed = isinstance(values, (list, tuple))
    tokens = int(values[0].shape[0]) if listed else int(values.shape[1])
    dtype = torch.float64 if exact else torch.float32
    for start in range(0, tokens, chunk):
        stop = min(tokens, start + chunk)
        parts = [v[start:stop] for v in values] if listed else [values[:, start:stop]]
        leaves = [part.detach().cpu().to(torch.float64 if exact else torch.bfloat16).requires_grad_(True)
                  for part in parts]
        q = query.detach().cpu().to(dtype).requires_grad_(True)
        with torch.autocast(device_type="cpu", enabled=False):
            packed = _packed(leaves if listed else leaves[0])
            if exact:
                value, key = packed, packed[..., packed.shape[-1] - q.numel():]
            else:
                value, key = _promoted(packed, q.numel(), torch.float32)
            out = _mix(value, key, q, eps, scale)
            if not exact:
                out = out.to(torch.bfloat16)
        upstream = grad_out[start:stop].detach().cpu().to(out.dtype)
        grads = torch.autograd.grad(out, (*leaves, q), upstream)
        rows = list(grads[:-1]) if listed else grads[0]
        yield start, stop, out.detach(), rows, grads[-1]


def chunked_with_grads(values, query, grad_out, *, eps: float = EPS, scale: float = 1.0, chunk: int = 2048,
                       exact: bool = False):
    """`oracle_with_grads` (or `exact_with_grads` when ``exact``) assembled from
    `oracle_chunks`.  The query gradient is the chunks' unrounded gradients
    added in chunk order and rounded once (BF16; float64 left as is), so it
    differs from the unchunked oracle's only by the FP32 summation order."""
    listed = isinstance(values, (list, tuple))
    outs, grad_rows, query_sum = [], [], None
    for _, _, out, rows, part in oracle_chunks(values, query, grad_out, eps=eps, scale=scale, chunk=chunk,
                                               exact=exact):
        outs.append(out)
        grad_rows.append(rows)
        query_sum = part if query_sum is None else query_sum + part
    out = torch.cat(outs)
    if listed:
        grad_values = [torch.cat([rows[s] for rows in grad_rows]) for s in range(len(values))]
    else:
        grad_values = torch.cat(grad_rows, dim=1)
    grad_query = query_sum if exact else query_sum.to(torch.bfloat16)
    return out, grad_values, grad_query


def softmax_statistics(values, query, *, eps: float = EPS, scale: float = 1.0):
    """FP32 routing statistics of the read, in the kernels' saved layout:
    ``logit[N, S]``, ``inv_rms[N, S]`` and ``stats[2, N]`` = (max over sources,
    1 / sum of exp(logit - max)).  Same promotion and op order as `oracle`."""
    rank = query.numel()
    with torch.no_grad(), torch.autocast(device_type=query.device.type, enabled=False):
        packed = _packed(values)
        sources, width = packed.shape[0], packed.shape[-1]
        key = packed.reshape(sources, -1, width)[..., width - rank:].float()
        inv_rms = torch.rsqrt(key.square().mean(-1) + eps)
        logit = (key * inv_rms[..., None] * query.float()).sum(-1) * scale
        maximum = logit.max(0).values
        inv_sum = 1.0 / (logit - maximum).exp().sum(0)
        return logit.T.contiguous(), inv_rms.T.contiguous(), torch.stack((maximum, inv_sum))


__all__ = ["BF16_TOLERANCE", "EPS", "chunked_with_grads", "exact_with_grads", "oracle", "oracle_chunks",
           "oracle_float64", "oracle_with_grads", "softmax_statistics"]
