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

Parity status of each function here: `oracle` is pinned by the float64
brute force and finite differences in `oracle/exact.py` and by the closed-form
known-answer cases of the reference's tests (equal logits, zero scale,
zero keys, single source; see `tests/test_oracle_pinning.py`).
"""

from __future__ import annotations

import torch

EPS = 2**-23
BF16_TOLERANCE = {"rtol": 0.05, "atol": 0.05}


def _packed(values) -> torch.Tensor:
    if isinstance(values, (list, tuple)):
        return torch.stack(tuple(values))
    return values


def oracle(values, query, *, eps: float = EPS, scale: float = 1.0) -> torch.Tensor:
    """BF16 AttnRes read with FP32 internal arithmetic; differentiable.

    ``values``: BF16 ``[S, ..., D]`` or a list/tuple of ``S`` BF16 ``[..., D]``;
    ``query``: BF16 ``[R]``.  Returns BF16 ``[..., D]``.
    """
    tensors = [*values, query] if isinstance(values, (list, tuple)) else [values, query]
    if any(tensor.dtype != torch.bfloat16 for tensor in tensors):
        raise TypeError("the oracle requires BF16 tensors")
    rank = query.numel()
    with torch.autocast(device_type=query.device.type, enabled=False):
        packed = _packed(values)
        value = packed.float()                      # direct path
        key = packed[..., packed.shape[-1] - rank:].float()   # routing path
        inv_rms = torch.rsqrt(key.square().mean(-1, keepdim=True) + eps)
        logit = (key * inv_rms * query.float()).sum(-1) * scale
        weight = logit.softmax(0)
        return (weight.unsqueeze(-1) * value).sum(0).to(torch.bfloat16)


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


__all__ = ["BF16_TOLERANCE", "EPS", "oracle", "oracle_with_grads", "softmax_statistics"]
