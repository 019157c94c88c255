"""Shared helpers for the parity tests (inputs, comparisons)."""

from __future__ import annotations

import torch

from oracle.oracle import BF16_TOLERANCE, oracle

SEEDS = (20260827, 20260903, 20260911)  # reference validation/protocol.json:7-11


def compare(actual: torch.Tensor, expected: torch.Tensor, *, tol=BF16_TOLERANCE) -> dict:
    """Finite check + the reference's BF16 gate; returns error metrics
    (reference validation/gpu_checks.py:12-25)."""
    actual = actual.detach().cpu()
    expected = expected.detach().cpu()
    assert torch.isfinite(actual.float()).all(), "non-finite result"
    assert torch.isfinite(expected.float()).all(), "non-finite oracle result"
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    assert actual.dtype == expected.dtype, (actual.dtype, expected.dtype)
    torch.testing.assert_close(actual, expected, **tol)
    diff = (actual.float() - expected.float()).abs()
    return {"max_abs": float(diff.max()) if diff.numel() else 0.0,
            "rel_l2": float(diff.norm() / expected.float().norm().clamp_min(1e-12))}


def oracle_grads(make_values, leaves, query_leaf, upstream, *, eps=2**-23, scale=1.0):
    """Oracle output and grads w.r.t. CPU copies of the given leaves.

    `make_values(leaves, query)` builds the operator inputs from the leaves
    (views, lists) exactly as the GPU side does."""
    cpu_leaves = [leaf.detach().cpu().requires_grad_(True) for leaf in leaves]
    cpu_query = query_leaf.detach().cpu().requires_grad_(True)
    values, query = make_values(cpu_leaves, cpu_query)
    out = oracle(values, query, eps=eps, scale=scale)
    grads = torch.autograd.grad(out, (*cpu_leaves, cpu_query), upstream.detach().cpu())
    return out, grads
