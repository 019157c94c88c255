"""Float64 brute-force restatement of the AttnRes read -- TEST INFRASTRUCTURE ONLY.

Independent of torch and of `oracle/oracle.py`: plain Python/NumPy loops in
float64 straight from the operator's equation (reference `docs/equation.md:44-55`):

    t_s = v_s[D-R:D];  r_s = sqrt(mean(t_s^2) + eps);  k_s = t_s / r_s
    z_s = scale * <k_s, q>;  p = softmax_s(z);  out = sum_s p_s v_s

Gradients are CENTRAL FINITE DIFFERENCES of the scalar <dO, out>, not an
analytic formula, so they pin the oracle's autograd (and the kernels'
hand-derived backward) without restating it.  For small inputs only.
"""

from __future__ import annotations

import math

import numpy as np


def read(values: np.ndarray, query: np.ndarray, eps: float, scale: float) -> np.ndarray:
    """values [S, N, D] float64, query [R] -> out [N, D] float64 (loops)."""
    sources, tokens, width = values.shape
    rank = query.shape[0]
    out = np.zeros((tokens, width), dtype=np.float64)
    for n in range(tokens):
        logits = []
        for s in range(sources):
            tail = values[s, n, width - rank:]
            mean_square = sum(float(x) * float(x) for x in tail) / rank
            r = math.sqrt(mean_square + eps)
            logits.append(scale * sum(float(tail[i]) / r * float(query[i]) for i in range(rank)))
        top = max(logits)
        weights = [math.exp(z - top) for z in logits]
        total = sum(weights)
        for s in range(sources):
            out[n] += (weights[s] / total) * values[s, n]
    return out


def gradients(values: np.ndarray, query: np.ndarray, grad_out: np.ndarray, eps: float,
              scale: float, step: float = 1e-6) -> tuple[np.ndarray, np.ndarray]:
    """Central differences of L = <grad_out, read(values, query)> in float64."""
    def loss(v, q):
        return float(np.sum(grad_out * read(v, q, eps, scale)))

    grad_values = np.zeros_like(values)
    for index in np.ndindex(values.shape):
        plus, minus = values.copy(), values.copy()
        plus[index] += step
        minus[index] -= step
        grad_values[index] = (loss(plus, query) - loss(minus, query)) / (2 * step)
    grad_query = np.zeros_like(query)
    for i in range(query.shape[0]):
        plus, minus = query.copy(), query.copy()
        plus[i] += step
        minus[i] -= step
        grad_query[i] = (loss(values, plus) - loss(values, minus)) / (2 * step)
    return grad_values, grad_query


__all__ = ["gradients", "read"]
