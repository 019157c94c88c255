"""Pin the CPU oracle (oracle/oracle.py) before trusting it as the checker.

Each oracle function is checked against something that does not restate its
formula:

* a float64 brute-force loop of the operator's equation (oracle/exact.py,
  reference docs/equation.md:44-55) for the forward value;
* central finite differences of <dO, read(values, query)> in float64 for the
  first-order gradients (no analytic backward is written down anywhere in
  the check);
* the closed-form known-answer cases of the reference's own tests:
  zero keys (tests/test_routing_checks.py:10-24), zero scale
  (tests/test_routing_checks.py:39-47), equal logits at |scale| = 2^24
  (validation/softmax_checks.py:9-30, tests/test_softmax_stats.py:6-15), a
  single source (envelope shape (1, 1, 1, 1), tests/test_full_kernel.py:121),
  autocast independence and the BF16-only boundary
  (tests/test_bf16_oracle.py:8-33);
* mutation checks: plausible mistakes (wrong key slice, softmax over the
  wrong axis, dropped eps, a sign flip, first-R key) planted in CPU copies of
  the oracle must fail the brute-force comparison, so the comparison is
  strong enough to pin the oracle.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import exact
from oracle.oracle import (EPS, chunked_with_grads, exact_with_grads, oracle, oracle_float64, oracle_with_grads,
                           softmax_statistics)

BF16_ULP = 2.0**-8  # relative spacing of BF16 (8 significant bits)


def _case(seed: int, sources: int, tokens: int, width: int, rank: int, spread: float = 1.0):
    generator = torch.Generator().manual_seed(seed)
    values = (torch.randn(sources, tokens, width, generator=generator) *
              (torch.rand(sources, 1, 1, generator=generator) * 3.5 + 0.5) * spread).to(torch.bfloat16)
    query = (torch.randn(rank, generator=generator) / math.sqrt(rank)).to(torch.bfloat16)
    upstream = torch.randn(tokens, width, generator=generator).to(torch.bfloat16)
    return values, query, upstream


def _f64(tensor: torch.Tensor) -> np.ndarray:
    return tensor.detach().double().numpy()


def _within_bf16(actual: torch.Tensor, exact_value: np.ndarray, ulps: float, floor: float) -> None:
    """|actual - exact| <= ulps * BF16 ulp of |exact| (plus an absolute floor)."""
    diff = np.abs(_f64(actual) - exact_value)
    bound = ulps * BF16_ULP * np.abs(exact_value) + floor
    worst = float(np.max(diff - bound))
    assert worst <= 0.0, f"exceeds the bound by {worst:.3g} (max diff {diff.max():.3g})"


# ------------------------------------------------------------- brute force

@pytest.mark.parametrize("seed,shape,scale,eps", [
    (20260827, (3, 4, 12, 12), 1.0, EPS),
    (20260903, (5, 3, 16, 5), 0.7, EPS),
    (20260911, (2, 6, 9, 3), -1.5, 2.0**-10),
    (7, (7, 2, 24, 24), 4.0, 1e-3),
])
def test_forward_matches_float64_brute_force(seed, shape, scale, eps):
    sources, tokens, width, rank = shape
    values, query, _ = _case(seed, sources, tokens, width, rank)
    expected = exact.read(_f64(values), _f64(query), eps, scale)
    actual = oracle(values, query, eps=eps, scale=scale)
    # FP32 internal arithmetic then one BF16 rounding: within one BF16 ulp.
    _within_bf16(actual, expected, ulps=1.0, floor=1e-6)


@pytest.mark.parametrize("seed,shape,scale,eps", [
    (20260905, (3, 2, 6, 4), 1.0, EPS),
    (20260906, (4, 2, 5, 5), -0.75, 2.0**-10),
    (11, (2, 3, 7, 2), 2.5, 1e-2),
])
def test_gradients_match_float64_finite_differences(seed, shape, scale, eps):
    sources, tokens, width, rank = shape
    values, query, upstream = _case(seed, sources, tokens, width, rank)
    _, grad_values, grad_query = oracle_with_grads(values, query, upstream, eps=eps, scale=scale)
    fd_values, fd_query = exact.gradients(_f64(values), _f64(query), _f64(upstream), eps, scale)
    # BF16 gradients.  The key tail of dv is the BF16 sum of two separately
    # rounded BF16 parts (direct + routing) that may cancel, so the absolute
    # error scales with the parts: bound it by two ulps of the element plus
    # one ulp of the tensor's largest magnitude.
    _within_bf16(grad_values, fd_values, ulps=2.0, floor=BF16_ULP * np.abs(fd_values).max())
    _within_bf16(grad_query, fd_query, ulps=2.0, floor=BF16_ULP * np.abs(fd_query).max())


def test_list_and_packed_forms_agree_bitwise():
    values, query, upstream = _case(3, 4, 3, 10, 6)
    packed = oracle_with_grads(values, query, upstream, scale=0.9)
    listed = oracle_with_grads(list(values.unbind(0)), query, upstream, scale=0.9)
    assert torch.equal(packed[0], listed[0])
    assert torch.equal(packed[1], torch.stack(listed[1]))
    assert torch.equal(packed[2], listed[2])


def test_softmax_statistics_match_float64():
    values, query, _ = _case(5, 6, 4, 16, 8)
    logit, inv_rms, stats = softmax_statistics(values, query, scale=1.3)
    v, q = _f64(values), _f64(query)
    tail = v[..., -8:]
    r = np.sqrt((tail**2).mean(-1) + EPS)
    z = 1.3 * (tail / r[..., None] * q).sum(-1)
    np.testing.assert_allclose(logit.T.double().numpy(), z, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(inv_rms.T.double().numpy(), 1 / r, rtol=1e-5)
    np.testing.assert_allclose(stats[0].double().numpy(), z.max(0), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(stats[1].double().numpy(), 1 / np.exp(z - z.max(0)).sum(0), rtol=1e-5)


# -------------------------------------------------------------- mutations

def _mutant(kind: str):
    """A copy of the oracle with one planted mistake (CPU only)."""
    def read(values, query, *, eps=EPS, scale=1.0):
        rank = query.numel()
        value = values.float()
        if kind == "first_r_key":
            key = values[..., :rank].float()
        else:
            key = values[..., values.shape[-1] - rank:].float()
        mean_square = key.square().mean(-1, keepdim=True)
        inv_rms = torch.rsqrt(mean_square if kind == "no_eps" else mean_square + eps)
        if kind == "no_norm":
            inv_rms = torch.ones_like(inv_rms)
        logit = (key * inv_rms * query.float()).sum(-1) * (-scale if kind == "sign" else scale)
        weight = logit.softmax(-1 if kind == "wrong_axis" else 0)
        return (weight.unsqueeze(-1) * value).sum(0).to(torch.bfloat16)
    return read


@pytest.mark.parametrize("kind", ["first_r_key", "no_norm", "sign", "wrong_axis", "no_eps"])
def test_brute_force_check_rejects_planted_mistakes(kind):
    eps = 0.5 if kind == "no_eps" else EPS  # a large eps makes a dropped eps visible
    values, query, _ = _case(99, 4, 3, 12, 6)
    expected = exact.read(_f64(values), _f64(query), eps, 1.0)
    with pytest.raises(AssertionError):
        _within_bf16(_mutant(kind)(values, query, eps=eps), expected, ulps=1.0, floor=1e-6)
    _within_bf16(oracle(values, query, eps=eps), expected, ulps=1.0, floor=1e-6)


# ----------------------------------------------------- known-answer cases

def test_zero_keys_have_closed_form_gradients():
    """Zero keys: p = 1/S, dk = scale*dz*q/sqrt(eps) and dq == 0 exactly
    (reference tests/test_routing_checks.py:10-24)."""
    torch.manual_seed(20260906)
    sources, rows, width, rank = 4, 3, 32, 16
    eps, scale = 2**-10, -0.75
    values = torch.randn(sources, rows, width).to(torch.bfloat16)
    values[..., :-rank] += torch.arange(sources, dtype=torch.bfloat16)[:, None, None]
    values[..., -rank:] = 0
    query = (torch.randn(rank) * 0.05).to(torch.bfloat16)
    upstream = torch.randn(rows, width).to(torch.bfloat16)
    _, dv, dq = oracle_with_grads(values, query, upstream, eps=eps, scale=scale)
    v, g, q = values.float(), upstream.float(), query.float()
    dz = ((v - v.mean(0)) * g).sum(-1) / sources
    dk = scale * dz[..., None] * q / math.sqrt(eps)
    assert torch.count_nonzero(dk) == dk.numel()
    torch.testing.assert_close(dv[..., -rank:], (g[None, ..., -rank:] / sources + dk).to(torch.bfloat16),
                               rtol=0.05, atol=0.05)
    torch.testing.assert_close(dq, torch.zeros_like(query), rtol=0, atol=0)


def test_zero_scale_is_a_uniform_average_exactly():
    """scale = 0: dv == dO/S and dq == 0 exactly (tests/test_routing_checks.py:39-47)."""
    values, query, upstream = _case(20260827, 4, 2, 32, 16)
    out, dv, dq = oracle_with_grads(values, query, upstream, eps=2**-10, scale=0.0)
    torch.testing.assert_close(dv, upstream.expand_as(values) / 4, rtol=0, atol=0)
    torch.testing.assert_close(dq, torch.zeros_like(query), rtol=0, atol=0)
    torch.testing.assert_close(out, values.float().mean(0).to(torch.bfloat16), rtol=0, atol=0)


@pytest.mark.parametrize("sources", [2, 4])
@pytest.mark.parametrize("scale", [2**24, -(2**24)])
def test_equal_large_logits_are_exact(sources, scale):
    """Identical sources at |scale| = 2^24: out == v, dv == dO/S, dq == 0
    exactly (validation/softmax_checks.py:9-30)."""
    values = torch.ones(sources, 2, 256, dtype=torch.bfloat16)
    query = torch.ones(16, dtype=torch.bfloat16)
    for factor in (1.0, -2.0, 4.0):
        upstream = torch.full((2, 256), factor, dtype=torch.bfloat16)
        out, dv, dq = oracle_with_grads(values, query, upstream, scale=scale)
        torch.testing.assert_close(out, values[0], rtol=0, atol=0)
        torch.testing.assert_close(dv, upstream.expand_as(values) / sources, rtol=0, atol=0)
        torch.testing.assert_close(dq, torch.zeros_like(query), rtol=0, atol=0)


@pytest.mark.parametrize("scale", [2**24, -(2**24)])
def test_two_part_statistics_keep_large_common_offsets(scale):
    """A single FP32 log-sum-exp loses the normaliser at logits ~2^24; the
    separate (max, 1/sum) statistics keep it (tests/test_softmax_stats.py:6-15)."""
    values = torch.ones(4, 2, 16, dtype=torch.bfloat16)
    query = torch.ones(16, dtype=torch.bfloat16)
    logit, _, stats = softmax_statistics(values, query, scale=scale)
    logit = logit.T
    lossy = (logit - (stats[0] + (1 / stats[1]).log())).exp()
    assert torch.equal(lossy, torch.ones_like(lossy))  # the information a single LSE loses
    two_part = (logit - stats[0]).exp() * stats[1]
    torch.testing.assert_close(two_part, torch.full_like(two_part, 0.25), rtol=0, atol=0)


def test_single_source_is_identity():
    values, query, upstream = _case(20260903, 1, 5, 20, 20)
    out, dv, dq = oracle_with_grads(values, query, upstream)
    assert torch.equal(out, values[0])
    assert torch.equal(dv[0], upstream)
    assert torch.equal(dq, torch.zeros_like(query))


@pytest.mark.parametrize("sequence", [False, True])
def test_autocast_does_not_change_the_oracle(sequence):
    """BF16 in and out, identical bits with autocast on or off
    (tests/test_bf16_oracle.py:8-27)."""
    values, query, upstream = _case(19, 5, 3, 17, 7)
    results = []
    for enabled in (False, True):
        with torch.autocast(device_type="cpu", dtype=torch.bfloat16, enabled=enabled):
            inputs = list(values.unbind()) if sequence else values
            result = oracle_with_grads(inputs, query, upstream, scale=0.7)
        flat = (result[0], *(result[1] if sequence else [result[1]]), result[2])
        assert all(tensor.dtype == torch.bfloat16 for tensor in flat)
        results.append(flat)
    for actual, expected in zip(*results):
        assert torch.equal(actual, expected)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_oracle_rejects_other_floating_dtypes(dtype):
    with pytest.raises(TypeError, match="requires BF16"):
        oracle(torch.ones(2, 3, 16, dtype=dtype), torch.ones(16, dtype=dtype))


# ----------------------------------------------------- float64 and chunked

@pytest.mark.parametrize("seed,shape,scale,eps", [
    (20260827, (3, 4, 12, 12), 1.0, EPS),
    (20260911, (2, 6, 9, 3), -1.5, 2.0**-10),
    (7, (7, 2, 24, 24), 4.0, 1e-3),
])
def test_float64_oracle_matches_brute_force_and_finite_differences(seed, shape, scale, eps):
    sources, tokens, width, rank = shape
    values, query, upstream = _case(seed, sources, tokens, width, rank)
    out, grad_values, grad_query = exact_with_grads(values, query, upstream, eps=eps, scale=scale)
    assert out.dtype == grad_values.dtype == grad_query.dtype == torch.float64
    expected = exact.read(_f64(values), _f64(query), eps, scale)
    np.testing.assert_allclose(out.numpy(), expected, rtol=1e-12, atol=1e-13)
    fd_values, fd_query = exact.gradients(_f64(values), _f64(query), _f64(upstream), eps, scale)
    scale_v, scale_q = np.abs(fd_values).max(), np.abs(fd_query).max()
    np.testing.assert_allclose(grad_values.numpy(), fd_values, rtol=1e-6, atol=1e-7 * scale_v)
    np.testing.assert_allclose(grad_query.numpy(), fd_query, rtol=1e-6, atol=1e-7 * scale_q)
    # the BF16 oracle is the float64 one plus its roundings
    _within_bf16(oracle(values, query, eps=eps, scale=scale), out.numpy(), ulps=1.0, floor=1e-6)


def test_float64_oracle_rejects_planted_mistakes():
    """A wrong-axis softmax or a first-R key in float64 fails the 1e-12 check."""
    values, query, _ = _case(99, 4, 3, 12, 6)
    expected = exact.read(_f64(values), _f64(query), EPS, 1.0)
    good = oracle_float64(values.double(), query.double())
    np.testing.assert_allclose(good.numpy(), expected, rtol=1e-12, atol=1e-13)
    for kind in ("first_r_key", "wrong_axis", "sign"):
        bad = _mutant(kind)(values, query).double().numpy()  # BF16 mutant: far beyond 1e-12
        with pytest.raises(AssertionError):
            np.testing.assert_allclose(bad, expected, rtol=1e-4, atol=1e-4)


def test_float64_oracle_rejects_other_dtypes():
    with pytest.raises(TypeError, match="float64"):
        oracle_float64(torch.ones(2, 3, 16, dtype=torch.bfloat16), torch.ones(16, dtype=torch.bfloat16))


@pytest.mark.parametrize("listed", [False, True])
def test_chunked_oracle_equals_the_whole_read(listed):
    values, query, upstream = _case(23, 5, 37, 24, 10)
    whole = oracle_with_grads(list(values.unbind()) if listed else values, query, upstream, scale=0.8)
    chunked = chunked_with_grads(list(values.unbind()) if listed else values, query, upstream, scale=0.8,
                                 chunk=8)
    assert torch.equal(chunked[0], whole[0])
    grads = torch.stack(chunked[1]) if listed else chunked[1]
    expected = torch.stack(whole[1]) if listed else whole[1]
    assert torch.equal(grads, expected)
    # dq: FP32 chunk sums rounded once, against one FP32 sum rounded once
    torch.testing.assert_close(chunked[2].float(), whole[2].float(), rtol=BF16_ULP, atol=0)
    exact_whole = exact_with_grads(values, query, upstream, scale=0.8)
    exact_chunked = chunked_with_grads(values, query, upstream, scale=0.8, chunk=8, exact=True)
    for a, e in zip(exact_chunked, exact_whole):
        np.testing.assert_allclose(a.numpy(), e.numpy(), rtol=1e-12, atol=1e-13)
