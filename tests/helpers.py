"""Shared helpers for the parity tests (inputs, comparisons, error records).

Two bars are applied to every HIP result:

* the reference's BF16 gate against the BF16 oracle, ``rtol = atol = 0.05``
  (`validation/protocol.json:12-15`, `validation/comparison.py:5-12`);
* a BF16-ulp bound against `oracle_float64` (the same read in float64, no
  rounding).  The kernels compute in FP32 and round once, so each result is
  within one BF16 ulp of the exact value, up to FP32 noise; the noise is
  covered by an absolute floor of ``2^-16`` times the largest magnitude in
  the element's row (its token row for out and dv, the whole vector for dq),
  far below what a dropped term or a wrong index moves.

  The value gradient of a read that saves its output (more than 6 sources)
  gets a floor of ``2^-13`` instead: its backward takes delta = <dO, o> from
  the saved BF16 output plus one refinement byte per element, which carry o
  to 1/512 of a BF16 ulp and delta to about 2^-17 relative, and dz =
  p (dw - delta) passes that on to the key coordinates of dv.  On the test
  inputs that error stays below 2^-14 of the row maximum, while a dropped
  refinement, a dropped RMS-norm Jacobian, or a 1% error in either key-side
  coefficient of dv exceeds the 2^-13 bound by tens to millions of ulps
  (`tests/test_parity_bounds.py` plants such mistakes in copies of the oracle).

  Differences below 2^-118 are not counted: the GPU flushes FP32 subnormals
  to zero, so a softmax weight below 2^-126 (exp(-88) and less) becomes 0 and
  its dv = p dO (at most 2^-126 |dO|, and |dO| < 2^8 in every test) becomes 0
  too; BF16 shares FP32's exponent range, so such values would otherwise
  read as hundreds of subnormal ulps.

Every comparison is recorded (max |a - e| and relative L2 against the BF16
oracle, max ulps against the oracle and against float64); with
``ATTNRES_PARITY_TABLE=<path>`` the session writes them as JSON.
"""

from __future__ import annotations

import torch

from oracle.oracle import BF16_TOLERANCE, exact_with_grads, oracle, oracle_float64, softmax_statistics

SEEDS = (20260827, 20260903, 20260911)  # reference validation/protocol.json:7-11

FLOOR = 2.0**-16       # absolute floor, relative to the row's largest magnitude
SAVED_DV_FLOOR = 2.0**-13  # dv of a read that saves its output (delta from the refinement)
TINY = 2.0**-118           # absolute floor: FP32 subnormals (< 2^-126) flushed, times |dO| < 2^8
STAT_RTOL = 1e-5       # saved statistics: relative tolerance (north_star)


def dv_floor(sources: int) -> float:
    """The dv floor for a read of ``sources`` sources under the product's
    save/recompute policy."""
    from attnres._ops import saves_refinement

    return SAVED_DV_FLOOR if saves_refinement(sources) else FLOOR

RECORDS: list[dict] = []
_CASE = [""]


def set_case(name: str) -> None:
    """Name under which the following comparisons are recorded."""
    _CASE[0] = name


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of BF16 numbers at |x| (float64): 2^(floor(log2|x|) - 7), with the
    subnormal spacing 2^-133 below the smallest normal."""
    ax = x.double().abs().clamp_min(2.0**-126)
    return torch.exp2(torch.floor(torch.log2(ax)) - 7)


def _row_floor(reference: torch.Tensor, floor: float = FLOOR) -> torch.Tensor:
    ref = reference.double().abs()
    if ref.dim() <= 1:
        return floor * ref.max().expand_as(ref) if ref.numel() else ref
    return floor * ref.amax(-1, keepdim=True).expand_as(ref)


def ulp_error(actual: torch.Tensor, reference: torch.Tensor, floor: float = FLOOR) -> float:
    """max over elements of (|a - r| - floor * row max |r|) / ulp(r), at least 0."""
    if actual.numel() == 0:
        return 0.0
    a, r = actual.detach().cpu().double(), reference.detach().cpu().double()
    excess = ((a - r).abs() - _row_floor(r, floor).clamp_min(TINY)).clamp_min(0.0)
    return float((excess / bf16_ulp(r)).max())


def compare(actual: torch.Tensor, expected: torch.Tensor, *, tol=BF16_TOLERANCE, exact=None,
            ulps: float | None = 1.0, name: str = "", floor: float = FLOOR) -> dict:
    """Finite check + the reference's BF16 gate against ``expected`` (BF16
    oracle); with ``exact`` (float64 oracle) also the ulp bound.  Returns and
    records the error metrics (reference validation/gpu_checks.py:12-25)."""
    actual = actual.detach().cpu()
    expected = expected.detach().cpu()
    assert torch.isfinite(actual.float()).all(), "non-finite result"
    assert torch.isfinite(expected.float()).all(), "non-finite oracle result"
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    assert actual.dtype == expected.dtype, (actual.dtype, expected.dtype)
    torch.testing.assert_close(actual, expected, **tol)
    diff = (actual.float() - expected.float()).abs()
    metrics = {"case": _CASE[0], "tensor": name,
               "max_abs": float(diff.max()) if diff.numel() else 0.0,
               "rel_l2": float(diff.norm() / expected.float().norm().clamp_min(1e-12)),
               "ulp_vs_oracle": ulp_error(actual, expected, floor), "floor": floor}
    if exact is not None:
        metrics["ulp_vs_float64"] = ulp_error(actual, exact, floor)
    RECORDS.append(metrics)
    if exact is not None and ulps is not None:
        assert metrics["ulp_vs_float64"] <= ulps, (
            f"{name or 'result'}: {metrics['ulp_vs_float64']:.3f} BF16 ulps from the float64 oracle "
            f"(bound {ulps}, floor {floor} x row max)")
    return metrics


class Streamed:
    """``compare`` for a result checked chunk by chunk (full-size reads): the
    gate per chunk, the metrics accumulated over the chunks, recorded and the
    ulp bound asserted by ``finish``."""

    def __init__(self, name: str, floor: float = FLOOR):
        self.name = name
        self.floor = floor
        self.max_abs = 0.0
        self.diff_sq = 0.0
        self.ref_sq = 0.0
        self.ulp_oracle = 0.0
        self.ulp_exact = None

    def add(self, actual: torch.Tensor, expected: torch.Tensor, exact: torch.Tensor | None = None) -> None:
        actual = actual.detach().cpu()
        expected = expected.detach().cpu()
        assert actual.shape == expected.shape and actual.dtype == expected.dtype
        assert torch.isfinite(actual.float()).all(), f"{self.name}: non-finite result"
        torch.testing.assert_close(actual, expected, **BF16_TOLERANCE)
        diff = (actual.float() - expected.float())
        self.max_abs = max(self.max_abs, float(diff.abs().max()) if diff.numel() else 0.0)
        self.diff_sq += float(diff.double().square().sum())
        self.ref_sq += float(expected.double().square().sum())
        self.ulp_oracle = max(self.ulp_oracle, ulp_error(actual, expected, self.floor))
        if exact is not None:
            self.ulp_exact = max(self.ulp_exact or 0.0, ulp_error(actual, exact, self.floor))

    def finish(self, ulps: float | None = 1.0) -> dict:
        metrics = {"case": _CASE[0], "tensor": self.name, "max_abs": self.max_abs,
                   "rel_l2": (self.diff_sq / max(self.ref_sq, 1e-24)) ** 0.5, "ulp_vs_oracle": self.ulp_oracle,
                   "floor": self.floor}
        if self.ulp_exact is not None:
            metrics["ulp_vs_float64"] = self.ulp_exact
        RECORDS.append(metrics)
        if self.ulp_exact is not None and ulps is not None:
            assert self.ulp_exact <= ulps, (f"{self.name}: {self.ulp_exact:.3f} BF16 ulps from the float64 oracle "
                                            f"(bound {ulps}, floor {self.floor} x row max)")
        return metrics


def compare_read(actual, expected, exact, names=None, *, sources: int | None = None) -> list[dict]:
    """``compare`` over (out, grad...) tuples from the HIP path, the BF16 oracle
    and the float64 oracle; value gradients (names starting with "dv") get
    ``dv_floor(sources)`` when the read's source count is given."""
    names = names or ["out"] + [f"grad{i}" for i in range(len(actual) - 1)]
    floor_dv = FLOOR if sources is None else dv_floor(sources)
    return [compare(a, e, exact=x, name=n, floor=floor_dv if n.startswith("dv") else FLOOR)
            for a, e, x, n in zip(actual, expected, exact, names)]


def _cpu_leaves(leaves, dtype):
    return [leaf.detach().cpu().to(dtype).requires_grad_(True) for leaf in leaves]


def oracle_grads(make_values, leaves, query_leaf, upstream, *, eps=2**-23, scale=1.0):
    """Oracle output and grads w.r.t. CPU copies of the given leaves.

    `make_values(leaves, query)` builds the operator inputs from the leaves
    (views, lists) exactly as the GPU side does."""
    cpu_leaves = _cpu_leaves(leaves, torch.bfloat16)
    cpu_query = query_leaf.detach().cpu().requires_grad_(True)
    values, query = make_values(cpu_leaves, cpu_query)
    out = oracle(values, query, eps=eps, scale=scale)
    grads = torch.autograd.grad(out, (*cpu_leaves, cpu_query), upstream.detach().cpu())
    return out, grads


def exact_grads(make_values, leaves, query_leaf, upstream, *, eps=2**-23, scale=1.0):
    """`oracle_grads` through `oracle_float64`: float64 leaves (exact copies of
    the BF16 leaves), float64 output and gradients, no rounding."""
    cpu_leaves = _cpu_leaves(leaves, torch.float64)
    cpu_query = query_leaf.detach().cpu().double().requires_grad_(True)
    values, query = make_values(cpu_leaves, cpu_query)
    out = oracle_float64(values, query, eps=eps, scale=scale)
    grads = torch.autograd.grad(out, (*cpu_leaves, cpu_query), upstream.detach().cpu().double())
    return out, grads


def both_oracles(make_values, leaves, query_leaf, upstream, *, eps=2**-23, scale=1.0):
    """(BF16 oracle results, float64 oracle results), each as (out, *grads)."""
    out, grads = oracle_grads(make_values, leaves, query_leaf, upstream, eps=eps, scale=scale)
    out64, grads64 = exact_grads(make_values, leaves, query_leaf, upstream, eps=eps, scale=scale)
    return (out, *grads), (out64, *grads64)


# ------------------------------------------------------------- statistics

def kernel_statistics(values, query, eps, scale):
    """The forward op's saved ``logit[N, S]``, ``inv_rms[N, S]``, ``stats[2, N]``
    for packed ``[S, N, D]`` values or a list of ``[N, D]`` sources."""
    import attnres._ops  # noqa: F401  (registers the ops)

    if isinstance(values, (list, tuple)):
        result = torch.ops.attnres_hip.sources_forward(list(values), query, eps, scale)
    else:
        result = torch.ops.attnres_hip.packed_forward(values, query, eps, scale)
    return result[2], result[3], result[4]


def check_statistics(values, query, *, eps=2**-23, scale=1.0, chunk: int = 4096) -> dict:
    """The kernels' saved statistics against `softmax_statistics` (FP32 oracle).

    * ``inv_rms`` within ``STAT_RTOL`` relative (a sum of squares: no cancellation);
    * ``logit`` within ``STAT_RTOL`` relative to the sum of the absolute
      products it adds up, ``|scale| * sum_i |k_i q_i|`` (taken from the oracle
      on |values| and |query|), which is the logit's own size unless the dot
      cancels;
    * ``stats[0]`` (max) as the largest logit bound of the token; ``stats[1]``
      (1/sum) within ``STAT_RTOL`` plus twice that bound relative, since it
      moves with the logits' differences.
    Large inputs are compared in token chunks."""
    logit, inv_rms, stats = (t.detach().cpu() for t in kernel_statistics(values, query, eps, scale))
    listed = isinstance(values, (list, tuple))
    tokens = int(values[0].shape[0]) if listed else int(values.shape[1])
    cpu_query = query.detach().cpu()
    worst = {"logit": 0.0, "inv_rms": 0.0, "max": 0.0, "inv_sum": 0.0}
    for start in range(0, tokens, chunk):
        stop = min(tokens, start + chunk)
        part = (torch.stack([v[start:stop].detach().cpu() for v in values]) if listed
                else values[:, start:stop].detach().cpu())
        e_logit, e_inv, e_stats = softmax_statistics(part, cpu_query, eps=eps, scale=scale)
        size, _, _ = softmax_statistics(part.abs(), cpu_query.abs(), eps=eps, scale=abs(scale))
        size = size.double()
        bound_z = STAT_RTOL * (e_logit.double().abs() + size)
        z_err = (logit[start:stop].double() - e_logit.double()).abs()
        worst["logit"] = max(worst["logit"], float((z_err / bound_z.clamp_min(1e-30)).max()))
        r_err = (inv_rms[start:stop].double() / e_inv.double() - 1).abs()
        worst["inv_rms"] = max(worst["inv_rms"], float(r_err.max()) / STAT_RTOL)
        token_bound = bound_z.amax(1)
        m_err = (stats[0, start:stop].double() - e_stats[0].double()).abs()
        worst["max"] = max(worst["max"], float((m_err / token_bound.clamp_min(1e-30)).max()))
        s_err = (stats[1, start:stop].double() / e_stats[1].double() - 1).abs()
        s_bound = STAT_RTOL + 2 * token_bound
        worst["inv_sum"] = max(worst["inv_sum"], float((s_err / s_bound).max()))
    RECORDS.append({"case": _CASE[0], "tensor": "statistics", **{f"{k}_of_bound": v for k, v in worst.items()}})
    for key, value in worst.items():
        assert value <= 1.0, f"saved {key}: {value:.3g} x its bound (rtol {STAT_RTOL})"
    return worst


__all__ = ["FLOOR", "RECORDS", "SAVED_DV_FLOOR", "SEEDS", "STAT_RTOL", "Streamed", "both_oracles", "dv_floor", "bf16_ulp", "check_statistics",
           "compare", "compare_read", "exact_grads", "exact_with_grads", "kernel_statistics", "oracle_grads",
           "set_case", "ulp_error"]
