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
  gets a further per-element allowance on its key coordinates.  Its
  backward takes delta = <dO, o> from the saved BF16 output plus one
  refinement byte per element, which carry o to within a step of
  ulp(bf16(o))/256; dz = p (dw - delta) passes the remaining delta error to
  the key coordinates of dv (`delta_allowance`).  That error is a sum of D
  independent rounding terms, so it grows like sqrt(D): at D = 8192 with a
  peaked softmax it reaches about 1e-3, above any fixed floor that still
  catches mistakes.  The allowance is six standard deviations of the
  modelled error, propagated through dz; a dropped refinement, a dropped
  RMS-norm Jacobian or a 1% error in either key-side coefficient of dv
  still exceeds it by tens to millions of ulps (`tests/test_parity_bounds.py`
  plants such mistakes in copies of the oracle, and emulates the kernel's
  refinement to show that the allowance covers it).

  Differences below 2^-90 are not counted: the GPU flushes FP32 subnormals
  to zero, so a softmax weight p below 2^-126 (exp(-88) and less) becomes 0,
  and with it the whole dv row p (dO + (dw - delta) c) (c the key
  coefficient; `delta_allowance`).  In every test |dO| < 2^8, |c| < 2^6
  (|scale| <= 2, |q| < 2^4, 1/rms < 2^2 wherever p underflows) and
  |dw - delta| <= |v - o| |dO| < D * 2^9 * 2^8 <= 2^30 (D <= 8192,
  |v| < 2^9), so such a row stays below 2^-126 * 2^36 = 2^-90 -- far
  smaller than anything a real mistake moves (a row of 3.3e-36 at
  D = 8192, S = 129 was flushed).  BF16 shares FP32's exponent range, so
  such values would otherwise read as hundreds of ulps.

Every comparison is recorded (max |a - e| and relative L2 against the BF16
oracle, max ulps against the oracle and against float64); with
``ATTNRES_PARITY_TABLE=<path>`` the session writes them as JSON.
"""

from __future__ import annotations

import torch
from torch.utils._python_dispatch import TorchDispatchMode

from oracle.oracle import BF16_TOLERANCE, exact_with_grads, oracle, oracle_float64, softmax_statistics

SEEDS = (20260827, 20260903, 20260911)  # reference validation/protocol.json:7-11

FLOOR = 2.0**-16       # absolute floor, relative to the row's largest magnitude
TINY = 2.0**-90        # absolute floor: rows of flushed (subnormal) softmax weights
STAT_RTOL = 1e-5       # saved statistics: relative tolerance (north_star)
DELTA_SIGMAS = 6.0     # saved-output reads: standard deviations of the delta error allowed


def saves_output(sources: int, width: int, rank: int) -> bool:
    """Whether a read of this shape saves its output and refinement (its
    backward takes delta from them) under the product's policy."""
    from attnres._ops import saves_refinement

    return saves_refinement(sources, width, rank)


def delta_allowance(packed: torch.Tensor, query: torch.Tensor, upstream: torch.Tensor, *,
                    eps: float = 2**-23, scale: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
    """What the saved output's precision adds to the gradients of a saving read.

    ``packed`` ``[S, ..., D]``, ``query`` ``[R]``, ``upstream`` ``[..., D]``
    (float64, exact copies of the BF16 inputs).  The backward of a saving read
    computes delta = <dO, o~> with o~ = bf16(o) + q * u / 256, u = ulp(bf16(o)),
    q the rounded refinement byte, so each element of o~ is off by at most
    u / 512, uniformly distributed; the delta error of token n has standard
    deviation sigma_n = sqrt(sum_i (dO_i u_i / 256)^2) / (2 sqrt 3), and the
    tokens' errors are independent.  It enters dz_s = p_s (dw_s - delta):

    * dv_s on the key coordinates through dz_s * (scale r_s q_i - r_s^2 z_s k_i / R)
      (r = 1/rms, z the scaled logit): the first result is
      ``DELTA_SIGMAS * sigma_n * p_s * |that coefficient|`` there, 0 elsewhere,
      in ``packed``'s shape;
    * dq_i = sum_n sum_s dz_s scale r_s k_i, whose error has variance
      sum_n sigma_n^2 c_ni^2 with c_ni = scale sum_s p_s r_s k_si: the second
      result is that variance ``[R]`` (add it up over token chunks, then take
      ``DELTA_SIGMAS * sqrt``)."""
    sources, width = packed.shape[0], packed.shape[-1]
    flat = packed.reshape(sources, -1, width).double()
    q = query.double()
    rank = q.numel()
    g = upstream.reshape(-1, width).double()
    key = flat[..., width - rank:]
    inv_rms = torch.rsqrt(key.square().mean(-1) + eps)
    logit = (key * inv_rms[..., None] * q).sum(-1) * scale
    weight = logit.softmax(0)
    out = (weight[..., None] * flat).sum(0)
    step = bf16_ulp(out.to(torch.bfloat16)) / 256
    sigma = (g * step).square().sum(-1).sqrt() / (2 * 3**0.5)
    coef = (scale * inv_rms[..., None] * q - (inv_rms * inv_rms * logit / rank)[..., None] * key).abs()
    dv = torch.zeros_like(flat)
    dv[..., width - rank:] = DELTA_SIGMAS * sigma[None, :, None] * weight[..., None] * coef
    c = scale * ((weight * inv_rms)[..., None] * key).sum(0)
    dq_variance = (sigma[:, None] * c).square().sum(0)
    return dv.reshape(packed.shape), dq_variance

RECORDS: list[dict] = []
_CASE = [""]


def set_case(name: str) -> None:
    """Name under which the following comparisons are recorded."""
    _CASE[0] = name


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of BF16 numbers at |x| (float64): 2^(floor(log2|x|) - 7), with the
    subnormal spacing 2^-133 below the smallest normal.  Read off the float64
    exponent field (exact, and much faster than log2/exp2 on large tensors)."""
    bits = x.detach().double().abs().view(torch.int64)
    exponent = ((bits >> 52) & 0x7FF) - 1023
    spacing = exponent.clamp_min(-126) - 7 + 1023
    return (spacing << 52).view(torch.float64)


def _row_floor(reference: torch.Tensor, floor: float = FLOOR) -> torch.Tensor:
    ref = reference.abs()
    if ref.dim() <= 1:
        return floor * ref.max().expand_as(ref) if ref.numel() else ref
    return floor * ref.amax(-1, keepdim=True).expand_as(ref)


def _ulp_excess(actual, reference, floor, extra):
    """Per-element excess in BF16 ulps of ``reference``.  The differences are
    taken in FP32: rounding the float64 reference to FP32 moves it by at most
    2^-24 of itself, 2^-16 of a BF16 ulp."""
    a = actual.detach().cpu().float()
    r64 = reference.detach().cpu()
    r = r64.float()
    excess = (a - r).abs_().sub_(_row_floor(r, floor).clamp_min(TINY))
    if extra is not None:
        excess.sub_(extra.detach().cpu().float())
    return excess.clamp_min_(0.0).div_(_bf16_ulp_f32(r))


def _bf16_ulp_f32(r: torch.Tensor) -> torch.Tensor:
    """`bf16_ulp` of an FP32 tensor, in FP32, from the exponent field (int32
    operations; 2^(e - 134) for the biased exponent e, which is subnormal in
    FP32 below e = 8)."""
    exponent = ((r.view(torch.int32) >> 23) & 0xFF).clamp_min_(1)
    normal = ((exponent - 7).clamp_min_(1) << 23).view(torch.float32)
    subnormal = (torch.ones_like(exponent) << (exponent + 15).clamp_max_(30)).view(torch.float32)
    return torch.where(exponent >= 8, normal, subnormal)


def ulp_error(actual: torch.Tensor, reference: torch.Tensor, floor: float = FLOOR,
              extra: torch.Tensor | None = None) -> float:
    """max over elements of (|a - r| - floor * row max |r| - extra) / ulp(r), at
    least 0; ``extra``: a per-element allowance (`delta_allowance`) or None."""
    if actual.numel() == 0:
        return 0.0
    return float(_ulp_excess(actual, reference, floor, extra).max())


def worst_element(actual: torch.Tensor, reference: torch.Tensor, floor: float = FLOOR,
                  extra: torch.Tensor | None = None, ulps: torch.Tensor | None = None) -> str:
    """The element with the largest ulp excess, for failure messages: its index,
    value, reference, allowance and row maximum (``ulps``: the excess, if
    already computed)."""
    if ulps is None:
        ulps = _ulp_excess(actual, reference, floor, extra)
    flat = int(ulps.argmax())
    index = tuple(int(i) for i in torch.unravel_index(torch.tensor(flat), ulps.shape))
    r = reference.detach().cpu().double()
    row_max = float(r.abs().amax(-1)[index[:-1]]) if r.dim() > 1 else float(r.abs().max())
    allowance = float(extra.detach().cpu().double()[index]) if extra is not None else 0.0
    return (f"worst at {index}: {float(actual.detach().cpu().double()[index]):.9g} vs "
            f"{float(r[index]):.9g} (allowance {allowance:.3g}, row max {row_max:.4g})")


def compare(actual: torch.Tensor, expected: torch.Tensor, *, tol=BF16_TOLERANCE, exact=None,
            ulps: float | None = 1.0, name: str = "", floor: float = FLOOR, extra=None) -> dict:
    """Finite check + the reference's BF16 gate against ``expected`` (BF16
    oracle); with ``exact`` (float64 oracle) also the ulp bound (``extra``: a
    per-element allowance added to the floor).  Returns and records the error
    metrics (reference validation/gpu_checks.py:12-25)."""
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
               "ulp_vs_oracle": ulp_error(actual, expected, floor, extra), "floor": floor,
               "allowance": extra is not None}
    if exact is not None:
        metrics["ulp_vs_float64"] = ulp_error(actual, exact, floor, extra)
        if extra is not None:
            metrics["ulp_vs_float64_floor_only"] = ulp_error(actual, exact, floor)
    RECORDS.append(metrics)
    if exact is not None and ulps is not None:
        assert metrics["ulp_vs_float64"] <= ulps, (
            f"{name or 'result'}: {metrics['ulp_vs_float64']:.3f} BF16 ulps from the float64 oracle "
            f"(bound {ulps}, floor {floor} x row max{' + delta allowance' if extra is not None else ''}); "
            + worst_element(actual, exact, floor, extra))
    return metrics


class Streamed:
    """``compare`` for a result checked chunk by chunk (full-size reads): the
    gate per chunk, the metrics accumulated over the chunks, recorded and the
    ulp bound asserted by ``finish``."""

    def __init__(self, name: str, floor: float = FLOOR, allowance: bool = False):
        self.name = name
        self.floor = floor
        self.allowance = allowance
        self.max_abs = 0.0
        self.diff_sq = 0.0
        self.ref_sq = 0.0
        self.ulp_exact = None
        self.ulp_floor_only = 0.0
        self.worst = ""

    def add(self, actual: torch.Tensor, expected: torch.Tensor, exact: torch.Tensor | None = None,
            extra: torch.Tensor | None = None) -> None:
        if exact is not None:
            assert (extra is not None) == self.allowance, f"{self.name}: allowance expected: {self.allowance}"
        actual = actual.detach().cpu()
        expected = expected.detach().cpu()
        assert actual.shape == expected.shape and actual.dtype == expected.dtype
        assert torch.isfinite(actual.float()).all(), f"{self.name}: non-finite result"
        torch.testing.assert_close(actual, expected, **BF16_TOLERANCE)
        if actual.numel() == 0:
            return
        diff = (actual.float() - expected.float())
        self.max_abs = max(self.max_abs, float(diff.abs().max()))
        self.diff_sq += float(diff.square().sum(dtype=torch.float64))
        self.ref_sq += float(expected.float().square().sum(dtype=torch.float64))
        if exact is not None:
            excess = _ulp_excess(actual, exact, self.floor, extra)
            ulps = float(excess.max())
            if ulps > (self.ulp_exact or 0.0):
                self.worst = worst_element(actual, exact, self.floor, extra, excess)
            self.ulp_exact = max(self.ulp_exact or 0.0, ulps)
            if extra is not None:
                self.ulp_floor_only = max(self.ulp_floor_only, ulp_error(actual, exact, self.floor))

    def finish(self, ulps: float | None = 1.0) -> dict:
        metrics = {"case": _CASE[0], "tensor": self.name, "max_abs": self.max_abs,
                   "rel_l2": (self.diff_sq / max(self.ref_sq, 1e-24)) ** 0.5,
                   "floor": self.floor, "allowance": self.allowance}
        if self.ulp_exact is not None:
            metrics["ulp_vs_float64"] = self.ulp_exact
            if self.allowance:
                metrics["ulp_vs_float64_floor_only"] = self.ulp_floor_only
        RECORDS.append(metrics)
        if self.ulp_exact is not None and ulps is not None:
            assert self.ulp_exact <= ulps, (f"{self.name}: {self.ulp_exact:.3f} BF16 ulps from the float64 oracle "
                                            f"(bound {ulps}, floor {self.floor} x row max); {self.worst}")
        return metrics


def compare_read(actual, expected, exact, names=None, *, sources: int | None = None) -> list[dict]:
    """``compare`` over (out, grad...) tuples from the HIP path, the BF16 oracle
    and the float64 oracle.  When the read's source count is given and the read
    saves its output, value gradients (names starting with "dv") and the query
    gradient ("dq") get the `delta_allowance` that `exact_grads` attached to
    their float64 gradient."""
    names = names or ["out"] + [f"grad{i}" for i in range(len(actual) - 1)]
    width = int(actual[0].shape[-1])
    rank = int(actual[names.index("dq")].numel()) if "dq" in names else width
    saved = sources is not None and saves_output(sources, width, rank)
    metrics = []
    for a, e, x, n in zip(actual, expected, exact, names):
        extra = None
        if saved and (n.startswith("dv") or n == "dq"):
            extra = getattr(x, "dv_allowance" if n.startswith("dv") else "dq_allowance", None)
            assert extra is not None, f"{n}: no delta allowance attached to the float64 gradient"
        metrics.append(compare(a, e, exact=x, name=n, extra=extra))
    return metrics


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
    the BF16 leaves), float64 output and gradients, no rounding.

    Each leaf's float64 gradient carries a ``dv_allowance`` attribute and the
    query's a ``dq_allowance``: the `delta_allowance` of the read mapped onto
    that leaf (through the same ``make_values`` views, by a second autograd
    pass over the linear maps leaves -> values and query leaf -> query), which
    `compare_read` applies to reads that save their output."""
    cpu_leaves = _cpu_leaves(leaves, torch.float64)
    cpu_query = query_leaf.detach().cpu().double().requires_grad_(True)
    values, query = make_values(cpu_leaves, cpu_query)
    g64 = upstream.detach().cpu().double()
    out = oracle_float64(values, query, eps=eps, scale=scale)
    grads = torch.autograd.grad(out, (*cpu_leaves, cpu_query), g64)
    values, query = make_values(cpu_leaves, cpu_query)
    packed = torch.stack(tuple(values)) if isinstance(values, (list, tuple)) else values
    dv_allow, dq_variance = delta_allowance(packed.detach(), query.detach(), g64, eps=eps, scale=scale)
    dq_allow = DELTA_SIGMAS * dq_variance.sqrt()
    mapped = torch.autograd.grad((packed * dv_allow).sum() + (query * dq_allow).sum(), (*cpu_leaves, cpu_query),
                                 allow_unused=True)
    for grad, extra, leaf in zip(grads, mapped, (*cpu_leaves, cpu_query)):
        extra = torch.zeros_like(leaf) if extra is None else extra
        if leaf is cpu_query:
            grad.dq_allowance = extra
        else:
            grad.dv_allowance = extra
    return out, grads


def both_oracles(make_values, leaves, query_leaf, upstream, *, eps=2**-23, scale=1.0):
    """(BF16 oracle results, float64 oracle results), each as (out, *grads)."""
    out, grads = oracle_grads(make_values, leaves, query_leaf, upstream, eps=eps, scale=scale)
    out64, grads64 = exact_grads(make_values, leaves, query_leaf, upstream, eps=eps, scale=scale)
    return (out, *grads), (out64, *grads64)


# ------------------------------------------------------ accumulated gradients

def accumulated_bound(per_read: list, allowances: list, roundings: int, floor: float = FLOOR) -> torch.Tensor:
    """Per-element bound on |result - exact| for a gradient summed over reads.

    ``per_read``: each read's exact (float64) contribution to the gradient;
    ``allowances``: each read's `delta_allowance` on it (None for a read that
    takes delta from the value rows); ``roundings``: how many times the
    running sum is rounded to BF16 (the accumulating BF16 backward rounds once
    per read; FP32 sums never; a BF16 store of an FP32 sum once).  Each
    rounding of a partial sum is at most half an ulp of it, and every partial
    sum is at most the sum of the reads' absolute contributions, so the
    roundings add at most ``roundings / 2`` ulps of that; each read adds its
    FP32 arithmetic (the ``floor`` times its own row maximum, as for a single
    read) and its delta allowance."""
    magnitude = sum(d.abs() for d in per_read)
    bound = 0.5 * roundings * bf16_ulp(magnitude)
    for d in per_read:
        bound = bound + _row_floor(d, floor)
    for extra in allowances:
        if extra is not None:
            bound = bound + extra
    return bound


def check_accumulated(actual: torch.Tensor, exact: torch.Tensor, bound: torch.Tensor, name: str) -> float:
    """Assert |actual - exact| <= bound element by element; return the largest
    ratio of the error to the bound (recorded under the current case)."""
    a = actual.detach().cpu().double()
    x = exact.detach().cpu().double()
    assert torch.isfinite(a).all(), f"{name}: non-finite result"
    error = (a - x).abs()
    ratio = error / bound.clamp_min(TINY)
    worst = float(ratio.max()) if ratio.numel() else 0.0
    RECORDS.append({"case": _CASE[0], "tensor": name, "accumulated_bound_ratio": worst})
    if worst > 1.0:
        index = tuple(int(i) for i in torch.unravel_index(ratio.argmax(), ratio.shape))
        raise AssertionError(f"{name}: error {float(error[index]):.4g} at {index} is {worst:.3g} x its bound "
                             f"{float(bound[index]):.4g} (result {float(a[index]):.6g}, exact {float(x[index]):.6g})")
    return worst


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


# ------------------------------------------------------- no source stack

class SourceStackGuard(TorchDispatchMode):
    """Fails on ``aten.stack`` / ``aten.cat`` of the read's sources: a list of
    ``count`` (or ``count + 1``) tensors, all of one of the sources' shapes
    (or that shape with a leading 1)."""

    def __init__(self, shapes, count):
        super().__init__()
        self.shapes = {tuple(shape) for shape in shapes}
        self.counts = {count, count + 1}
        self.seen = 0

    @classmethod
    def ignore_compile_internals(cls):
        return True  # watch the compiled artefact, not dynamo's own tracing

    def _is_source(self, shape):
        return shape in self.shapes or (len(shape) > 1 and shape[0] == 1 and shape[1:] in self.shapes)

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        self.seen += 1
        if func in (torch.ops.aten.stack.default, torch.ops.aten.cat.default) and args and args[0]:
            shapes = [tuple(t.shape) for t in args[0]]
            if len(shapes) in self.counts and len(set(shapes)) == 1 and self._is_source(shapes[0]):
                raise AssertionError(f"the source-list path stacked its sources ({func})")
        return func(*args, **(kwargs or {}))


__all__ = ["DELTA_SIGMAS", "FLOOR", "RECORDS", "SEEDS", "STAT_RTOL", "SourceStackGuard", "Streamed", "accumulated_bound", "check_accumulated", "both_oracles", "bf16_ulp",
           "check_statistics", "delta_allowance", "saves_output", "worst_element",
           "compare", "compare_read", "exact_grads", "exact_with_grads", "kernel_statistics", "oracle_grads",
           "set_case", "ulp_error"]
