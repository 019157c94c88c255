"""The GPU parity bounds (tests/helpers.py) are strong enough to catch real mistakes.

The kernels' value gradients are held to one BF16 ulp of the float64 oracle,
up to a floor of 2^-16 times the row's largest magnitude; a read that saves
its output (its backward takes delta = <dO, o> from the BF16 output plus one
refinement byte per element) also gets `helpers.delta_allowance` on its key
coordinates.  Here, on the CPU:

* the kernel's saved-output backward is emulated in float64 (delta from the
  BF16 output and the rounded refinement byte, as `refine_encode` stores it)
  and its BF16-rounded dv must meet the bound with the allowance, including
  the shapes where the delta error is largest (S = 129, D = 8192, peaked
  softmax);
* plausible mistakes, planted in copies of the oracle's arithmetic
  (`oracle.oracle._mix` in float64) or of the emulated backward, must fail it:
  the RMS-norm Jacobian dropped (``inv_rms`` treated as a constant) or scaled
  by 1.01, the whole routing gradient (through the logit) scaled by 1.01, and
  the refinement dropped (delta from the BF16 output alone);
* the correctly rounded float64 gradient passes at half an ulp.

Inputs: peaked softmax (query x 0.25, as in the envelope tests), the
BASELINE distribution of c2 (R = D) and of c3 (sliced, R = D/4), and a
small rank.
"""

from __future__ import annotations

import math

import pytest
import torch

import bench
from helpers import DELTA_SIGMAS, FLOOR, bf16_ulp, delta_allowance, ulp_error
from oracle.oracle import _packed, exact_with_grads


class _ScaleGrad(torch.autograd.Function):
    """Identity forward; the gradient scaled by ``factor`` (a planted mistake)."""

    @staticmethod
    def forward(ctx, tensor, factor):
        ctx.factor = factor
        return tensor.view_as(tensor)

    @staticmethod
    def backward(ctx, grad):
        return grad * ctx.factor, None


def _mutant_grads(values, query, grad_out, mistake, eps=2**-23, scale=1.0):
    """dv of a float64 copy of the oracle's read with one planted mistake."""
    leaf = values.detach().double().requires_grad_(True)
    q = query.detach().double()
    packed = _packed(leaf)
    key = packed[..., packed.shape[-1] - q.numel():]
    inv_rms = torch.rsqrt(key.square().mean(-1, keepdim=True) + eps)
    if mistake == "rms_jacobian_dropped":
        inv_rms = inv_rms.detach()
    elif mistake == "rms_jacobian_1pct":
        inv_rms = _ScaleGrad.apply(inv_rms, 1.01)
    logit = (key * inv_rms * q).sum(-1) * scale
    if mistake == "routing_1pct":
        logit = _ScaleGrad.apply(logit, 1.01)
    out = (logit.softmax(0).unsqueeze(-1) * packed).sum(0)
    return torch.autograd.grad(out, leaf, grad_out.double())[0]


def _emulated_saved_grads(values, query, grad_out, refine=True, eps=2**-23, scale=1.0):
    """(dv, dq) of the saving backward in float64: delta = <dO, o~> with o~ the
    BF16 output plus its refinement byte (o - bf16(o) in steps of ulp/256,
    rounded, clamped to +-127), or the BF16 output alone when ``refine`` is
    False; every other quantity exact."""
    v = values.double()
    q = query.double()
    g = grad_out.double()
    width, rank = v.shape[-1], q.numel()
    key = v[..., width - rank:]
    inv_rms = torch.rsqrt(key.square().mean(-1) + eps)
    logit = (key * inv_rms[..., None] * q).sum(-1) * scale
    weight = logit.softmax(0)
    out = (weight[..., None] * v).sum(0)
    rounded = out.float().to(torch.bfloat16).double()
    stored = rounded
    if refine:
        unit = bf16_ulp(rounded) / 256
        stored = rounded + torch.clamp(torch.round((out - rounded) / unit), -127, 127) * unit
    delta = (g * stored).sum(-1)
    dz = weight * ((v * g).sum(-1) - delta)
    dv = weight[..., None] * g
    dv[..., width - rank:] += dz[..., None] * (scale * inv_rms[..., None] * q -
                                               (inv_rms * inv_rms * logit / rank)[..., None] * key)
    dq = (dz[..., None] * scale * inv_rms[..., None] * key).sum((0, 1))
    return dv, dq


def _cases():
    generator = torch.Generator().manual_seed(20260827)
    peaked = (torch.randn(9, 48, 1024, generator=generator).to(torch.bfloat16),
              (torch.randn(1024, generator=generator) * 0.25).to(torch.bfloat16),
              torch.randn(48, 1024, generator=generator).to(torch.bfloat16))
    small_rank = (torch.randn(9, 48, 256, generator=generator).to(torch.bfloat16),
                  (torch.randn(64, generator=generator) * 0.25).to(torch.bfloat16),
                  torch.randn(48, 256, generator=generator).to(torch.bfloat16))
    cases = {"peaked S=9 D=1024": peaked, "small rank D=256 R=64": small_rank}
    for tokens, rank in ((8, 8192), (2, 6144)):
        cases[f"peaked S=129 N={tokens} D=8192 R={rank}"] = (
            torch.randn(129, tokens, 8192, generator=generator).to(torch.bfloat16),
            (torch.randn(rank, generator=generator) * 0.25).to(torch.bfloat16),
            torch.randn(tokens, 8192, generator=generator).to(torch.bfloat16))
    for name in ("c2", "c3"):
        cfg = dict(bench.CONFIGS[name], batch=(64,), input_device="cpu")
        cases[f"{name} inputs, 64 tokens"] = bench.make_inputs(cfg, "cpu", seed=0)
    return cases


CASES = _cases()


_EXACT = {}


def _exact(case):
    """(float64 dv, float64 dq, dv allowance, dq allowance) of a case."""
    if case not in _EXACT:
        values, query, grad_out = CASES[case]
        _, dv, dq = exact_with_grads(values, query, grad_out)
        dv_allow, dq_variance = delta_allowance(values.double(), query.double(), grad_out.double())
        _EXACT[case] = dv, dq, dv_allow, DELTA_SIGMAS * dq_variance.sqrt()
    return _EXACT[case]


@pytest.mark.parametrize("case", sorted(CASES))
def test_correct_rounding_passes_the_floor(case):
    dv, dq, _, _ = _exact(case)
    assert ulp_error(dv.to(torch.bfloat16), dv, FLOOR) <= 0.5
    assert ulp_error(dq.to(torch.bfloat16), dq, FLOOR) <= 0.5


@pytest.mark.parametrize("case", sorted(CASES))
def test_emulated_refinement_stays_within_the_allowance(case):
    values, query, grad_out = CASES[case]
    dv, dq, dv_allow, dq_allow = _exact(case)
    emulated_dv, emulated_dq = _emulated_saved_grads(values, query, grad_out)
    assert ulp_error(emulated_dv.to(torch.bfloat16), dv, FLOOR, dv_allow) <= 0.5
    assert ulp_error(emulated_dq.to(torch.bfloat16), dq, FLOOR, dq_allow) <= 0.5


@pytest.mark.parametrize("mistake", ["rms_jacobian_dropped", "rms_jacobian_1pct", "routing_1pct",
                                     "refinement_dropped"])
@pytest.mark.parametrize("case", sorted(CASES))
def test_planted_gradient_mistakes_fail_the_saved_path_bound(case, mistake):
    values, query, grad_out = CASES[case]
    dv, _, allowance, _ = _exact(case)
    if mistake == "refinement_dropped":
        wrong = _emulated_saved_grads(values, query, grad_out, refine=False)[0]
    else:
        wrong = _mutant_grads(values, query, grad_out, mistake)
    assert ulp_error(wrong.to(torch.bfloat16), dv, FLOOR, allowance) > 10.0, f"{mistake} is not caught on {case}"


@pytest.mark.parametrize("case", sorted(CASES))
def test_dropped_refinement_fails_the_query_gradient_bound(case):
    values, query, grad_out = CASES[case]
    _, dq, _, dq_allow = _exact(case)
    wrong = _emulated_saved_grads(values, query, grad_out, refine=False)[1]
    # dq sums the per-token errors with mixed signs over few tokens here, so the
    # margin is smaller than for dv (4 ulps at D = 256, thousands at D = 8192)
    assert ulp_error(wrong.to(torch.bfloat16), dq, FLOOR, dq_allow) > 2.0


def test_floor_lies_below_a_bf16_ulp_of_the_row():
    # half a BF16 ulp of the row maximum is at least 2^-9 of it
    assert FLOOR == 2.0**-16 and math.log2(FLOOR) < -9


# ------------------------------------------------- gradients summed over reads

def _read_grads(values, query, grad_out, scale, delta_from="refined", key_factor=1.0, eps=2**-23):
    """One read's float64 dv with delta from the refined BF16 output
    ("refined", the saving kernels) or exact ("exact"); the key-coordinate
    term scaled by ``key_factor`` (a planted mistake when not 1)."""
    v = values.double()
    q = query.double()
    g = grad_out.double()
    width, rank = v.shape[-1], q.numel()
    key = v[..., width - rank:]
    inv_rms = torch.rsqrt(key.square().mean(-1) + eps)
    logit = (key * inv_rms[..., None] * q).sum(-1) * scale
    weight = logit.softmax(0)
    out = (weight[..., None] * v).sum(0)
    if delta_from == "refined":
        rounded = out.float().to(torch.bfloat16).double()
        unit = bf16_ulp(rounded) / 256
        out = rounded + torch.clamp(torch.round((out - rounded) / unit), -127, 127) * unit
    dz = weight * ((v * g).sum(-1) - (g * out).sum(-1))
    dv = weight[..., None] * g
    dv[..., width - rank:] += key_factor * dz[..., None] * (
        scale * inv_rms[..., None] * q - (inv_rms * inv_rms * logit / rank)[..., None] * key)
    return dv


def _bf16_running_sum(contributions):
    """The accumulating BF16 backward: the first read writes bf16(dv), each
    later one bf16(old + dv) with the addition in FP32."""
    total = None
    for dv in contributions:
        step = dv.float() if total is None else total.float() + dv.float()
        total = step.to(torch.bfloat16)
    return total


def _shared_reads(width, rank, seed):
    generator = torch.Generator().manual_seed(seed)
    values = torch.stack([(torch.randn(64, width, generator=generator) * (0.5 + s / 4)).to(torch.bfloat16)
                          for s in range(9)])
    reads = [((torch.randn(rank, generator=generator) / math.sqrt(rank)).to(torch.bfloat16),
              torch.randn(64, width, generator=generator).to(torch.bfloat16), scale) for scale in (1.0, 0.5, 2.0)]
    return values, reads


@pytest.mark.parametrize("width,rank", [(2048, 2048), (1000, 96)])
def test_accumulated_bound_holds_and_catches_a_key_term_mistake(width, rank):
    """Three reads of nine shared sources (`SharedSources`, c4-like): the
    emulated accumulating backward stays within `helpers.accumulated_bound`
    of the exact sum over the reads, and a 1% error in one read's key term
    (the routing gradient on the key coordinates) exceeds it."""
    from helpers import accumulated_bound

    values, reads = _shared_reads(width, rank, seed=20261202 + width)
    exact = [_read_grads(values, q, g, s, "exact") for q, g, s in reads]
    allowances = [delta_allowance(values.double(), q.double(), g.double(), scale=s)[0] for q, g, s in reads]
    bound = accumulated_bound(exact, allowances, roundings=len(reads))
    total = sum(exact)
    emulated = _bf16_running_sum([_read_grads(values, q, g, s) for q, g, s in reads])
    ratio = float(((emulated.double() - total).abs() / bound).max())
    assert ratio <= 1.0, ratio
    mistaken = _bf16_running_sum([_read_grads(values, q, g, s, key_factor=1.01 if i == 1 else 1.0)
                                  for i, (q, g, s) in enumerate(reads)])
    planted = float(((mistaken.double() - total).abs() / bound).max())
    assert planted > 2.0, planted
