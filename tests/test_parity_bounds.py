"""The GPU parity bounds (tests/helpers.py) are strong enough to catch real mistakes.

The kernels' value gradients are held to one BF16 ulp of the float64 oracle,
up to a floor of 2^-16 (recompute path) or 2^-13 (saved-output path) times
the row's largest magnitude.  Here, on the CPU, plausible mistakes are
planted in copies of the oracle's arithmetic (`oracle.oracle._mix` in
float64) and their BF16-rounded gradients must fail the looser 2^-13 bound,
while the correctly rounded float64 gradient passes it at half an ulp:

* the RMS-norm Jacobian dropped (``inv_rms`` treated as a constant);
* the RMS-norm Jacobian scaled by 1.01;
* the whole routing gradient (through the logit) scaled by 1.01.

Inputs: peaked softmax (query x 0.25, as in the envelope tests), the
BASELINE distribution of c2 (R = D) and of c3 (sliced, R = D/4), and a
small rank.
"""

from __future__ import annotations

import math

import pytest
import torch

import bench
from helpers import FLOOR, SAVED_DV_FLOOR, ulp_error
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


def _cases():
    generator = torch.Generator().manual_seed(20260827)
    peaked = (torch.randn(9, 48, 1024, generator=generator).to(torch.bfloat16),
              (torch.randn(1024, generator=generator) * 0.25).to(torch.bfloat16),
              torch.randn(48, 1024, generator=generator).to(torch.bfloat16))
    small_rank = (torch.randn(9, 48, 256, generator=generator).to(torch.bfloat16),
                  (torch.randn(64, generator=generator) * 0.25).to(torch.bfloat16),
                  torch.randn(48, 256, generator=generator).to(torch.bfloat16))
    cases = {"peaked S=9 D=1024": peaked, "small rank D=256 R=64": small_rank}
    for name in ("c2", "c3"):
        cfg = dict(bench.CONFIGS[name], batch=(64,), input_device="cpu")
        cases[f"{name} inputs, 64 tokens"] = bench.make_inputs(cfg, "cpu", seed=0)
    return cases


CASES = _cases()


@pytest.mark.parametrize("case", sorted(CASES))
def test_correct_rounding_passes_both_floors(case):
    values, query, grad_out = CASES[case]
    _, dv, _ = exact_with_grads(values, query, grad_out)
    rounded = dv.to(torch.bfloat16)
    assert ulp_error(rounded, dv, FLOOR) <= 0.5
    assert ulp_error(rounded, dv, SAVED_DV_FLOOR) <= 0.5


@pytest.mark.parametrize("mistake", ["rms_jacobian_dropped", "rms_jacobian_1pct", "routing_1pct"])
@pytest.mark.parametrize("case", sorted(CASES))
def test_planted_gradient_mistakes_fail_the_saved_path_bound(case, mistake):
    values, query, grad_out = CASES[case]
    _, dv, _ = exact_with_grads(values, query, grad_out)
    wrong = _mutant_grads(values, query, grad_out, mistake).to(torch.bfloat16)
    assert ulp_error(wrong, dv, SAVED_DV_FLOOR) > 10.0, f"{mistake} is not caught on {case}"


def test_floors_are_powers_of_two_below_a_bf16_ulp_of_the_row():
    # both floors lie well below half a BF16 ulp of the row maximum (2^-9)
    assert FLOOR == 2.0**-16 and SAVED_DV_FLOOR == 2.0**-13
    assert math.log2(SAVED_DV_FLOOR) < -9
