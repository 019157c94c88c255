"""The benchmark configurations at full size, checked through properties that
do not depend on the size (the CPU oracle cannot run them whole in a test).

* Tokens are independent: a sample of token rows read on their own, through
  the same kernels, gives bit-identical output rows and dv rows.
* The sample against the CPU oracle, at the BF16 gate.
* dq is a sum over tokens: the dq of the whole read equals the sum of the dq
  of four token chunks, to BF16 rounding.
* The output is a convex combination of the sources: every element lies
  between the sources' minimum and maximum, up to the output's BF16 rounding.

Shapes: c2 packed [25, 16384, 2048] R = 2048, c3 packed [16, 16384, 4096]
R = 1024 (key masks), c4 a list of 9 separately allocated [32768, 2048].
"""

from __future__ import annotations

import math

import pytest
import torch

from attnres import attnres
from helpers import compare, oracle_grads

pytestmark = pytest.mark.gpu

CONFIGS = {"c2": (25, 16384, 2048, 2048, "packed"), "c3": (16, 16384, 4096, 1024, "packed"),
           "c4": (9, 32768, 2048, 2048, "list")}


def _read(values, query, layout):
    return attnres(tuple(values.unbind(0)) if layout == "list" else values, query)


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_full_size_read_properties(name):
    sources, tokens, width, rank, layout = CONFIGS[name]
    print(f"full size {name}: S={sources} N={tokens} D={width} R={rank} {layout}", flush=True)
    generator = torch.Generator(device="cuda").manual_seed(17)
    scales = torch.rand(sources, 1, 1, generator=generator, device="cuda") * 3.5 + 0.5
    values = torch.empty(sources, tokens, width, device="cuda", dtype=torch.bfloat16)
    for s in range(sources):  # per source keeps the FP32 temporary small
        values[s] = (torch.randn(tokens, width, generator=generator, device="cuda") * scales[s]).to(torch.bfloat16)
    values.requires_grad_()
    query = (torch.randn(rank, generator=generator, device="cuda") / math.sqrt(rank)).to(torch.bfloat16)
    query.requires_grad_()
    upstream = torch.randn(tokens, width, generator=generator, device="cuda").to(torch.bfloat16)

    out = _read(values, query, layout)
    grad_values, grad_query = torch.autograd.grad(out, (values, query), upstream)

    # tokens are independent: a sample read on its own gives the same rows
    sample = torch.randperm(tokens, generator=generator, device="cuda")[:96].sort().values
    sub_values = values.detach()[:, sample].contiguous().requires_grad_()
    sub_out = _read(sub_values, query, layout)
    sub_grad_values, _ = torch.autograd.grad(sub_out, (sub_values, query), upstream[sample])
    assert torch.equal(sub_out, out[sample])
    assert torch.equal(sub_grad_values, grad_values[:, sample])

    # the sample against the oracle
    def make(leaves, q):
        return (tuple(leaves[0].unbind(0)) if layout == "list" else leaves[0]), q

    expected, (expected_values, _) = oracle_grads(make, [sub_values], query, upstream[sample])
    compare(sub_out, expected)
    compare(sub_grad_values, expected_values)

    # dq is a sum over tokens: four chunks add up to the whole read's dq
    chunk_sum = torch.zeros(rank, device="cuda")
    for chunk in torch.arange(tokens, device="cuda").chunk(4):
        part = values.detach()[:, chunk].contiguous()
        part_out = _read(part, query, layout)
        chunk_sum += torch.autograd.grad(part_out, query, upstream[chunk])[0].float()
    torch.testing.assert_close(chunk_sum, grad_query.float(), rtol=2.0**-6,
                               atol=2.0**-6 * float(grad_query.float().abs().max()))

    # convexity, up to the output's rounding (half a BF16 ulp of the bound)
    low = values.detach().amin(0).float()
    high = values.detach().amax(0).float()
    slack = torch.maximum(low.abs(), high.abs()) * 2.0**-8
    result = out.float()
    assert bool(((result >= low - slack) & (result <= high + slack)).all())
