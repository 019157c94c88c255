"""The save/recompute policy on the GPU: reads of at most 6 sources store no
output refinement, and their backward (`attnres_bwd_recompute_kernel`) gets
delta = <dO, o> = sum_s p_s <v_s, dO> from the value rows.

Checked against the CPU oracle on every row geometry (group of 16/32/64
lanes, one or several chunks per lane, a whole workgroup per token above
D = 2048), with and without key masks, on the vectorised (aligned) and the
element-wise (padded rows) path, packed and as a source list; and against
the saved-refinement backward on the same inputs, which computes the same
gradients from the saved output instead (the reference recomputes for
S <= 3, `src/attnres/_kernels/fla_full_sources.py:146-161`; the register-resident
backward pays up to S = 6 here).
"""

from __future__ import annotations

import math

import pytest
import torch

from attnres import _ops, attnres
from helpers import SEEDS, both_oracles, check_statistics, compare_read, set_case

pytestmark = pytest.mark.gpu

# (width, rank): geometry (lanes, chunks) -- 16x1 masked, 32x1, 32x2, 32x4 masked,
# 64x4, 64x8 (run as 256x2) with and without masks, 256x4 with and without masks
WIDTHS = [(128, 40), (256, 256), (512, 512), (1000, 96), (2048, 2048), (3000, 257), (4096, 4096),
          (6144, 1024), (8192, 8192)]


def _inputs(sources, tokens, width, rank, padded, seed):
    torch.manual_seed(seed)
    pad = 7 if padded else 0
    producer = torch.randn(sources, tokens, width + pad, device="cuda", dtype=torch.bfloat16)
    producer = producer * torch.linspace(0.5, 4, sources, device="cuda", dtype=torch.bfloat16)[:, None, None]
    producer.requires_grad_()
    query = (torch.randn(rank, device="cuda", dtype=torch.bfloat16) / math.sqrt(rank)).requires_grad_()
    upstream = torch.randn(tokens, width, device="cuda", dtype=torch.bfloat16)
    return producer, query, upstream


@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("padded", [False, True], ids=["aligned", "padded"])
@pytest.mark.parametrize("width,rank", WIDTHS, ids=lambda v: str(v))
@pytest.mark.parametrize("sources", [1, 2, 3, 4, 6])
def test_recompute_backward_matches_oracle(sources, width, rank, padded, layout):
    tokens = 37
    producer, query, upstream = _inputs(sources, tokens, width, rank, padded, SEEDS[0] + width + sources)

    def make(leaves, q):
        values = leaves[0][..., :width]
        return (tuple(values.unbind(0)) if layout == "list" else values), q

    print(f"recompute S={sources} D={width} R={rank} padded={padded} layout={layout}", flush=True)
    set_case(f"recompute S={sources} D={width} R={rank} padded={padded} {layout}")
    actual = attnres(make([producer], query)[0], query)
    grads = torch.autograd.grad(actual, (producer, query), upstream)
    expected, exact = both_oracles(make, [producer], query, upstream)
    torch.cuda.synchronize()
    compare_read((actual, *grads), expected, exact, ["out", "dv", "dq"], sources=sources)
    check_statistics(make([producer.detach()], query)[0], query.detach())


@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("width,rank", [(1000, 96), (2048, 2048), (4096, 1024), (8192, 8192)],
                         ids=lambda v: str(v))
@pytest.mark.parametrize("sources", [2, 3, 5, 6])
def test_recompute_agrees_with_the_saved_refinement_path(sources, width, rank, layout):
    """Same inputs through both backward kernels: the forward output is the
    same bits, dv agrees to BF16 rounding and dq to FP32 rounding of delta."""
    tokens = 513
    producer, query, upstream = _inputs(sources, tokens, width, rank, False, SEEDS[1] + width)
    values = producer.detach()
    q = query.detach()
    print(f"recompute vs saved S={sources} D={width} R={rank} layout={layout}", flush=True)
    results = {}
    for save in (False, True):
        if layout == "packed":
            out, refine, logit, inv_rms, stats = _ops.packed_forward_impl(values, q, 2**-23, 1.0, save)
            dv, dq = _ops.packed_backward(values, q, out, refine, upstream, logit, inv_rms, stats, 1.0)
        else:
            listed = list(values.unbind(0))
            out, refine, logit, inv_rms, stats = _ops.sources_forward_impl(listed, q, 2**-23, 1.0, save)
            grads = _ops.sources_backward(listed, q, out, refine, upstream, logit, inv_rms, stats, 1.0)
            dv, dq = torch.stack(grads[:-1]), grads[-1]
        assert refine.shape[0] == (tokens if save else 0)
        results[save] = (out, dv, dq)
    torch.cuda.synchronize()
    (out_r, dv_r, dq_r), (out_s, dv_s, dq_s) = results[False], results[True]
    assert torch.equal(out_r, out_s)
    scale_dv = float(dv_s.float().abs().max())
    torch.testing.assert_close(dv_r.float(), dv_s.float(), rtol=2.0**-7, atol=2.0**-9 * scale_dv)
    rel = float((dq_r.float() - dq_s.float()).norm() / dq_s.float().norm())
    assert rel < 2e-3, rel


def test_recompute_special_cases_are_exact():
    """S = 1: dv == dO, dq == 0; two identical sources: dv == dO / 2, dq == 0
    (delta = sum_s p_s dw_s equals dw exactly when p is 1 or 1/2)."""
    torch.manual_seed(SEEDS[2])
    upstream = torch.randn(19, 2048, device="cuda", dtype=torch.bfloat16)
    one = torch.randn(1, 19, 2048, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    query = torch.randn(2048, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    out = attnres(one, query)
    dv, dq = torch.autograd.grad(out, (one, query), upstream)
    assert torch.equal(out, one[0]) and torch.equal(dv[0], upstream)
    assert torch.count_nonzero(dq) == 0
    twin = one.detach().expand(2, -1, -1).contiguous().requires_grad_()
    out = attnres(twin, query, scale=3.0)
    dv, dq = torch.autograd.grad(out, (twin, query), upstream)
    assert torch.equal(out, twin[0])
    assert torch.equal(dv, (upstream.float() / 2).to(torch.bfloat16).expand(2, -1, -1))
    assert torch.count_nonzero(dq) == 0


# The key-resident backward (`attnres_bwd_keyres_kernel`): reads of 7..16
# sources whose rows are 2048 or 4096 elements wide and whose key is their last
# 512 or 1024 elements save no refinement either; the backward keeps the key
# chunks of a token's rows in registers and takes delta from the value rows.
KEYRES_SHAPES = [(2048, 512), (2048, 1024), (4096, 512), (4096, 1024)]


KEYRES_CASES = [(s, w, r) for s in (7, 8, 13, 16) for w, r in KEYRES_SHAPES] + \
    [(s, 2048, 2048) for s in (7, 9, 12)]  # the whole 2048-wide row as key, up to 12 sources


@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("padded", [False, True], ids=["aligned", "padded"])
@pytest.mark.parametrize("sources,width,rank", KEYRES_CASES, ids=lambda v: str(v))
def test_key_resident_backward_matches_oracle(sources, width, rank, padded, layout):
    """Against the oracle at the full bars with no delta allowance: delta is
    an FP32 sum over the value rows, not the refined BF16 output.  Padded rows
    (7 elements of padding) take the element-wise path."""
    assert not _ops.saves_refinement(sources, width, rank)
    tokens = 37
    producer, query, upstream = _inputs(sources, tokens, width, rank, padded, SEEDS[0] + 3 * width + sources)

    def make(leaves, q):
        values = leaves[0][..., :width]
        return (tuple(values.unbind(0)) if layout == "list" else values), q

    print(f"key-resident S={sources} D={width} R={rank} padded={padded} layout={layout}", flush=True)
    set_case(f"key-resident S={sources} D={width} R={rank} padded={padded} {layout}")
    actual = attnres(make([producer], query)[0], query)
    grads = torch.autograd.grad(actual, (producer, query), upstream)
    expected, exact = both_oracles(make, [producer], query, upstream)
    torch.cuda.synchronize()
    compare_read((actual, *grads), expected, exact, ["out", "dv", "dq"], sources=sources)
    check_statistics(make([producer.detach()], query)[0], query.detach())


def _random_keyres_cases(count: int, seed: int = 20261202) -> list[tuple]:
    """Reads the key-resident backward takes, drawn at random: every key
    shape, any source count it accepts, token counts from 1 to 1500 (odd ones,
    and fewer than a grid's token groups, leave groups idle or with one token
    and put padding items at every group's end), aligned or padded rows,
    packed or list."""
    import random

    rng = random.Random(seed)
    shapes = KEYRES_SHAPES + [(2048, 2048)]
    cases = []
    for _ in range(count):
        width, rank = rng.choice(shapes)
        top = _ops.KEYRES_FULL_MAX_SOURCES if width == rank else _ops.KEYRES_MAX_SOURCES
        sources = rng.randint(_ops.RECOMPUTE_MAX_SOURCES + 1, top)
        tokens = rng.choice([1, 2, 3, rng.randint(4, 200), rng.randint(200, 1500) | 1])
        cases.append((sources, tokens, width, rank, rng.random() < 0.3, rng.choice(["packed", "list"])))
    return cases


@pytest.mark.parametrize("sources,tokens,width,rank,padded,layout", _random_keyres_cases(24), ids=lambda v: str(v))
def test_key_resident_random_shapes_match_oracle(sources, tokens, width, rank, padded, layout):
    """Random key-resident reads against the oracle at the full bars (no delta
    allowance)."""
    assert not _ops.saves_refinement(sources, width, rank)
    producer, query, upstream = _inputs(sources, tokens, width, rank, padded, SEEDS[2] + 17 + sources * tokens + width)

    def make(leaves, q):
        values = leaves[0][..., :width]
        return (tuple(values.unbind(0)) if layout == "list" else values), q

    print(f"key-resident random S={sources} N={tokens} D={width} R={rank} padded={padded} {layout}", flush=True)
    set_case(f"key-resident random S={sources} N={tokens} D={width} R={rank} padded={padded} {layout}")
    actual = attnres(make([producer], query)[0], query)
    grads = torch.autograd.grad(actual, (producer, query), upstream)
    expected, exact = both_oracles(make, [producer], query, upstream)
    torch.cuda.synchronize()
    compare_read((actual, *grads), expected, exact, ["out", "dv", "dq"], sources=sources)


@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("sources,tokens,width,rank",
                         [(s, n, w, r) for s, n in ((7, 5003), (16, 2053), (9, 1)) for w, r in KEYRES_SHAPES] +
                         [(7, 5003, 2048, 2048), (12, 2053, 2048, 2048), (9, 1, 2048, 2048)], ids=lambda v: str(v))
def test_key_resident_agrees_with_the_saved_refinement_path(sources, tokens, width, rank, layout):
    """Same inputs through the key-resident and the saved-refinement backward
    (streaming kernel, delta from the saved output), on grids where a group
    takes several tokens in turn: the forward output is the same bits, dv
    agrees to BF16 rounding and dq to the refinement's delta error."""
    producer, query, upstream = _inputs(sources, tokens, width, rank, False, SEEDS[1] + width + tokens)
    values = producer.detach()
    q = query.detach()
    print(f"key-resident vs saved S={sources} N={tokens} D={width} R={rank} layout={layout}", flush=True)
    results = {}
    for save in (False, True):
        if layout == "packed":
            out, refine, logit, inv_rms, stats = _ops.packed_forward_impl(values, q, 2**-23, 1.0, save)
            dv, dq = _ops.packed_backward(values, q, out, refine, upstream, logit, inv_rms, stats, 1.0)
        else:
            listed = list(values.unbind(0))
            out, refine, logit, inv_rms, stats = _ops.sources_forward_impl(listed, q, 2**-23, 1.0, save)
            grads = _ops.sources_backward(listed, q, out, refine, upstream, logit, inv_rms, stats, 1.0)
            dv, dq = torch.stack(grads[:-1]), grads[-1]
        assert refine.shape[0] == (tokens if save else 0)
        results[save] = (out, dv, dq)
    torch.cuda.synchronize()
    (out_k, dv_k, dq_k), (out_s, dv_s, dq_s) = results[False], results[True]
    assert torch.equal(out_k, out_s)
    # the non-key coordinates are p dO in both kernels: the same bits (up to the sign of zero)
    key0 = width - rank
    assert torch.equal(dv_k[..., :key0].float(), dv_s[..., :key0].float())
    scale_dv = float(dv_s.float().abs().max())
    torch.testing.assert_close(dv_k.float(), dv_s.float(), rtol=2.0**-7, atol=2.0**-9 * scale_dv)
    rel = float((dq_k.float() - dq_s.float()).norm() / dq_s.float().norm())
    assert rel < 2e-3, rel


@pytest.mark.parametrize("sources,width,rank", [(16, 4096, 1024), (17, 4096, 1024), (12, 2048, 2048),
                                                (13, 2048, 2048)], ids=lambda v: str(v))
def test_key_resident_policy_boundary(sources, width, rank):
    """16 sources of (4096, 1024) and 12 of (2048, 2048) take the key-resident
    backward and save no refinement; 17 and 13 save it (the streaming and the
    token-block backward).  All match the oracle (the saving reads with the
    saved path's delta allowance)."""
    tokens = 67
    producer, query, upstream = _inputs(sources, tokens, width, rank, False, SEEDS[2] + sources)
    values = producer.detach()
    out, refine, *_ = _ops.packed_forward_impl(values, query.detach(), 2**-23, 1.0,
                                               _ops.saves_refinement(sources, width, rank))
    assert refine.shape[0] == (0 if sources in (12, 16) else tokens)

    def make(leaves, q):
        return leaves[0], q

    set_case(f"key-resident boundary S={sources}")
    actual = attnres(producer, query)
    grads = torch.autograd.grad(actual, (producer, query), upstream)
    expected, exact = both_oracles(make, [producer], query, upstream)
    compare_read((actual, *grads), expected, exact, ["out", "dv", "dq"], sources=sources)
