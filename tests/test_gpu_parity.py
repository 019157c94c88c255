"""HIP kernels vs the CPU oracle: outputs and first-order gradients.

Shapes and input patterns follow the reference's GPU tests:
envelope shapes (`tests/test_full_kernel.py:118-148`), protocol smoke shapes
(`validation/protocol.json:16-59`), strided producers and transposed
upstream gradients (`validation/gpu_checks.py:28-44`), container forms with
per-source strides and a duplicated source (`tests/test_api.py:112-142`),
exact known-answer cases (`validation/softmax_checks.py:9-30`,
`tests/test_routing_checks.py`), bitwise replay
(`tests/test_bf16_packed_kernels.py:90-94`) and >2^31 offsets
(`tests/test_offsets.py`).  Bars: the reference's BF16 gate rtol=atol=0.05
against the BF16 oracle, one BF16 ulp against the float64 oracle (out, dv,
dq), and the saved statistics (logit, 1/rms, max, 1/sum) within 1e-5
relative of the oracle's (tests/helpers.py).
"""

from __future__ import annotations

import math

import pytest
import torch

from attnres import attnres
from helpers import SEEDS, both_oracles, check_statistics, compare, compare_read, oracle_grads, set_case

pytestmark = pytest.mark.gpu

ENVELOPE = [
    (1, 1, 1, 1), (3, 5, 17, 5), (9, 257, 768, 64), (9, 17, 1024, 512),
    (9, 17, 1024, 1024), (5, 7, 3000, 257), (9, 8, 3072, 3072), (5, 3, 4096, 32),
    (129, 1, 8192, 8192), (2, 5, 17, 5), (4, 5, 63, 33), (3, 7, 64, 33),
    (9, 17, 1024, 768), (129, 1, 8192, 6144),
]
SMOKE = [
    (1, 2, 128, 16), (9, 65, 768, 64), (33, 128, 1536, 128), (97, 16, 4096, 64),
    (129, 8, 7168, 128), (129, 8, 8192, 8192), (9, 32, 3000, 127),
]


def _strided_case(shape, layout, seed):
    """Producer with 7 padding columns, query[::2], transposed upstream."""
    torch.manual_seed(seed)
    s, n, d, r = shape
    producer = torch.randn(s, n, d + 7, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    query = (torch.randn(2 * r, device="cuda", dtype=torch.bfloat16) * 0.25).requires_grad_()
    upstream = torch.randn(d, n, device="cuda", dtype=torch.bfloat16).t()

    def make(leaves, q):
        values = leaves[0][..., :d]
        return (tuple(values.unbind(0)) if layout == "list" else values), q[::2]

    values, q = make([producer], query)
    print(f"case shape={shape} layout={layout} seed={seed}", flush=True)
    set_case(f"strided {shape} {layout}")
    actual = attnres(values, q)
    grads = torch.autograd.grad(actual, (producer, query), upstream)
    expected, exact = both_oracles(make, [producer], query, upstream)
    torch.cuda.synchronize()
    metrics = compare_read((actual, *grads), expected, exact, ["out", "dv", "dq"], sources=s)
    check_statistics(values, q.detach())
    return metrics


@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("shape", ENVELOPE, ids=lambda s: "x".join(map(str, s)))
def test_envelope_matches_oracle(shape, layout):
    _strided_case(shape, layout, SEEDS[0])


@pytest.mark.parametrize("shape", SMOKE, ids=lambda s: "x".join(map(str, s)))
def test_protocol_smoke_shapes_packed(shape):
    _strided_case(shape, "packed", SEEDS[1])


@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("width,rank", [(2048, 2048), (4096, 1024), (1024, 256), (2048, 512)])
def test_aligned_fast_path_matches_oracle(width, rank, layout):
    """Contiguous, 16-byte-aligned rows: the vectorised path of the kernels."""
    torch.manual_seed(SEEDS[2])
    s, n = 7, 96
    values = torch.randn(s, n, width, device="cuda", dtype=torch.bfloat16)
    values = (values * torch.linspace(0.5, 4, s, device="cuda", dtype=torch.bfloat16)[:, None, None])
    values.requires_grad_()
    query = (torch.randn(rank, device="cuda", dtype=torch.bfloat16) / math.sqrt(rank)).requires_grad_()
    upstream = torch.randn(n, width, device="cuda", dtype=torch.bfloat16)

    def make(leaves, q):
        return (tuple(leaves[0].unbind(0)) if layout == "list" else leaves[0]), q

    set_case(f"aligned D={width} R={rank} {layout}")
    actual = attnres(make([values], query)[0], query)
    grads = torch.autograd.grad(actual, (values, query), upstream)
    expected, exact = both_oracles(make, [values], query, upstream)
    compare_read((actual, *grads), expected, exact, ["out", "dv", "dq"], sources=s)
    check_statistics(make([values.detach()], query)[0], query.detach())


@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("sources,tokens", [(5, 1), (6, 3), (7, 4097), (9, 1031), (12, 2049)],
                         ids=lambda v: str(v))
def test_token_block_forward_matches_oracle(sources, tokens, layout):
    """Aligned, unmasked rows of 2048 elements (R = D) of 5 to 12 sources take
    the token-block forward, two tokens per group: a single token, odd token
    counts (the last block repeats a token and stores nothing for it), reads
    with and without the saved refinement; outputs, gradients and the saved
    statistics against the oracle."""
    torch.manual_seed(SEEDS[2] + sources * tokens)
    width = rank = 2048
    values = torch.randn(sources, tokens, width, device="cuda", dtype=torch.bfloat16)
    values = (values * torch.linspace(0.5, 4, sources, device="cuda", dtype=torch.bfloat16)[:, None, None])
    values.requires_grad_()
    query = (torch.randn(rank, device="cuda", dtype=torch.bfloat16) / math.sqrt(rank)).requires_grad_()
    upstream = torch.randn(tokens, width, device="cuda", dtype=torch.bfloat16)

    def make(leaves, q):
        return (tuple(leaves[0].unbind(0)) if layout == "list" else leaves[0]), q

    print(f"token-block forward S={sources} N={tokens} layout={layout}", flush=True)
    set_case(f"token-block forward S={sources} N={tokens} {layout}")
    actual = attnres(make([values], query)[0], query)
    grads = torch.autograd.grad(actual, (values, query), upstream)
    expected, exact = both_oracles(make, [values], query, upstream)
    compare_read((actual, *grads), expected, exact, ["out", "dv", "dq"], sources=sources)
    check_statistics(make([values.detach()], query)[0], query.detach())


@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("sources,tokens,width,rank",
                         [(13, 1, 4096, 4096), (13, 3, 3072, 3072), (16, 1027, 4096, 1024), (17, 2049, 2560, 640),
                          (25, 130, 4000, 4000), (48, 517, 3072, 768),
                          (5, 1, 1536, 1536), (6, 3, 1280, 320), (9, 2051, 1536, 384), (48, 130, 1280, 1280),
                          (5, 1, 5120, 5120), (6, 3, 6144, 1536), (25, 131, 8192, 8192), (48, 17, 7168, 1792),
                          (5, 1, 512, 512), (6, 3, 384, 96), (25, 1027, 448, 448), (9, 2049, 768, 768),
                          (13, 3, 520, 520), (48, 130, 640, 160), (5, 3, 256, 256), (25, 1027, 200, 40)],
                         ids=lambda v: str(v))
def test_two_token_block_forward_matches_oracle(sources, tokens, width, rank, layout):
    """The token-block forward with two tokens per group: 16-byte aligned rows
    of 2049 to 4096 elements (64 lanes of 8 chunks) of more than 12 sources,
    with and without key masks, full and partial rows (chunks past D idle);
    aligned rows of 1025 to 2047 elements (64 lanes of 4 chunks, some idle)
    and of 4097 to 8192 elements (a workgroup of 256 lanes per token group) of
    5 sources and more; 32-lane groups, two per wavefront, at 129 to 512
    elements (two rows per token in flight) from 5 sources and at 513 to 1023
    from 9; including the few-source reads that save no refinement: a single token,
    odd token counts (the last block repeats a token and stores nothing for
    it); outputs, gradients and the saved statistics against the oracle."""
    torch.manual_seed(SEEDS[2] + sources * tokens + width)
    values = torch.randn(sources, tokens, width, device="cuda", dtype=torch.bfloat16)
    values = (values * torch.linspace(0.5, 4, sources, device="cuda", dtype=torch.bfloat16)[:, None, None])
    values.requires_grad_()
    query = (torch.randn(rank, device="cuda", dtype=torch.bfloat16) / math.sqrt(rank)).requires_grad_()
    upstream = torch.randn(tokens, width, device="cuda", dtype=torch.bfloat16)

    def make(leaves, q):
        return (tuple(leaves[0].unbind(0)) if layout == "list" else leaves[0]), q

    print(f"two-token block forward S={sources} N={tokens} D={width} R={rank} layout={layout}", flush=True)
    set_case(f"two-token block forward S={sources} N={tokens} D={width} R={rank} {layout}")
    actual = attnres(make([values], query)[0], query)
    grads = torch.autograd.grad(actual, (values, query), upstream)
    expected, exact = both_oracles(make, [values], query, upstream)
    compare_read((actual, *grads), expected, exact, ["out", "dv", "dq"], sources=sources)
    check_statistics(make([values.detach()], query)[0], query.detach())


@pytest.mark.parametrize("sources,width,rank", [(9, 2048, 2048), (13, 2048, 2048), (25, 2048, 2048),
                                                (13, 3072, 768), (5, 5120, 5120), (9, 384, 384), (9, 1536, 1536)],
                         ids=["forward_blocks_2", "backward_blocks", "both_blocks_4", "forward_64x8",
                              "forward_256", "forward_32x2", "forward_64x4_short"])
def test_token_blocks_with_padded_strides(sources, width, rank):
    """The token-block kernels on packed values viewed out of a wider buffer:
    rows D + 64 elements apart (still 16-byte aligned) and sources a further
    64 rows apart, so neither stride is N*D."""
    torch.manual_seed(SEEDS[0] + sources + width)
    tokens = 1027
    big = torch.randn(sources, tokens + 64, width + 64, device="cuda", dtype=torch.bfloat16)
    values = big[:, :tokens, :width]
    values.mul_(torch.linspace(0.5, 4, sources, device="cuda", dtype=torch.bfloat16)[:, None, None])
    values.requires_grad_()
    assert values.stride() == ((tokens + 64) * (width + 64), width + 64, 1)
    query = (torch.randn(rank, device="cuda", dtype=torch.bfloat16) / math.sqrt(rank)).requires_grad_()
    upstream = torch.randn(tokens, width, device="cuda", dtype=torch.bfloat16)

    def make(leaves, q):
        return leaves[0], q

    print(f"token blocks, padded strides S={sources} D={width} R={rank}", flush=True)
    set_case(f"token blocks padded strides S={sources} D={width} R={rank}")
    actual = attnres(values, query)
    grads = torch.autograd.grad(actual, (values, query), upstream)
    expected, exact = both_oracles(make, [values], query, upstream)
    compare_read((actual, *grads), expected, exact, ["out", "dv", "dq"], sources=sources)


@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("sources,tokens", [(13, 1), (13, 3), (14, 4097), (16, 1030), (25, 2049), (49, 130), (129, 37)],
                         ids=lambda v: str(v))
def test_token_block_backward_matches_oracle(sources, tokens, layout):
    """Aligned, unmasked rows of 2048 elements (R = D) of at least 13 sources
    take the token-block backward, four tokens per group: a single token, token counts that are not
    a multiple of four (the last block repeats a token and stores nothing for
    it), grids of few and of many blocks, up to the envelope's 129 sources."""
    torch.manual_seed(SEEDS[1] + sources * tokens)
    width = rank = 2048
    values = torch.randn(sources, tokens, width, device="cuda", dtype=torch.bfloat16)
    values = (values * torch.linspace(0.5, 4, sources, device="cuda", dtype=torch.bfloat16)[:, None, None])
    values.requires_grad_()
    query = (torch.randn(rank, device="cuda", dtype=torch.bfloat16) / math.sqrt(rank)).requires_grad_()
    upstream = torch.randn(tokens, width, device="cuda", dtype=torch.bfloat16)

    def make(leaves, q):
        return (tuple(leaves[0].unbind(0)) if layout == "list" else leaves[0]), q

    print(f"token blocks S={sources} N={tokens} layout={layout}", flush=True)
    set_case(f"token blocks S={sources} N={tokens} {layout}")
    actual = attnres(make([values], query)[0], query)
    grads = torch.autograd.grad(actual, (values, query), upstream)
    expected, exact = both_oracles(make, [values], query, upstream)
    compare_read((actual, *grads), expected, exact, ["out", "dv", "dq"], sources=sources)


@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("tokens,width,rank", [(2048, 1024, 1024), (4096, 1024, 1024), (4096, 1024, 256),
                                               (2048, 1024, 256), (3000, 2048, 512), (64, 8192, 8192)],
                         ids=lambda v: str(v))
def test_backward_ring_depths_match_oracle(tokens, width, rank, layout):
    """The aligned 4-chunk backward keeps two rows per group at D = 1025..2048
    and above 4096 always, and at D = 513..1024 only on small grids (at most 4
    wavefronts per CU: N <= 2048 on 256 CUs), one row otherwise: both depths,
    with and without key masks."""
    torch.manual_seed(SEEDS[0] + tokens + rank)
    s = 5
    values = torch.randn(s, tokens, width, device="cuda", dtype=torch.bfloat16)
    values = (values * torch.linspace(0.5, 4, s, device="cuda", dtype=torch.bfloat16)[:, None, None])
    values.requires_grad_()
    query = (torch.randn(rank, device="cuda", dtype=torch.bfloat16) / math.sqrt(rank)).requires_grad_()
    upstream = torch.randn(tokens, width, device="cuda", dtype=torch.bfloat16)

    def make(leaves, q):
        return (tuple(leaves[0].unbind(0)) if layout == "list" else leaves[0]), q

    print(f"ring depths N={tokens} D={width} R={rank} layout={layout}", flush=True)
    set_case(f"ring N={tokens} D={width} R={rank} {layout}")
    actual = attnres(make([values], query)[0], query)
    grads = torch.autograd.grad(actual, (values, query), upstream)
    expected, exact = both_oracles(make, [values], query, upstream)
    compare_read((actual, *grads), expected, exact, ["out", "dv", "dq"], sources=s)


@pytest.mark.parametrize("container", ["list", "tuple", "packed_values"])
def test_source_containers_with_per_source_strides(container):
    """Differently-strided producers, a strided query and a repeated source
    (reference tests/test_api.py:112-142)."""
    torch.manual_seed(29)
    width, rank = 13, 5
    leaves = [
        torch.randn(2, 3, 2 * width, device="cuda", dtype=torch.bfloat16, requires_grad=True),
        torch.randn(3, 2, width, device="cuda", dtype=torch.bfloat16, requires_grad=True),
        torch.randn(2, 3, width + 7, device="cuda", dtype=torch.bfloat16, requires_grad=True),
    ]
    query = (torch.randn(2 * rank, device="cuda", dtype=torch.bfloat16) * 0.25).requires_grad_()
    upstream = torch.randn(width, 3, 2, device="cuda", dtype=torch.bfloat16).permute(2, 1, 0)

    def make(ls, q):
        values = [ls[0][..., ::2], ls[1].transpose(0, 1), ls[2][..., :width]]
        values.append(values[0])
        if container == "tuple":
            values = tuple(values)
        elif container == "packed_values":
            values = torch.stack(values)
        return values, q[::2]

    set_case(f"containers {container}")
    actual = attnres(*make(leaves, query))
    grads = torch.autograd.grad(actual, (*leaves, query), upstream)
    expected, exact = both_oracles(make, leaves, query, upstream)
    # the duplicated source's gradient is autograd's BF16 sum of two reads' rows
    compare_read((actual, *grads[1:]), (expected[0], *expected[2:]), (exact[0], *exact[2:]),
                 ["out", "dv1", "dv2", "dq"], sources=4)
    compare(grads[0], expected[1], name="dv0+dv3")


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("sources,rows", [(2, 2), (4, 2), (4, 1024)])
@pytest.mark.parametrize("scale", [2**24, -(2**24)])
def test_equal_large_logits_are_exact(sources, rows, packed, scale):
    """Identical sources at |scale| = 2^24: out == v, dv == g/S, dq == 0 exactly
    (reference validation/softmax_checks.py:9-30)."""
    width, rank = 256, 16
    values = torch.ones(sources, rows, width, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    query = torch.ones(rank, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    upstream = torch.ones(rows, width, device="cuda", dtype=torch.bfloat16)
    inputs = values if packed else tuple(values.unbind())
    for factor in (1.0, -2.0, 4.0):
        output = attnres(inputs, query, eps=2**-23, scale=scale)
        dv, dq = torch.autograd.grad(output, (values, query), upstream * factor)
        torch.testing.assert_close(output, values[0], rtol=0, atol=0)
        torch.testing.assert_close(dv, (upstream * factor).expand_as(values) / sources, rtol=0, atol=0)
        torch.testing.assert_close(dq, torch.zeros_like(query), rtol=0, atol=0)


@pytest.mark.parametrize("packed", [False, True])
def test_zero_scale_is_uniform_average_exactly(packed):
    """scale=0: p = 1/S, dv == g/S exactly, dq == 0 exactly
    (reference tests/test_routing_checks.py:39-47)."""
    torch.manual_seed(SEEDS[0])
    values = torch.randn(4, 2, 32, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    query = torch.randn(16, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    upstream = torch.randn(2, 32, device="cuda", dtype=torch.bfloat16)
    inputs = values if packed else tuple(values.unbind())
    output = attnres(inputs, query, eps=2**-10, scale=0.0)
    dv, dq = torch.autograd.grad(output, (values, query), upstream)
    torch.testing.assert_close(dv, upstream.expand_as(values) / 4, rtol=0, atol=0)
    torch.testing.assert_close(dq, torch.zeros_like(query), rtol=0, atol=0)
    expected = (values.detach().float().mean(0)).to(torch.bfloat16)
    compare(output, expected)


def test_zero_keys_have_closed_form_gradients():
    """All-zero keys: p = 1/S, dk = scale*dz*q/sqrt(eps), dq == 0 exactly
    (reference tests/test_routing_checks.py:10-24)."""
    torch.manual_seed(20260906)
    sources, rows, width, rank = 4, 3, 32, 16
    eps, scale = 2**-10, -0.75
    values = torch.randn(sources, rows, width, device="cuda", dtype=torch.bfloat16)
    values[..., :-rank] += torch.arange(sources, device="cuda", dtype=torch.bfloat16)[:, None, None]
    values[..., -rank:] = 0
    values.requires_grad_()
    query = (torch.randn(rank, device="cuda", dtype=torch.bfloat16) * 0.05).requires_grad_()
    upstream = torch.randn(rows, width, device="cuda", dtype=torch.bfloat16)
    output = attnres(values, query, eps=eps, scale=scale)
    dv, dq = torch.autograd.grad(output, (values, query), upstream)
    v, g, q = values.detach().float(), upstream.float(), query.detach().float()
    dz = ((v - v.mean(0)) * g).sum(-1) / sources
    dk = scale * dz[..., None] * q / math.sqrt(eps)
    assert torch.count_nonzero(dk) == dk.numel()
    compare(dv[..., -rank:], (g[None, ..., -rank:] / sources + dk).to(torch.bfloat16))
    torch.testing.assert_close(dq, torch.zeros_like(query), rtol=0, atol=0)


def test_single_source_is_identity():
    """S = 1: out == v, dv == g, dq == 0 exactly."""
    torch.manual_seed(SEEDS[1])
    values = torch.randn(1, 33, 640, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    query = torch.randn(640, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    upstream = torch.randn(33, 640, device="cuda", dtype=torch.bfloat16)
    output = attnres(values, query)
    dv, dq = torch.autograd.grad(output, (values, query), upstream)
    torch.testing.assert_close(output, values[0], rtol=0, atol=0)
    torch.testing.assert_close(dv[0], upstream, rtol=0, atol=0)
    torch.testing.assert_close(dq, torch.zeros_like(query), rtol=0, atol=0)


@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("width,rank", [(1024, 64), (1024, 384), (2048, 2048)])
def test_bitwise_replay_is_deterministic(width, rank, layout):
    """Same inputs twice -> identical bits for out, dv and dq
    (reference tests/test_bf16_packed_kernels.py:90-94)."""
    torch.manual_seed(20260905 + rank)
    values = torch.randn(5, 4099, width, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    query = torch.randn(rank, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    upstream = torch.randn(4099, width, device="cuda", dtype=torch.bfloat16)
    inputs = values if layout == "packed" else tuple(values.unbind())
    runs = []
    for _ in range(3):
        output = attnres(inputs, query)
        runs.append((output, *torch.autograd.grad(output, (values, query), upstream)))
    for other in runs[1:]:
        for a, b in zip(runs[0], other):
            assert torch.equal(a, b)


def test_duplicate_consumers_accumulate():
    """Block-style reads: a source read by several queries and a duplicated
    consumer accumulate gradients (reference validation/gpu_checks.py:47-74)."""
    torch.manual_seed(SEEDS[0])
    s, n, d, rank = 3, 11, 128, 16
    source = torch.randn(s, n, d, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    partial = torch.randn(n, d, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    queries = (torch.randn(3, rank, device="cuda", dtype=torch.bfloat16) * 0.25).requires_grad_()
    weights = [torch.randn(d, n, device="cuda", dtype=torch.bfloat16).T for _ in range(5)]

    def loss_of(read, leaves, ws):
        src, part, qs = leaves
        combined = torch.cat((src, part[None]), dim=0)
        outputs = [read(combined, qs[i]) for i in (0, 1, 1, 2)]
        outputs.append(read(src, qs[0]))
        return sum((o.float() * w.float()).sum() for o, w in zip(outputs, ws))

    from oracle.oracle import oracle
    leaves = (source, partial, queries)
    actual = torch.autograd.grad(loss_of(attnres, leaves, weights), leaves)
    cpu = tuple(t.detach().cpu().requires_grad_() for t in leaves)
    expected = torch.autograd.grad(loss_of(oracle, cpu, [w.cpu() for w in weights]), cpu)
    repeat = torch.autograd.grad(loss_of(attnres, leaves, weights), leaves)
    for a, e, r in zip(actual, expected, repeat):
        compare(a, e)
        assert torch.equal(a, r)


def test_source_offsets_above_int32():
    """Sources more than 2^31 elements apart (reference tests/test_offsets.py:13-37)."""
    torch.manual_seed(SEEDS[0])
    width, rank = 8192, 127
    stride = 2**31 + 32
    storage = torch.empty(stride + width + rank, device="cuda", dtype=torch.bfloat16)
    values = storage.as_strided((2, 1, width), (stride, width, 1)).detach()
    values.copy_(torch.randn_like(values))
    values.requires_grad_()
    query = (torch.randn(rank, device="cuda", dtype=torch.bfloat16) * 0.25).requires_grad_()
    upstream = torch.randn(1, width, device="cuda", dtype=torch.bfloat16)
    set_case("source offsets > 2^31")
    actual = attnres(values, query)
    grads = torch.autograd.grad(actual, (values, query), upstream)
    expected, exact = both_oracles(lambda ls, q: (ls[0], q), [values], query, upstream)
    compare_read((actual, *grads), expected, exact, ["out", "dv", "dq"], sources=2)
    del storage


@pytest.mark.parametrize("rank", [17, 5])
def test_source_list_row_stride_above_int32(rank):
    """A list source whose row stride exceeds 2^31 elements
    (reference tests/test_offsets.py:40-59)."""
    torch.manual_seed(SEEDS[0])
    width = 17
    stride = 2**31 + 32
    storage = torch.empty(stride + width + rank, device="cuda", dtype=torch.bfloat16)
    value = storage.as_strided((2, width), (stride, 1)).detach()
    value.copy_(torch.randn_like(value))
    value.requires_grad_()
    other = torch.randn(2, width, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    query = (torch.randn(rank, device="cuda", dtype=torch.bfloat16) * 0.25).requires_grad_()
    upstream = torch.randn(2, width, device="cuda", dtype=torch.bfloat16)
    set_case(f"list row stride > 2^31 R={rank}")
    actual = attnres((value, other), query)
    grads = torch.autograd.grad(actual, (value, other, query), upstream)
    expected, exact = both_oracles(lambda ls, q: (tuple(ls), q), [value, other], query, upstream)
    compare_read((actual, *grads), expected, exact, ["out", "dv0", "dv1", "dq"], sources=2)
    del storage
