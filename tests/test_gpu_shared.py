"""SharedSources on the GPU: several reads of one source list whose source
gradients are summed inside the backward kernels.

Compared with the same reads through ``attnres`` (autograd sums the
per-read BF16 gradients with add kernels) and with the oracle: outputs and
dq are bit-identical to ``attnres`` (same kernels); the source gradients
agree to the rounding of a BF16 sum (the bank adds each read's FP32 dv to the
running BF16 sum; autograd adds BF16-rounded dv) and match the oracle's
summed gradients to the BF16 gate.  The shapes follow config c4 at a reduced
token count (9 separately allocated sources, 3 reads) plus a masked width.
Reads that need no gradient run the forward alone, with the same output bits.
"""

from __future__ import annotations

import gc
import math

import pytest
import torch

from attnres import SharedSources, attnres
from helpers import accumulated_bound, check_accumulated, compare, exact_grads, oracle_grads, set_case, ulp_error
from oracle.oracle import oracle

pytestmark = pytest.mark.gpu


def _case(sources=9, tokens=(2, 301), width=2048, rank=2048, reads=3, seed=31):
    torch.manual_seed(seed)
    src = [(torch.randn(*tokens, width, device="cuda") * (0.5 + s / 4)).to(torch.bfloat16).requires_grad_()
           for s in range(sources)]
    queries = [(torch.randn(rank, device="cuda") / math.sqrt(rank)).to(torch.bfloat16).requires_grad_()
               for _ in range(reads)]
    grads = [torch.randn(*tokens, width, device="cuda").to(torch.bfloat16) for _ in range(reads)]
    scales = [1.0, 0.5, 2.0][:reads]
    return src, queries, grads, scales


def _run(read_fn, src, queries, grads, scales):
    outs = [read_fn(q, s) for q, s in zip(queries, scales)]
    loss = sum((o.float() * g.float()).sum() for o, g in zip(outs, grads))
    params = (*src, *queries)
    return outs, torch.autograd.grad(loss, params)


@pytest.mark.parametrize("width,rank", [(2048, 2048), (1000, 96)], ids=["d2048_r2048", "d1000_r96"])
def test_shared_sources_match_autograd_sums_and_the_oracle(width, rank):
    src, queries, grads, scales = _case(width=width, rank=rank)
    print(f"shared sources width={width} rank={rank}", flush=True)
    bank = SharedSources(src)
    outs_bank, grads_bank = _run(lambda q, s: bank.read(q, scale=s), src, queries, grads, scales)
    outs_ref, grads_ref = _run(lambda q, s: attnres(tuple(src), q, scale=s), src, queries, grads, scales)
    torch.cuda.synchronize()
    count = len(src)
    for a, b in zip(outs_bank, outs_ref):
        assert torch.equal(a, b)
    for a, b in zip(grads_bank[count:], grads_ref[count:]):
        # dq: the same terms summed in the order of each kernel's grid; at D = 2048, R = D the
        # plain read runs the token-block backward, whose grid differs from the accumulating one
        assert ulp_error(a, b.double()) <= 1.0
    _check_against_float64(src, queries, grads, scales, grads_bank, f"shared sources D={width} R={rank}")


def _check_against_float64(src, queries, grads, scales, results, case):
    """Each source's gradient summed over the reads by the accumulating
    kernel against the exact sum of the reads' float64 gradients, within
    `helpers.accumulated_bound`: one BF16 rounding per read (the first read
    writes bf16(dv), each later one bf16(old + dv)), each read's FP32 floor
    and its delta allowance (these reads save their output).  Each query's
    gradient is one read's dq: one ulp of float64 plus its allowance, and the
    BF16 oracle's gate."""
    count = len(src)
    make = lambda leaves, q: (tuple(leaves), q)  # noqa: E731
    per_read = [exact_grads(make, src, q, g, scale=s)[1] for q, g, s in zip(queries, grads, scales)]
    set_case(case)
    for i in range(count):
        contributions = [grads64[i] for grads64 in per_read]
        bound = accumulated_bound(contributions, [c.dv_allowance for c in contributions], roundings=len(per_read))
        check_accumulated(results[i], sum(contributions), bound, f"dv{i}")
    for r, (q, g, s) in enumerate(zip(queries, grads, scales)):
        expected = oracle_grads(make, src, q, g, scale=s)[1][count]
        exact = per_read[r][count]
        compare(results[count + r], expected, exact=exact, name=f"dq{r}", extra=exact.dq_allowance)


def test_each_backward_pass_starts_a_fresh_sum():
    src, queries, grads, scales = _case(sources=7, tokens=(64,), width=512, rank=512, reads=2)
    bank = SharedSources(src)
    outs = [bank.read(q, scale=s) for q, s in zip(queries, scales)]
    loss = sum((o.float() * g.float()).sum() for o, g in zip(outs, grads))
    first = torch.autograd.grad(loss, src, retain_graph=True)
    second = torch.autograd.grad(loss, src)
    for a, b in zip(first, second):
        assert torch.equal(a, b)


def test_unused_reads_and_sources_without_grad():
    # 7 sources: attnres saves the refinement too (smaller reads use the recompute
    # kernel, SharedSources always the saved one), so the results are bit-identical
    src, queries, grads, scales = _case(sources=7, tokens=(40,), width=256, rank=64, reads=2)
    src[1].requires_grad_(False)
    bank = SharedSources(src)
    used = bank.read(queries[0])
    bank.read(queries[1])  # never reaches the loss: its backward does not run
    g0, g2, gq = torch.autograd.grad((used.float() * grads[0].float()).sum(), (src[0], src[2], queries[0]))
    ref = attnres(tuple(src), queries[0])
    r0, r2, rq = torch.autograd.grad((ref.float() * grads[0].float()).sum(), (src[0], src[2], queries[0]))
    assert torch.equal(g0, r0) and torch.equal(g2, r2) and torch.equal(gq, rq)


def _stream_case(width, rank, events=4, seed=41, tokens=37):
    torch.manual_seed(seed)
    embedded = torch.randn(2, tokens, width, device="cuda", requires_grad=True)
    weights = [torch.randn(width, width, device="cuda") / math.sqrt(width) for _ in range(events)]
    queries = [(torch.randn(rank, device="cuda") / math.sqrt(rank)).requires_grad_() for _ in range(events)]
    grads = [torch.randn(2, tokens, width, device="cuda") for _ in range(events)]
    return embedded, weights, queries, grads


def _run_stream(read, push, embedded, weights, queries):
    """Full-schedule stream: read all sources so far, transform, push; FP32 outside the reads."""
    push(embedded)
    outs = []
    for weight, query in zip(weights, queries):
        x = read(query)
        outs.append(x)
        push(torch.tanh(x @ weight))
    return outs


@pytest.mark.parametrize("gradients", ["gather", "accumulate"])
@pytest.mark.parametrize("width,rank", [(512, 512), (1024, 128)], ids=["d512_r512", "d1024_r128"])
def test_source_bank_matches_the_plain_stream_and_the_oracle(width, rank, gradients):
    from attnres import SourceBank

    embedded, weights, queries, grads = _stream_case(width, rank)
    print(f"source bank width={width} rank={rank} gradients={gradients}", flush=True)
    bank = SourceBank(len(weights) + 1, gradients=gradients)
    outs_bank = _run_stream(lambda q: bank.read(q.to(torch.bfloat16)).float(), bank.push, embedded, weights, queries)
    sources = []
    outs_ref = _run_stream(
        lambda q: attnres(torch.stack([s.to(torch.bfloat16) for s in sources]), q.to(torch.bfloat16)).float(),
        sources.append, embedded, weights, queries)
    for a, b in zip(outs_bank, outs_ref):
        assert torch.equal(a, b)
    params = (embedded, *queries)
    g_bank = torch.autograd.grad(outs_bank, params, grads)
    g_ref = torch.autograd.grad(outs_ref, params, grads)
    for a, b in zip(g_bank, g_ref):
        # FP32 sums of FP32 dv (bank) vs FP32 sums of BF16-rounded dv (plain path)
        torch.testing.assert_close(a, b, rtol=2.0**-6, atol=2.0**-6 * float(b.abs().max()))
    cpu = [t.detach().cpu().requires_grad_() for t in params]
    cpu_sources = []

    def oracle_read(q):
        return oracle(tuple(s.to(torch.bfloat16) for s in cpu_sources), q.to(torch.bfloat16)).float()

    outs_cpu = _run_stream(oracle_read, cpu_sources.append, cpu[0], [w.cpu() for w in weights], cpu[1:])
    g_cpu = torch.autograd.grad(outs_cpu, cpu, [g.cpu() for g in grads])
    for a, e in zip(g_bank, g_cpu):
        # the stream carries each read's last-ulp BF16 differences through tanh and later
        # reads, so the gate is on the gradient's scale, as for the model caller (the first
        # read has one source: its dq is exactly zero on both sides)
        error = float((a.cpu() - e).abs().max() / e.abs().max().clamp_min(1e-12))
        print(f"  relative to scale {float(e.abs().max()):.3g}: {error:.3g}", flush=True)
        assert error < 2e-2
    assert len(bank) == len(weights) + 1
    with pytest.raises(ValueError, match="full"):
        bank.push(embedded)


def test_a_pass_that_stops_short_leaves_no_stale_sum():
    # autograd.grad with respect to the queries only runs the reads' backward but never
    # the node that hands the sums to the sources; the next pass must start afresh
    from attnres import SourceBank

    src, queries, grads, scales = _case(sources=7, tokens=(64,), width=512, rank=512, reads=2)
    shared = SharedSources(src)
    outs = [shared.read(q, scale=s) for q, s in zip(queries, scales)]
    loss = sum((o.float() * g.float()).sum() for o, g in zip(outs, grads))
    torch.autograd.grad(loss, queries, retain_graph=True)
    full = torch.autograd.grad(loss, src)
    ref_outs = [attnres(tuple(src), q, scale=s) for q, s in zip(queries, scales)]
    ref = torch.autograd.grad(sum((o.float() * g.float()).sum() for o, g in zip(ref_outs, grads)), src)
    for a, b in zip(full, ref):
        torch.testing.assert_close(a.float(), b.float(), rtol=2.0**-6, atol=2.0**-6 * float(b.float().abs().max()))

    embedded, weights, qs, gs = _stream_case(256, 256, events=3)
    bank = SourceBank(4)
    outs = _run_stream(lambda q: bank.read(q.to(torch.bfloat16)).float(), bank.push, embedded, weights, qs)
    loss = sum((o * g).sum() for o, g in zip(outs, gs))
    torch.autograd.grad(loss, qs, retain_graph=True)
    first = torch.autograd.grad(loss, embedded, retain_graph=True)[0]
    kept = first.clone()
    second = torch.autograd.grad(loss, embedded)[0]
    assert torch.equal(first, second)
    assert torch.equal(first, kept)  # the second pass did not write into the first pass's sums


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 37, 512), (3, 5, 13)], ids=["vector", "ragged"])
def test_push_sum_is_the_add_and_the_cast(shape, dtype):
    """push_sum == (prev + emitted, bf16 of it) bit for bit, on the vectorised
    and the element-wise path; its gradient reaches both inputs."""
    from attnres import SourceBank

    torch.manual_seed(43)
    prev = torch.randn(*shape, device="cuda", dtype=dtype, requires_grad=True)
    emitted = torch.randn(*shape, device="cuda", dtype=dtype, requires_grad=True)
    bank = SourceBank(2)
    bank.push(prev, slot=0)
    partial = bank.push_sum(prev, emitted, slot=1)
    expected = prev + emitted
    assert partial.dtype == dtype and torch.equal(partial, expected)
    assert torch.equal(bank._state._values[1], expected.to(torch.bfloat16))
    grad = torch.randn_like(partial)
    gp, ge = torch.autograd.grad(partial, (prev, emitted), grad)
    assert torch.equal(gp, grad) and torch.equal(ge, grad)


@pytest.mark.parametrize("gradients", ["gather", "accumulate"])
def test_source_bank_tail_reads_match_attnres(gradients):
    """Block-style reads (completed slots plus a partial in a tail slot)
    against attnres over the same BF16 sources: outputs and dq identical,
    source gradients equal to autograd's sums within BF16 rounding."""
    from attnres import SourceBank

    torch.manual_seed(47)
    width, rank, tokens = 1024, 256, (2, 33)
    blocks = [torch.randn(*tokens, width, device="cuda", requires_grad=True) for _ in range(3)]
    emitted = [torch.randn(*tokens, width, device="cuda", requires_grad=True) for _ in range(3)]
    queries = [(torch.randn(rank, device="cuda") / math.sqrt(rank)).to(torch.bfloat16).requires_grad_()
               for _ in range(4)]
    grads = [torch.randn(*tokens, width, device="cuda") for _ in range(4)]

    def run(bank_mode):
        outs = []
        if bank_mode:
            bank = SourceBank(6, gradients=gradients)
            for i, block in enumerate(blocks):
                bank.push(block, slot=i)
            bank.push(emitted[0], slot=3)
            outs.append(bank.read(queries[0], count=3, tail=3).float())
            partial = bank.push_sum(emitted[0], emitted[1], slot=4)
            outs.append(bank.read(queries[1], count=3, tail=4).float())
            partial = bank.push_sum(partial, emitted[2], slot=5)
            outs.append(bank.read(queries[2], count=2, tail=5).float())
            outs.append(bank.read(queries[3], count=3).float())
        else:
            bf = [b.to(torch.bfloat16) for b in blocks]
            outs.append(attnres((*bf, emitted[0].to(torch.bfloat16)), queries[0]).float())
            partial = emitted[0] + emitted[1]
            outs.append(attnres((*bf, partial.to(torch.bfloat16)), queries[1]).float())
            partial = partial + emitted[2]
            outs.append(attnres((*bf[:2], partial.to(torch.bfloat16)), queries[2]).float())
            outs.append(attnres(torch.stack(bf), queries[3]).float())
        params = (*blocks, *emitted, *queries)
        return outs, torch.autograd.grad(outs, params, grads)

    print(f"source bank tail reads gradients={gradients}", flush=True)
    outs_bank, g_bank = run(True)
    outs_ref, g_ref = run(False)
    for a, b in zip(outs_bank, outs_ref):
        assert torch.equal(a, b)
    # dq: for these 4- and 3-source reads attnres takes the recompute kernel (delta from the
    # value rows) and the bank the saved refinement
    for sources, a, b in zip((4, 4, 3, 3), g_bank[-4:], g_ref[-4:]):
        if sources > 6:
            assert torch.equal(a, b)
        else:
            assert float((a.float() - b.float()).norm() / b.float().norm()) < 2e-3
    for a, b in zip(g_bank[:-4], g_ref[:-4]):
        torch.testing.assert_close(a, b, rtol=2.0**-6, atol=2.0**-6 * float(b.abs().max()))


def test_gather_matches_accumulate_over_many_reads():
    """A slot read by more reads than one gather launch takes (48), with two
    query lengths among them: the gathered gradients equal the accumulated
    ones to FP32 rounding."""
    from attnres import SourceBank

    torch.manual_seed(59)
    width, tokens, reads = 512, (67,), 53
    sources = [torch.randn(*tokens, width, device="cuda", requires_grad=True) for _ in range(3)]
    queries = [(torch.randn(width if r % 3 else 128, device="cuda") / 8).to(torch.bfloat16) for r in range(reads)]
    grads = [torch.randn(*tokens, width, device="cuda") for _ in range(reads)]
    results = {}
    for mode in ("gather", "accumulate"):
        bank = SourceBank(3, gradients=mode)
        for source in sources:
            bank.push(source)
        outs = [bank.read(q, count=1 + r % 3).float() for r, q in enumerate(queries)]
        results[mode] = torch.autograd.grad(outs, sources, grads)
    for a, b in zip(results["gather"], results["accumulate"]):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5 * float(b.abs().max()))


def test_source_bank_rejects_misuse():
    from attnres import SourceBank

    width = 64
    a = torch.randn(3, width, device="cuda")
    bank = SourceBank(4)
    assert bank.push(a) == 0 and len(bank) == 1
    with pytest.raises(ValueError, match="already holds"):
        bank.push(a, slot=0)
    with pytest.raises(ValueError, match="slot must be"):
        bank.push(a, slot=4)
    with pytest.raises(ValueError, match="same logical shape"):
        bank.push(torch.randn(2, width, device="cuda"))
    with pytest.raises(TypeError, match="floating-point"):
        bank.push(torch.ones(3, width, device="cuda", dtype=torch.int32))
    query = torch.randn(width, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="pushed slots"):
        bank.read(query, count=2)  # slot 1 is empty
    bank.push(a, slot=2)
    with pytest.raises(ValueError, match="needs count"):
        bank.read(query, tail=2)
    with pytest.raises(ValueError, match="tail must be"):
        bank.read(query, count=1, tail=3)  # not pushed
    with pytest.raises(ValueError, match="push_sum needs"):
        bank.push_sum(a, a.double(), slot=3)
    with pytest.raises(TypeError, match="float32 and bfloat16"):
        bank.push_sum(a.half(), a.half(), slot=3)
    out = bank.read(query, count=1, tail=2)  # slots 0 and 2
    assert out.shape == (3, width) and out.dtype == torch.bfloat16
    with pytest.raises(ValueError, match="gradients must be"):
        SourceBank(2, gradients="sum")


def test_source_bank_source_also_used_outside_the_bank():
    """A pushed source that also feeds other ops gets both gradients summed by autograd."""
    from attnres import SourceBank

    torch.manual_seed(67)
    width, rank = 256, 64
    x = torch.randn(5, width, device="cuda", requires_grad=True)
    y = torch.randn(5, width, device="cuda", requires_grad=True)
    query = (torch.randn(rank, device="cuda") / 8).to(torch.bfloat16)
    for mode in ("gather", "accumulate"):
        bank = SourceBank(2, gradients=mode)
        bank.push(x)
        bank.push(y)
        loss = (bank.read(query).float() * 3).sum() + (x * x).sum()
        gx, gy = torch.autograd.grad(loss, (x, y))
        ref = attnres(torch.stack([x.to(torch.bfloat16), y.to(torch.bfloat16)]), query)
        rx, ry = torch.autograd.grad((ref.float() * 3).sum() + (x * x).sum(), (x, y))
        torch.testing.assert_close(gx, rx, rtol=2.0**-6, atol=2.0**-6 * float(rx.abs().max()))
        torch.testing.assert_close(gy, ry, rtol=2.0**-6, atol=2.0**-6 * float(ry.abs().max()))


def test_banks_free_their_buffers_with_the_graph():
    """The buffers of a SourceBank (slots, sums, kept dO rows) and of a
    SharedSources (sums) are freed as soon as the graph and the outputs are
    gone, with Python's cycle collector off: nothing forms a reference cycle
    through the bank object."""
    from attnres import SourceBank

    embedded, weights, queries, grads = _stream_case(512, 512)
    src, shared_queries, shared_grads, _ = _case(sources=7, tokens=(64,), width=512, rank=512, reads=2)
    gc.collect()
    torch.cuda.synchronize()
    gc.disable()
    try:
        before = torch.cuda.memory_allocated()
        for gradients in ("gather", "accumulate"):
            bank = SourceBank(len(weights) + 1, gradients=gradients)
            outs = _run_stream(lambda q: bank.read(q.to(torch.bfloat16)).float(), bank.push, embedded, weights,
                               queries)
            result = torch.autograd.grad(outs, (embedded, *queries), grads)
            del bank, outs, result
            assert torch.cuda.memory_allocated() == before, gradients
        shared = SharedSources(src)
        outs = [shared.read(q) for q in shared_queries]
        result = torch.autograd.grad(outs, src, shared_grads)
        del shared, outs, result
        assert torch.cuda.memory_allocated() == before
    finally:
        gc.enable()


@pytest.mark.parametrize("width,rank,reads", [(1024, 1024, 4), (1003, 96, 4), (4096, 4096, 3), (256, 256, 50)],
                         ids=["d1024", "d1003_r96_unaligned", "d4096", "d256_50_reads"])
def test_bf16_gathered_gradients_equal_the_converted_fp32_sums(width, rank, reads, monkeypatch):
    """BF16 sources: the gather stores the gradient as BF16 itself, which is
    bit-identical to the FP32 gather converted by torch (both round the same
    FP32 sum once, to nearest even).  With 50 reads slot 0 needs two gather
    launches, so it takes the FP32 path and the conversion in both runs."""
    from attnres import SourceBank, shared

    torch.manual_seed(53)
    embedded = torch.randn(3, 41, width, device="cuda").to(torch.bfloat16).requires_grad_()
    weights = [torch.randn(width, width, device="cuda") / math.sqrt(width) for _ in range(min(reads, 4))]
    queries = [(torch.randn(rank, device="cuda") / math.sqrt(rank)).to(torch.bfloat16).requires_grad_()
               for _ in range(reads)]
    grads = [torch.randn(3, 41, width, device="cuda").to(torch.bfloat16) for _ in range(reads)]
    print(f"bf16 gather width={width} rank={rank} reads={reads}", flush=True)

    def run():
        bank = SourceBank(reads + 1)
        bank.push(embedded)
        outs = []
        for i, query in enumerate(queries):
            x = bank.read(query)
            outs.append(x)
            bank.push(torch.tanh(x.float() @ weights[i % len(weights)]).to(torch.bfloat16))
        return torch.autograd.grad(outs, (embedded, *queries), grads)

    direct = run()
    monkeypatch.setattr(shared, "_BF16_GATHER", False)
    converted = run()
    assert direct[0].dtype == torch.bfloat16
    for a, b in zip(direct, converted):
        assert torch.equal(a, b)


@pytest.mark.parametrize("gradients", ["gather", "accumulate"])
def test_source_bank_on_a_large_grid_matches_the_plain_stream(gradients):
    """N = 4200 tokens at D = 1024: more than 4 wavefronts per CU, so the
    32-lane coefficient backward keeps one row per group (small grids keep
    two); same comparison as the small stream."""
    from attnres import SourceBank

    embedded, weights, queries, grads = _stream_case(1024, 1024, tokens=2100)
    print(f"source bank large grid gradients={gradients}", flush=True)
    bank = SourceBank(len(weights) + 1, gradients=gradients)
    outs_bank = _run_stream(lambda q: bank.read(q.to(torch.bfloat16)).float(), bank.push, embedded, weights, queries)
    sources = []
    outs_ref = _run_stream(
        lambda q: attnres(torch.stack([s.to(torch.bfloat16) for s in sources]), q.to(torch.bfloat16)).float(),
        sources.append, embedded, weights, queries)
    for a, b in zip(outs_bank, outs_ref):
        assert torch.equal(a, b)
    params = (embedded, *queries)
    g_bank = torch.autograd.grad(outs_bank, params, grads)
    g_ref = torch.autograd.grad(outs_ref, params, grads)
    for a, b in zip(g_bank, g_ref):
        torch.testing.assert_close(a, b, rtol=2.0**-6, atol=2.0**-6 * float(b.abs().max()))


@pytest.mark.parametrize("gradients", ["gather", "accumulate"])
@pytest.mark.parametrize("width,rank", [(1024, 1024), (1000, 96), (2048, 512)], ids=["d1024", "d1000_r96", "d2048_r512"])
def test_source_bank_slot_gradients_within_float64_bound(width, rank, gradients):
    """FP32 sources pushed into a bank and read as growing prefixes (2, 3, 4,
    5 slots): each source's gradient is an FP32 sum over the reads that saw
    it (gathered once from the reads' dO rows and coefficients, or added read
    by read), so against the exact float64 sum it may differ only by each
    read's FP32 floor and delta allowance (bank reads save their output); no
    BF16 rounding enters.  Each query's gradient is one read's dq."""
    from attnres import SourceBank

    torch.manual_seed(71 + width)
    tokens = (2, 37)
    leaves = [(torch.randn(*tokens, width, device="cuda") * (0.5 + s / 3)).requires_grad_() for s in range(5)]
    counts = (2, 3, 4, 5)
    queries = [(torch.randn(rank, device="cuda") / math.sqrt(rank)).to(torch.bfloat16).requires_grad_()
               for _ in counts]
    upstream = [torch.randn(*tokens, width, device="cuda") for _ in counts]
    print(f"source bank float64 bound D={width} R={rank} gradients={gradients}", flush=True)
    bank = SourceBank(len(leaves), gradients=gradients)
    for leaf in leaves:
        bank.push(leaf)
    outs = [bank.read(q, count=c).float() for q, c in zip(queries, counts)]
    results = torch.autograd.grad(sum((o * g).sum() for o, g in zip(outs, upstream)), (*leaves, *queries))
    # the reads see the BF16 copies of the sources and the BF16 upstream gradient (the output's cast)
    slots = [leaf.detach().to(torch.bfloat16) for leaf in leaves]
    make = lambda ls, q: (tuple(ls), q)  # noqa: E731
    per_read = [exact_grads(make, slots[:c], q, g.to(torch.bfloat16)) for q, g, c in zip(queries, upstream, counts)]
    set_case(f"source bank D={width} R={rank} {gradients}")
    for i, result in enumerate(results[:len(leaves)]):
        contributions = [grads64[i] for c, (_, grads64) in zip(counts, per_read) if i < c]
        bound = accumulated_bound(contributions, [x.dv_allowance for x in contributions], roundings=0)
        check_accumulated(result, sum(contributions), bound, f"slot{i}")
    for r, (q, g, c) in enumerate(zip(queries, upstream, counts)):
        exact = per_read[r][1][c]
        expected = oracle_grads(make, slots[:c], q, g.to(torch.bfloat16))[1][c]
        compare(results[len(leaves) + r], expected, exact=exact, name=f"dq{r}", extra=exact.dq_allowance)


@pytest.mark.parametrize("gradients", ["gather", "accumulate"])
def test_source_bank_tail_reads_within_float64_bound(gradients):
    """Block-style reads of completed slots plus a partial-sum slot (the FP32
    source-list sums, `ListGradsF32`): blocks b0..b2 in slots 0..2, then
    partials p1 = e0, p2 = e0 + e1, p3 = e0 + e1 + e2 (`push_sum`) read as a
    tail slot.  Each FP32 leaf's gradient against the exact sum of the
    contributions that reach it (a partial's gradient reaches every emitted
    term in it), within each read's FP32 floor and delta allowance."""
    from attnres import SourceBank

    torch.manual_seed(79)
    width, rank, tokens = 1024, 256, (2, 33)
    blocks = [torch.randn(*tokens, width, device="cuda", requires_grad=True) for _ in range(3)]
    emitted = [torch.randn(*tokens, width, device="cuda", requires_grad=True) for _ in range(3)]
    queries = [(torch.randn(rank, device="cuda") / math.sqrt(rank)).to(torch.bfloat16).requires_grad_()
               for _ in range(4)]
    upstream = [torch.randn(*tokens, width, device="cuda") for _ in range(4)]
    print(f"source bank tail reads float64 bound gradients={gradients}", flush=True)
    bank = SourceBank(6, gradients=gradients)
    for i, block in enumerate(blocks):
        bank.push(block, slot=i)
    bank.push(emitted[0], slot=3)
    outs = [bank.read(queries[0], count=3, tail=3).float()]
    partial = bank.push_sum(emitted[0], emitted[1], slot=4)
    outs.append(bank.read(queries[1], count=3, tail=4).float())
    bank.push_sum(partial, emitted[2], slot=5)
    outs.append(bank.read(queries[2], count=2, tail=5).float())
    outs.append(bank.read(queries[3], count=3).float())
    params = (*blocks, *emitted, *queries)
    results = torch.autograd.grad(sum((o * g).sum() for o, g in zip(outs, upstream)), params)

    bf = lambda t: t.detach().to(torch.bfloat16)  # noqa: E731
    p2 = emitted[0].detach() + emitted[1].detach()
    p3 = p2 + emitted[2].detach()
    # (sources of each read, which leaves each source's gradient reaches)
    reads = [([bf(b) for b in blocks] + [bf(emitted[0])], [[0], [1], [2], [3]]),
             ([bf(b) for b in blocks] + [bf(p2)], [[0], [1], [2], [3, 4]]),
             ([bf(b) for b in blocks[:2]] + [bf(p3)], [[0], [1], [3, 4, 5]]),
             ([bf(b) for b in blocks], [[0], [1], [2]])]
    make = lambda ls, q: (tuple(ls), q)  # noqa: E731
    contributions = [[] for _ in range(6)]
    allowances = [[] for _ in range(6)]
    set_case(f"source bank tail reads {gradients}")
    for r, ((sources, reach), q, g) in enumerate(zip(reads, queries, upstream)):
        _, grads64 = exact_grads(make, sources, q, g.to(torch.bfloat16))
        for position, leaves_reached in enumerate(reach):
            for leaf in leaves_reached:
                contributions[leaf].append(grads64[position])
                allowances[leaf].append(grads64[position].dv_allowance)
        dq = grads64[len(sources)]
        expected = oracle_grads(make, sources, q, g.to(torch.bfloat16))[1][len(sources)]
        compare(results[6 + r], expected, exact=dq, name=f"dq{r}", extra=dq.dq_allowance)
    for leaf in range(6):
        bound = accumulated_bound(contributions[leaf], allowances[leaf], roundings=0)
        check_accumulated(results[leaf], sum(contributions[leaf]), bound, f"leaf{leaf}")


@pytest.mark.parametrize("kind", ["shared", "bank", "bank-tail"])
def test_reads_without_gradients_run_the_forward_alone(kind):
    """A SharedSources or SourceBank read that needs no gradient (grad mode
    off, or neither the query nor the sources requiring grad) runs the
    forward alone: no autograd node, no refinement bytes or saved state, and
    the output of the same read with gradients, bit for bit."""
    from attnres import SourceBank

    torch.manual_seed(13)
    print(f"no-grad {kind} read", flush=True)
    sources = [(torch.randn(2, 150, 1024, device="cuda") * (0.5 + s / 4)).to(torch.bfloat16) for s in range(9)]
    query = (torch.randn(1024, device="cuda") / 32).to(torch.bfloat16)

    def read(leaves, q):
        if kind == "shared":
            return SharedSources(leaves).read(q)
        bank = SourceBank(len(leaves))
        for leaf in leaves:
            bank.push(leaf)
        return bank.read(q, count=4, tail=7) if kind == "bank-tail" else bank.read(q)

    trained = read([s.clone().requires_grad_() for s in sources], query.clone().requires_grad_())
    assert trained.grad_fn is not None
    expected = trained.detach().clone()
    del trained
    for mode in ("no_grad", "no input requires grad"):
        if mode == "no_grad":
            with torch.no_grad():
                out = read([s.clone().requires_grad_() for s in sources], query.clone().requires_grad_())
        else:
            out = read(sources, query)
        assert out.grad_fn is None, mode
        assert torch.equal(out, expected), f"{mode}: the output differs from the read with gradients"
