"""The BASELINE configurations at full size against the CPU oracle.

Every token row is compared.  The oracle runs over token chunks
(`oracle.oracle_chunks`: the oracle's own graph per chunk; tokens are
independent, so a chunk's output and value-gradient rows are exactly the
whole read's), and the query gradient is the chunks' unrounded gradients
summed and rounded once.  Bars (tests/helpers.py): the BF16 gate against the
BF16 oracle, one BF16 ulp against the float64 oracle (value gradients of
reads that save their output with the delta allowance), and the saved
statistics within 1e-5 relative of the oracle's.

* c1: the CPU plumbing configuration's exact inputs (packed [8, 2, 512, 1024],
  R = 1024, seed 0, drawn on the CPU by `bench.make_inputs` as
  ``bench.py --config c1`` draws them).
* c2 packed [25, 8x2048, 2048] R = 2048 and c3 packed [16, 16384, 4096]
  R = 1024 with `bench.make_inputs` (per-source std U[0.5, 4], 1% of channels
  x8); c4: 9 separately allocated [32768, 2048] sources (`bench.make_block_sources`),
  its first read.  All rows against the float64 oracle too.
* c5 subset at N = 16384: S in {1, 6, 7, 12, 13, 25, 48} x D in {1024, 4096}
  x R in {D, D/4}, the first S sources of the tensor ``bench.py --config c5``
  sweeps: every row and dq against the BF16 oracle (dq within one ulp of it:
  both are FP32 sums rounded once), three 512-token samples against float64.

Also at full size: a token sample read on its own gives bit-identical output
and value-gradient rows (no interference between tokens at another grid size).
"""

from __future__ import annotations

import pytest
import torch

import bench
from attnres import attnres
from helpers import DELTA_SIGMAS, Streamed, check_statistics, compare, delta_allowance, saves_output, set_case
from oracle.oracle import oracle_chunks

pytestmark = pytest.mark.gpu

_C5_SOURCES = (1, 6, 7, 12, 13, 25, 48)


def _read(values, query, upstream, listed):
    """The HIP read and its gradients; values packed [S, ..., D] or a list."""
    if listed:
        leaves = [v.detach().requires_grad_() for v in values]
        q = query.detach().requires_grad_()
        out = attnres(tuple(leaves), q)
        grads = torch.autograd.grad(out, (*leaves, q), upstream)
        return out, list(grads[:-1]), grads[-1]
    leaf = values.detach().requires_grad_()
    q = query.detach().requires_grad_()
    out = attnres(leaf, q)
    dv, dq = torch.autograd.grad(out, (leaf, q), upstream)
    return out, dv, dq


def _rows(values, listed, start, stop):
    return [v[start:stop] for v in values] if listed else values[:, start:stop]


def _stack(rows, listed):
    return torch.stack(rows) if listed else rows


def _check_full(values, query, upstream, *, listed, chunk=2048, exact_all=True):
    """Every row of the read against the chunked oracle.  ``exact_all``: every
    chunk and dq against float64 too; else three 512-token samples against
    float64 and dq against the BF16 oracle."""
    width = int(upstream.shape[-1])
    tokens = int(values[0].shape[0]) if listed else values.numel() // (values.shape[0] * width)
    flat = values if listed else values.reshape(values.shape[0], tokens, width)
    g = upstream.reshape(tokens, width)
    out, dv, dq = _read(flat, query, g, listed)
    torch.cuda.synchronize()
    sources = len(values) if listed else int(values.shape[0])
    saved = saves_output(sources, width, int(query.numel()))
    out_check, dv_check = Streamed("out"), Streamed("dv", allowance=saved)
    dq32 = dq64 = None
    dq_variance = torch.zeros(int(query.numel()), dtype=torch.float64)

    def rows_of(start, stop, exact):
        return next(oracle_chunks(_rows(flat, listed, start, stop), query, g[start:stop], chunk=stop - start,
                                  exact=exact))

    def add(start, stop, o, rows, o64=None, rows64=None, whole=False):
        """``whole``: a chunk of the pass over every token (its dq variance counts)."""
        nonlocal dq_variance
        out_check.add(out[start:stop], o, o64)
        extra = None
        if saved and (rows64 is not None or whole):
            packed = _stack([r.cpu() for r in _rows(flat, listed, start, stop)], True) if listed \
                else flat[:, start:stop].cpu()
            extra, variance = delta_allowance(packed.double(), query.cpu().double(), g[start:stop].cpu().double())
            if whole:
                dq_variance = dq_variance + variance
        dv_check.add(_stack(_rows(dv, listed, start, stop), listed), _stack(rows, listed),
                     None if rows64 is None else _stack(rows64, listed), extra)

    for start in range(0, tokens, chunk):
        stop = min(tokens, start + chunk)
        _, _, o, rows, q_part = rows_of(start, stop, False)
        dq32 = q_part if dq32 is None else dq32 + q_part
        o64 = rows64 = None
        if exact_all:
            _, _, o64, rows64, q64 = rows_of(start, stop, True)
            dq64 = q64 if dq64 is None else dq64 + q64
        add(start, stop, o, rows, o64, rows64, whole=True)
    if not exact_all:
        for start in sorted({0, tokens // 2, max(0, tokens - 512)}):
            stop = min(tokens, start + 512)
            _, _, o, rows, _ = rows_of(start, stop, False)
            _, _, o64, rows64, _ = rows_of(start, stop, True)
            add(start, stop, o, rows, o64, rows64)
    out_check.finish()
    dv_check.finish()
    dq_extra = DELTA_SIGMAS * dq_variance.sqrt() if saved else None
    metrics = compare(dq, dq32.to(torch.bfloat16), exact=dq64, name="dq", extra=dq_extra)
    if dq64 is None:
        assert metrics["ulp_vs_oracle"] <= 1.0, f"dq: {metrics['ulp_vs_oracle']:.3f} ulps from the BF16 oracle"
    check_statistics(flat, query)
    return out, dv


def _independent_sample(values, query, upstream, listed, out, dv):
    """A token sample read on its own reproduces the full read's rows bit for bit."""
    width = int(upstream.shape[-1])
    tokens = int(values[0].shape[0]) if listed else values.numel() // (values.shape[0] * width)
    flat = values if listed else values.reshape(values.shape[0], tokens, width)
    generator = torch.Generator(device="cuda").manual_seed(17)
    sample = torch.randperm(tokens, generator=generator, device="cuda")[:96].sort().values
    part = [v[sample].contiguous() for v in flat] if listed else flat[:, sample].contiguous()
    sub_out, sub_dv, _ = _read(part, query, upstream.reshape(tokens, width)[sample], listed)
    assert torch.equal(sub_out, out.reshape(tokens, width)[sample])
    full_dv = torch.stack(dv) if listed else dv.reshape(dv.shape[0], tokens, width)
    assert torch.equal(_stack(sub_dv, listed), full_dv[:, sample])


@pytest.mark.parametrize("name", ["c1", "c2", "c3"])
def test_packed_config_every_row_matches_oracle(name):
    cfg = bench.CONFIGS[name]
    print(f"full size {name}: {cfg['name']}", flush=True)
    set_case(f"{name} full size")
    values, query, upstream = bench.make_inputs(cfg, "cuda", seed=0)
    out, dv = _check_full(values, query, upstream, listed=False)
    _independent_sample(values, query, upstream, False, out, dv)


def test_block_list_config_every_row_matches_oracle():
    cfg = bench.CONFIGS["c4"]
    print(f"full size c4: {cfg['name']}", flush=True)
    set_case("c4 full size (first read)")
    sources, queries, upstreams = bench.make_block_sources(cfg, "cuda", seed=0)
    out, dv = _check_full(sources, queries[0], upstreams[0], listed=True)
    _independent_sample(sources, queries[0], upstreams[0], True, out, dv)


@pytest.mark.parametrize("sources", _C5_SOURCES)
@pytest.mark.parametrize("width,rank", [(1024, 1024), (1024, 256), (4096, 4096), (4096, 1024)],
                         ids=lambda v: str(v))
def test_sweep_subset_matches_oracle(width, rank, sources):
    """One read of the c5 subset per test (its rows are the first S sources of
    the sweep's [48, N, D] input), so that no single test runs for minutes."""
    tokens = bench.CONFIGS["c5"]["batch"][0]
    values, query, upstream = bench.make_inputs(dict(sources=max(_C5_SOURCES), batch=(tokens,), width=width,
                                                     rank=rank), "cuda", seed=width + rank)
    print(f"c5 subset S={sources} N={tokens} D={width} R={rank}", flush=True)
    set_case(f"c5 S={sources} D={width} R={rank}")
    _check_full(values[:sources], query, upstream, listed=False,
                chunk=2048 if width <= 1024 else 1024, exact_all=False)


def test_block_list_three_shared_reads_full_size():
    """c4 as its step runs it: the three reads of the 9 shared sources through
    `SharedSources`, whose backward adds each read's dv to the sources'
    gradients inside the kernel.  Every row of every source's summed gradient
    against the exact sum of the three reads' float64 gradients, within
    `helpers.accumulated_bound` (three BF16 roundings, each read's FP32 floor
    and delta allowance); every output row within one ulp of float64; each
    query's gradient within one ulp of float64 plus its allowance."""
    from attnres import SharedSources
    from helpers import DELTA_SIGMAS, accumulated_bound, check_accumulated, exact_grads, ulp_error

    cfg = bench.CONFIGS["c4"]
    print(f"full size c4, three shared reads: {cfg['name']}", flush=True)
    set_case("c4 full size, three shared reads")
    sources, queries, upstreams = bench.make_block_sources(cfg, "cuda", seed=0)
    leaves = [s.requires_grad_() for s in sources]
    queries = [q.requires_grad_() for q in queries]
    bank = SharedSources(leaves)
    outs = [bank.read(q) for q in queries]
    results = torch.autograd.grad(sum((o.float() * g.float()).sum() for o, g in zip(outs, upstreams)),
                                  (*leaves, *queries))
    torch.cuda.synchronize()
    count, tokens = len(leaves), int(leaves[0].shape[0])
    make = lambda ls, q: (tuple(ls), q)  # noqa: E731
    dq_exact = [0.0] * len(queries)
    dq_variance = [0.0] * len(queries)
    worst = 0.0
    for start in range(0, tokens, 2048):
        stop = min(tokens, start + 2048)
        rows = [leaf[start:stop] for leaf in leaves]
        per_read = [exact_grads(make, rows, q, g[start:stop]) for q, g in zip(queries, upstreams)]
        for r, (out64, grads64) in enumerate(per_read):
            assert ulp_error(outs[r][start:stop], out64) <= 1.0, f"read {r} output rows {start}..{stop}"
            dq_exact[r] = dq_exact[r] + grads64[count]
            dq_variance[r] = dq_variance[r] + (grads64[count].dq_allowance / DELTA_SIGMAS) ** 2
        for i in range(count):
            contributions = [grads64[i] for _, grads64 in per_read]
            bound = accumulated_bound(contributions, [c.dv_allowance for c in contributions], roundings=len(per_read))
            worst = max(worst, check_accumulated(results[i][start:stop], sum(contributions), bound,
                                                 f"source {i} rows {start}..{stop}"))
    print(f"  worst error / bound over every source row: {worst:.3f}", flush=True)
    for r in range(len(queries)):
        allowance = DELTA_SIGMAS * dq_variance[r].sqrt()
        assert ulp_error(results[count + r], dq_exact[r], extra=allowance) <= 1.0, f"dq of read {r}"
