"""Compiler and graph boundaries of the HIP read.

* ``torch.compile(fullgraph=True)`` traces ``attnres`` as a single graph
  through the registered custom ops and their fake kernels (the reference
  tests the same boundary in `tests/test_cuda.py` with `fullgraph=True`).
  With the ``aot_eager`` backend the same HIP kernels run and the results
  equal eager mode bit for bit; new inputs of the same shapes do not
  recompile (dynamo's counters are unchanged).
* Compiled (inductor) reads with strided producers, a strided query and
  transposed upstream gradients, checked against the oracle, then captured in
  a CUDA/HIP graph and replayed on 8 changed inputs, each checked against the
  oracle, with no recompilation (reference `tests/test_full_kernel.py:151-221`).
* The eager read captured in a graph (``torch.cuda.graph``) and replayed on
  changed inputs: each replay equals an eager read of the same inputs bit for
  bit (reference `validation/gpu_checks.py:77-132`).
* Equal logits at |scale| = 2^24 under replay with changed upstream gradients:
  out == v, dv == dO/S, dq == 0 exactly (reference
  `validation/softmax_checks.py:9-52`).

Capture contract (PyTorch's, and the reference harness's,
`validation/gpu_checks.py:99-113`): the static leaves are created on the
capture stream and warmed up there, and ``torch.cuda.graph`` is given that
stream.  A leaf whose autograd accumulator node was created on the default
(legacy) stream and is still alive records that stream in its input metadata,
and the backward pass then synchronises the capture stream with the legacy
stream, which no capture may do.  A kept ``out.clone()`` keeps that node
alive through ``CloneBackward``; the results kept for comparison are detached.
"""

from __future__ import annotations

import math

import pytest
import torch

import attnres._ops  # noqa: F401  (loaded before tracing)
from attnres import attnres
from helpers import SEEDS, both_oracles, compare_read, set_case

pytestmark = pytest.mark.gpu


def _inputs(layout, sources=5, tokens=(3, 129), width=1024, rank=384, seed=20260905):
    torch.manual_seed(seed)
    values = torch.randn(sources, *tokens, width, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    query = (torch.randn(rank, device="cuda", dtype=torch.bfloat16) * 0.25).requires_grad_()
    upstream = torch.randn(*tokens, width, device="cuda", dtype=torch.bfloat16)
    return values, query, upstream


def _read(layout):
    def read(values, query):
        inputs = values if layout == "packed" else tuple(values.unbind(0))
        return attnres(inputs, query, eps=2.0**-20, scale=0.75)
    return read


def _stats():
    return dict(torch._dynamo.utils.counters["stats"])


@pytest.mark.parametrize("layout", ["packed", "list"])
def test_compile_fullgraph_matches_eager_bitwise(layout):
    values, query, upstream = _inputs(layout)
    read = _read(layout)
    print(f"compile fullgraph layout={layout}", flush=True)
    eager = read(values, query)
    eager_grads = torch.autograd.grad(eager, (values, query), upstream)
    torch._dynamo.reset()
    compiled = torch.compile(read, fullgraph=True, backend="aot_eager")
    for _ in range(2):
        out = compiled(values, query)
        grads = torch.autograd.grad(out, (values, query), upstream)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        for g, e in zip(grads, eager_grads):
            assert torch.equal(g, e)
    # new inputs of the same shapes: no recompilation, still eager's bits
    counters = _stats()
    other_values = torch.randn_like(values).requires_grad_()
    other_query = torch.randn_like(query).requires_grad_()
    out = compiled(other_values, other_query)
    grads = torch.autograd.grad(out, (other_values, other_query), upstream)
    assert _stats() == counters, "changed inputs recompiled"
    expected = read(other_values, other_query)
    expected_grads = torch.autograd.grad(expected, (other_values, other_query), upstream)
    assert torch.equal(out, expected)
    for g, e in zip(grads, expected_grads):
        assert torch.equal(g, e)


@pytest.mark.parametrize("layout", ["packed", "list", "list_nonaffine"])
@pytest.mark.parametrize("width,rank", [(17, 5), (63, 33), (1024, 384)], ids=lambda v: str(v))
def test_compiled_changed_inputs_and_graph(layout, width, rank):
    """Reference tests/test_full_kernel.py:151-221 on the HIP read."""
    torch.manual_seed(SEEDS[0])
    source = torch.randn(3, 2, 5, 2 * width, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    query = (torch.randn(2 * rank, device="cuda", dtype=torch.bfloat16) * .25).requires_grad_()
    upstream = torch.randn(width, 5, 2, device="cuda", dtype=torch.bfloat16).permute(2, 1, 0)
    if layout == "list_nonaffine":
        upstream = upstream.transpose(0, 1)
    replay_inputs = [(torch.randn_like(source), torch.randn_like(query) * .25, torch.randn_like(upstream))
                     for _ in range(8)]

    def views(v):
        return (v.transpose(1, 2) if layout == "list_nonaffine" else v)[..., ::2]

    def forward(v, q):
        v = views(v)
        return attnres(v, q[::2]) if layout == "packed" else attnres(tuple(v.unbind(0)), q[::2])

    torch._dynamo.reset()
    compiled = torch.compile(forward, fullgraph=True, dynamic=False)

    def step():
        out = compiled(source, query)
        return (out, *torch.autograd.grad(out, (source, query), upstream))

    def check(actual, label):
        set_case(f"compiled graph {layout} D={width} R={rank} {label}")
        expected, exact = both_oracles(lambda ls, q: (views(ls[0]) if layout == "packed"
                                                      else tuple(views(ls[0]).unbind(0)), q[::2]),
                                       [source], query, upstream)
        compare_read(actual, expected, exact, ["out", "dv", "dq"], sources=3)

    print(f"compiled changed inputs + graph layout={layout} D={width} R={rank}", flush=True)
    check(step(), "first call")
    counters = _stats()
    with torch.no_grad():
        source.copy_(replay_inputs[0][0])
        query.copy_(replay_inputs[0][1])
        upstream.copy_(replay_inputs[0][2])
    check(step(), "changed input")
    assert _stats() == counters, "changed inputs recompiled"
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        captured = step()
    for index, (replay_source, replay_query, replay_upstream) in enumerate(replay_inputs):
        with torch.no_grad():
            source.copy_(replay_source)
            query.copy_(replay_query)
            upstream.copy_(replay_upstream)
        graph.replay()
        torch.cuda.synchronize()
        check(captured, f"replay {index}")
    assert _stats() == counters, "graph capture or replay recompiled"


@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("shape", [(5, (3, 129), 1024, 384), (25, (4, 64), 2048, 2048)],
                         ids=["s5_d1024_r384", "s25_d2048_r2048"])
def test_hip_graph_replays_match_eager(layout, shape):
    """The eager read (forward + backward) captured with ``torch.cuda.graph``
    and replayed on changed inputs; every replay equals an eager read of the
    same inputs bit for bit, with eager reads and synchronisations between
    the replays (reference validation/gpu_checks.py:77-132)."""
    sources, tokens, width, rank = shape
    read = _read(layout)
    print(f"hip graph layout={layout} shape={shape}", flush=True)
    torch.manual_seed(SEEDS[1] + width)
    replay_inputs = [(torch.randn(sources, *tokens, width, device="cuda", dtype=torch.bfloat16),
                      torch.randn(rank, device="cuda", dtype=torch.bfloat16) * 0.25,
                      torch.randn(*tokens, width, device="cuda", dtype=torch.bfloat16)) for _ in range(4)]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        # static leaves made and warmed up on the capture stream
        values = torch.randn(sources, *tokens, width, device="cuda", dtype=torch.bfloat16).requires_grad_()
        query = (torch.randn(rank, device="cuda", dtype=torch.bfloat16) * 0.25).requires_grad_()
        upstream = torch.randn(*tokens, width, device="cuda", dtype=torch.bfloat16)

        def step():
            out = read(values, query)
            return (out, *torch.autograd.grad(out, (values, query), upstream))

        for _ in range(3):
            step()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            captured = step()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()

    def eager_read(v, q, g):
        v, q = v.detach().clone().requires_grad_(), q.detach().clone().requires_grad_()
        out = read(v, q)
        return [t.detach() for t in (out, *torch.autograd.grad(out, (v, q), g))]

    for index, (v, q, g) in enumerate(replay_inputs):
        with torch.no_grad():
            values.copy_(v)
            query.copy_(q)
            upstream.copy_(g)
        graph.replay()
        torch.cuda.synchronize()
        expected = eager_read(v, q, g)
        torch.cuda.synchronize()
        for t, e in zip(captured, expected):
            assert torch.equal(t, e), f"replay {index}"


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("sources,rows", [(2, 2), (4, 2), (4, 1024)])
@pytest.mark.parametrize("scale", [2**24, -(2**24)])
def test_equal_logits_exact_under_graph_replay(sources, rows, packed, scale):
    """Reference validation/softmax_checks.py:9-52: identical sources, replayed
    with changed upstream gradients, give out == v, dv == dO/S and dq == 0."""
    width, rank = 256, 16
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):  # views create autograd nodes too: made on the capture stream
        values = torch.ones(sources, rows, width, device="cuda", dtype=torch.bfloat16, requires_grad=True)
        query = torch.ones(rank, device="cuda", dtype=torch.bfloat16, requires_grad=True)
        inputs = values if packed else tuple(values.unbind())
        upstream = torch.ones_like(values[0])

    def call():
        output = attnres(inputs, query, eps=2**-23, scale=scale)
        return output, *torch.autograd.grad(output, (values, query), upstream)

    def check(result):
        output, dv, dq = result
        torch.testing.assert_close(output, values[0], rtol=0, atol=0)
        torch.testing.assert_close(dv, upstream.expand_as(values) / sources, rtol=0, atol=0)
        torch.testing.assert_close(dq, torch.zeros_like(query), rtol=0, atol=0)

    with torch.cuda.stream(stream):
        check(call())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            result = call()
        for factor in (-2.0, 4.0):
            upstream.fill_(factor)
            graph.replay()
            torch.cuda.synchronize()
            check(result)
    torch.cuda.current_stream().wait_stream(stream)
