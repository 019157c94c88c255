"""The op boundary on the GPU: what the read keeps, copies and traces.

* Lifetimes (reference `tests/test_cuda.py:175-293`): after a completed
  eager, compiled or graph-captured read (Full and Block source forms,
  standard and sliced ranks, packed and list), no input tensor is kept alive
  by the operator; only autograd holds arguments between forward and
  backward.
* Non-affine output batches (reference `tests/test_cuda.py:320-343`): a
  transposed upstream gradient over a batch of tokens, eager and compiled.
* No source stack on the list path (reference
  `validation/source_checks.py:11-37`): a dispatch mode that fails on any
  ``aten.stack`` / ``aten.cat`` whose inputs are the read's sources watches
  an eager and a compiled list read, forward and backward.  A negative control
  shows the guard catches the oracle's own stack.
* The eager C++ nodes against the ops, bit for bit, on every backward path;
  the packed node flattening batch axes itself (no view nodes), on fixed and
  seeded random layouts.
* Reads without gradients (no_grad, inference_mode, no input requiring
  grad), eager and compiled: the forward alone, no saved state, the training
  forward's output bit for bit; checkpointed reads (reentrant or not) against
  the plain read.
"""

from __future__ import annotations

import gc
import weakref

import pytest
import torch

from attnres import attnres
from helpers import SEEDS, SourceStackGuard, both_oracles, compare_read, set_case
from oracle.oracle import oracle

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------- lifetimes

def _lifetime_refs(rank, mode, sequence):
    values = [torch.randn(5, 17, device="cuda", dtype=torch.bfloat16, requires_grad=True) for _ in range(3)]
    query = torch.randn(rank, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    refs = [weakref.ref(tensor) for tensor in (*values, query)]
    inputs = tuple(values) if sequence else torch.stack(values)
    if mode == "block":
        partial = torch.randn_like(values[0], requires_grad=True)
        refs.append(weakref.ref(partial))
        inputs = (*inputs, partial) if sequence else torch.cat((inputs, partial[None]))
    loss = attnres(inputs, query).square().sum()
    # from here on only autograd may hold the arguments
    del values, query, inputs
    if mode == "block":
        del partial
    gc.collect()
    loss.backward()
    return refs


@pytest.mark.parametrize("rank", [17, 5], ids=["standard", "sliced"])
@pytest.mark.parametrize("mode", ["full", "block"])
@pytest.mark.parametrize("sequence", [False, True])
def test_eager_reads_release_their_inputs(rank, mode, sequence):
    torch.manual_seed(SEEDS[0])
    for _ in range(2):
        refs = _lifetime_refs(rank, mode, sequence)
        torch.cuda.synchronize()
        gc.collect()
        assert all(ref() is None for ref in refs), "a completed read kept an input tensor alive"


def _compiled_lifetime_refs(compiled, rank, mode, graph):
    values = tuple(torch.randn(5, 17, device="cuda", dtype=torch.bfloat16, requires_grad=True) for _ in range(3))
    query = torch.randn(rank, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    partial = torch.randn_like(values[0], requires_grad=True) if mode == "block" else None
    leaves = (*values, query, *((partial,) if partial is not None else ()))
    refs = [weakref.ref(tensor) for tensor in leaves]

    def step():
        for tensor in leaves:
            if tensor.grad is not None:
                tensor.grad.zero_()
        compiled(values, query, partial).backward()

    if graph:
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):  # fresh leaves: their accumulators are made on this stream
            step()
            step()
        stream.synchronize()
        captured = torch.cuda.CUDAGraph()
        with torch.cuda.graph(captured, stream=stream):
            step()
        for _ in range(8):
            with torch.no_grad():
                for tensor in leaves:
                    tensor.add_(0.01)
            captured.replay()
        torch.cuda.synchronize()
        del captured, stream
    else:
        loss = compiled(values, query, partial)
        del step, leaves, values, query, partial
        gc.collect()
        loss.backward()
    return refs


@pytest.mark.parametrize("rank", [17, 5], ids=["standard", "sliced"])
@pytest.mark.parametrize("mode", ["full", "block"])
@pytest.mark.parametrize("graph", [False, True], ids=["compiled", "compiled_graph"])
def test_compiled_reads_release_their_inputs(rank, mode, graph):
    counters = torch._dynamo.utils.counters

    def forward(values, query, partial):
        if mode == "full":
            return attnres(values, query).square().sum()
        return attnres((*values, partial), query).square().sum()

    torch.manual_seed(SEEDS[0])
    torch._dynamo.reset()
    compiled = torch.compile(forward, fullgraph=True, dynamic=False)
    graph_breaks = dict(counters["graph_break"])
    graphs = None
    for _ in range(2):
        refs = _compiled_lifetime_refs(compiled, rank, mode, graph)
        torch.cuda.synchronize()
        gc.collect()
        assert all(ref() is None for ref in refs), "a compiled read kept an input tensor alive"
        assert dict(counters["graph_break"]) == graph_breaks
        current = counters["stats"]["unique_graphs"]
        assert graphs is None or current == graphs, "fresh inputs recompiled"
        graphs = current


# ------------------------------------------------------ non-affine batches

@pytest.mark.parametrize("rank", [17, 5], ids=["standard", "sliced"])
@pytest.mark.parametrize("sequence", [False, True])
def test_non_affine_output_batches_keep_every_gradient(rank, sequence):
    torch.manual_seed(SEEDS[0])
    values = torch.randn(3, 2, 3, 17, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    query = torch.randn(rank, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    upstream = torch.randn(3, 2, 17, device="cuda", dtype=torch.bfloat16).transpose(0, 1)

    def forward(v, q):
        return attnres(tuple(v.unbind(0)) if sequence else v, q)

    torch._dynamo.reset()
    for label, function in (("eager", forward), ("compiled", torch.compile(forward, fullgraph=True, dynamic=False))):
        set_case(f"non-affine batch R={rank} sequence={sequence} {label}")
        actual = function(values, query)
        grads = torch.autograd.grad(actual, (values, query), upstream)
        expected, exact = both_oracles(lambda ls, q: (ls[0], q), [values], query, upstream)
        compare_read((actual, *grads), expected, exact, ["out", "dv", "dq"], sources=3)


# --------------------------------------------------------- no source stack

def _list_inputs(count, tokens, width, rank):
    torch.manual_seed(SEEDS[2])
    leaves = [torch.randn(tokens, width, device="cuda", dtype=torch.bfloat16, requires_grad=True)
              for _ in range(count)]
    query = (torch.randn(rank, device="cuda", dtype=torch.bfloat16) * 0.25).requires_grad_()
    upstream = torch.randn(tokens, width, device="cuda", dtype=torch.bfloat16)
    return leaves, query, upstream


@pytest.mark.parametrize("compiled", [False, True], ids=["eager", "compiled"])
@pytest.mark.parametrize("count", [3, 9])
def test_list_path_never_stacks_its_sources(count, compiled):
    leaves, query, upstream = _list_inputs(count, 33, 256, 64)

    def read(*args):
        *sources, q = args
        return attnres(tuple(sources), q)

    torch._dynamo.reset()
    function = torch.compile(read, fullgraph=True, dynamic=False) if compiled else read
    if compiled:  # compile outside the guard, then run the artefact under it
        function(*leaves, query)
    guard = SourceStackGuard([leaf.shape for leaf in leaves], count)
    with guard:
        out = function(*leaves, query)
        grads = torch.autograd.grad(out, (*leaves, query), upstream)
    assert guard.seen > 0, "the guard saw no dispatch"
    set_case(f"no-stack guard count={count} compiled={compiled}")
    expected, exact = both_oracles(lambda ls, q: (tuple(ls), q), leaves, query, upstream)
    compare_read((out, *grads), expected, exact, ["out", *[f"dv{i}" for i in range(count)], "dq"], sources=count)


def test_the_guard_catches_a_stacked_read():
    """Negative control: the oracle stacks its list input, and the guard fails it."""
    leaves = [torch.randn(7, 16, dtype=torch.bfloat16) for _ in range(3)]
    query = torch.randn(16, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="stacked its sources"):
        with SourceStackGuard([leaf.shape for leaf in leaves], 3):
            oracle(tuple(leaves), query)


# ------------------------------------------- eager Function against the ops

@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("shape", [(5, 300, 1024, 1024), (9, 257, 1024, 256), (9, 300, 2048, 2048),
                                   (16, 300, 4096, 1024), (25, 300, 2048, 2048)],
                         ids=["recompute", "saved", "key-resident-row", "key-resident-key", "saved-block"])
def test_eager_function_matches_the_ops_bit_for_bit(layout, shape):
    """In eager mode a read runs through the C++ autograd node of
    csrc/attnres_autograd.cpp, which keeps its saved state in one pooled
    allocation and passes addresses to the library; the registered ops (used
    under torch.compile) allocate each saved tensor apart.  Both must launch the same kernels on the same
    state: out, dv and dq bit-identical, on every backward path (recompute,
    saved refinement, key-resident with a partial and a whole-row key, token
    blocks)."""
    sources, tokens, width, rank = shape
    torch.manual_seed(3)
    print(f"eager vs ops {layout} S,N,D,R={shape}", flush=True)
    values = torch.randn(sources, tokens, width, device="cuda").to(torch.bfloat16)
    query = (torch.randn(rank, device="cuda") / rank ** 0.5).to(torch.bfloat16)
    upstream = torch.randn(tokens, width, device="cuda").to(torch.bfloat16)
    from attnres import _ops  # noqa: F401  (registers the ops)

    if layout == "packed":
        leaf = values.clone().requires_grad_()
        q = query.clone().requires_grad_()
        out = attnres(leaf, q)
        eager = (out, *torch.autograd.grad(out, (leaf, q), upstream))
        saved = torch.ops.attnres_hip.packed_forward(values, query, 2**-23, 1.0)
        grads = torch.ops.attnres_hip.packed_backward(values, query, saved[0], saved[1], upstream, *saved[2:], 1.0)
        ops = (saved[0], *grads)
    else:
        leaves = [values[s].clone().requires_grad_() for s in range(sources)]
        q = query.clone().requires_grad_()
        out = attnres(leaves, q)
        grads = torch.autograd.grad(out, (*leaves, q), upstream)
        eager = (out, torch.stack(grads[:-1]), grads[-1])
        listed = list(values.unbind(0))
        saved = torch.ops.attnres_hip.sources_forward(listed, query, 2**-23, 1.0)
        grads = torch.ops.attnres_hip.sources_backward(listed, query, saved[0], saved[1], upstream, *saved[2:], 1.0)
        ops = (saved[0], torch.stack(grads[:-1]), grads[-1])
    for name, a, b in zip(("out", "dv", "dq"), eager, ops):
        assert torch.equal(a, b), f"{name} differs between the eager Function and the ops"


@pytest.mark.parametrize("layout", ["batch-axes", "uncollapsible", "feature-strided", "no-batch"])
@pytest.mark.parametrize("sources", [5, 9])
def test_eager_node_flattens_batch_axes_itself(layout, sources):
    """The eager node takes packed values [S, ..., D] as they come and
    flattens the batch axes inside its forward (a view where they collapse to
    one row stride, a copy otherwise or when a row is not unit-stride), so
    the graph holds the node alone: no view node between it and the leaf,
    the output in the batch shape, the value gradient in the shape of values.
    Results are those of the ops on the flattened contiguous values,
    bit for bit, on the recompute (S = 5) and saved (S = 9) paths."""
    torch.manual_seed(11)
    width, rank = 1024, 256
    print(f"eager node batch axes {layout} S={sources}", flush=True)
    if layout == "batch-axes":
        leaf = torch.randn(sources, 3, 70, width, device="cuda").to(torch.bfloat16)
    elif layout == "uncollapsible":  # [S, 70, 3, D] viewed as [S, 3, 70, D]: no single row stride
        leaf = torch.randn(sources, 70, 3, width, device="cuda").to(torch.bfloat16).transpose(1, 2)
    elif layout == "feature-strided":  # [S, D, 210] transposed: rows are not unit-stride
        leaf = torch.randn(sources, width, 210, device="cuda").to(torch.bfloat16).transpose(1, 2)
    else:  # [S, D]: one token
        leaf = torch.randn(sources, width, device="cuda").to(torch.bfloat16)
    leaf.requires_grad_()
    query = (torch.randn(rank, device="cuda") / rank ** 0.5).to(torch.bfloat16).requires_grad_()
    upstream = torch.randn(leaf.shape[1:], device="cuda").to(torch.bfloat16)
    out = attnres(leaf, query)
    assert out.shape == leaf.shape[1:]
    assert all(type(fn).__name__ in ("AccumulateGrad", "NoneType") for fn, _ in out.grad_fn.next_functions), \
        f"expected the node alone, found {out.grad_fn.next_functions}"
    dv, dq = torch.autograd.grad(out, (leaf, query), upstream)
    assert dv.shape == leaf.shape

    from attnres import _ops  # noqa: F401  (registers the ops)
    flat = leaf.detach().reshape(sources, -1, width).contiguous()
    q = query.detach()
    saved = torch.ops.attnres_hip.packed_forward(flat, q, 2**-23, 1.0)
    grads = torch.ops.attnres_hip.packed_backward(flat, q, saved[0], saved[1], upstream.reshape(-1, width),
                                                  *saved[2:], 1.0)
    assert torch.equal(out.reshape(-1, width), saved[0]), "out differs from the ops"
    assert torch.equal(dv.reshape(sources, -1, width), grads[0]), "dv differs from the ops"
    assert torch.equal(dq, grads[1]), "dq differs from the ops"


@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("sources", [5, 9, 25])
def test_reads_without_gradients_store_no_saved_state(layout, sources):
    """With grad mode off (torch.no_grad, torch.inference_mode) or no input
    requiring grad, an eager read runs the forward alone: no autograd node,
    no refinement bytes and no saved state held after the call, and the
    output is the training forward's, bit for bit (the recompute, saved and
    token-block paths)."""
    torch.manual_seed(5)
    width, tokens = 2048, 300
    print(f"no-grad read {layout} S={sources}", flush=True)
    values = torch.randn(sources, 3, tokens // 3, width, device="cuda").to(torch.bfloat16)
    query = (torch.randn(width, device="cuda") / width ** 0.5).to(torch.bfloat16)

    def call(v, q):
        return attnres(v if layout == "packed" else list(v.unbind(0)), q)

    leaf = values.clone().requires_grad_()
    trained = call(leaf, query)
    assert trained.grad_fn is not None
    expected = trained.detach().clone()
    del trained, leaf
    torch.cuda.synchronize()
    out_bytes = expected.numel() * expected.element_size()
    for mode in ("no_grad", "inference_mode", "no input requires grad"):
        before = torch.cuda.memory_allocated()
        if mode == "no_grad":
            with torch.no_grad():
                out = call(values.clone().requires_grad_(), query)
        elif mode == "inference_mode":
            with torch.inference_mode():
                out = call(values, query)
        else:
            out = call(values, query)
        torch.cuda.synchronize()
        assert out.grad_fn is None, mode
        assert torch.equal(out, expected), f"{mode}: the output differs from the training forward's"
        held = torch.cuda.memory_allocated() - before
        assert held <= out_bytes + 512, f"{mode}: {held} bytes held after the call, the output is {out_bytes}"
        del out


@pytest.mark.parametrize("layout", ["packed", "list"])
def test_compiled_reads_without_gradients_call_the_forward_alone(layout, monkeypatch):
    """Under torch.compile a read that needs no gradient calls
    ``packed_forward_out`` / ``sources_forward_out`` (the output alone, no
    refinement bytes or saved state) instead of the saving forward op, and
    its output is the eager training forward's, bit for bit.  Both ops launch
    through ``*_forward_impl``; the calls it records name the op that ran
    (``save`` False and the state pooled for the forward alone)."""
    from attnres import _ops

    torch.manual_seed(6)
    sources, width = 25, 2048
    print(f"compiled no-grad read {layout}", flush=True)
    values = torch.randn(sources, 256, width, device="cuda").to(torch.bfloat16)
    query = (torch.randn(width, device="cuda") / width ** 0.5).to(torch.bfloat16)

    def read(v, q):
        return attnres(v if layout == "packed" else list(v.unbind(0)), q)

    expected = read(values.clone().requires_grad_(), query).detach()
    name = "packed_forward_impl" if layout == "packed" else "sources_forward_impl"
    impl = getattr(_ops, name)
    calls = []

    def recording(*args, **kwargs):
        calls.append((args[4], kwargs.get("pooled", args[5] if len(args) > 5 else False)))
        return impl(*args, **kwargs)

    monkeypatch.setattr(_ops, name, recording)
    torch._dynamo.reset()
    compiled = torch.compile(read, fullgraph=True, dynamic=False)
    with torch.no_grad():
        compiled(values, query)  # compile
        calls.clear()
        out = compiled(values, query)
    assert calls == [(False, True)], f"expected the forward alone, got (save, pooled) calls {calls}"
    assert torch.equal(out, expected), "the compiled no-grad output differs from the training forward's"
    torch._dynamo.reset()


def test_autograd_nodes_raise_the_library_errors():
    """The C++ nodes map a status the C ABI returns to the Python binding's
    exception classes (ValueError for argument errors) with the library's
    message.  `attnres` validates first, so these calls go to the nodes
    directly, with arguments the library rejects on the host before any
    launch: a rank above the width, and a NaN eps."""
    from attnres import _native

    nodes = _native.load_autograd()
    values = torch.randn(3, 8, 16, device="cuda").to(torch.bfloat16)
    query = torch.randn(17, device="cuda").to(torch.bfloat16)
    with pytest.raises(ValueError, match="attnres packed forward"):
        nodes.packed_read(values, query, 2**-23, 1.0)
    with pytest.raises(ValueError, match="attnres source-list forward"):
        nodes.sources_read(query, 2**-23, 1.0, list(values.unbind(0)))
    with pytest.raises(ValueError, match="attnres packed forward"):
        nodes.packed_read(values, query[:16], float("nan"), 1.0)


def _random_layout_cases(count=24, seed=20261203):
    """Seeded (S, batch shape, D, R, layout) draws over the envelope: one to
    three batch axes, widths from 8 to 4096 (aligned or not), any rank, and
    three memory layouts of the packed tensor."""
    import random

    rng = random.Random(seed)
    cases = []
    for _ in range(count):
        sources = rng.choice([1, 2, 5, 7, 9, 13, 16, 25, 30])
        width = rng.choice([8, 40, 200, 512, 1000, 1024, 2048, 3000, 4096])
        rank = rng.choice([width, max(1, width // 4), rng.randint(1, width)])
        batch = tuple(rng.randint(1, 40) for _ in range(rng.randint(1, 3)))
        layout = rng.choice(["contiguous", "batch-transposed", "feature-strided"])
        cases.append((sources, batch, width, rank, layout))
    return cases


@pytest.mark.parametrize("sources,batch,width,rank,layout", _random_layout_cases())
def test_eager_node_random_layouts_match_the_ops(sources, batch, width, rank, layout):
    """Random packed layouts through the eager node against the ops on the
    flattened contiguous values, bit for bit (out, dv, dq), and the forward
    without gradients against the training forward."""
    torch.manual_seed(sources * 1000 + width + rank)
    print(f"random layout S={sources} batch={batch} D={width} R={rank} {layout}", flush=True)
    if layout == "contiguous":
        base = torch.randn(sources, *batch, width, device="cuda").to(torch.bfloat16)
    elif layout == "batch-transposed" and len(batch) >= 2:
        base = torch.randn(sources, *batch[::-1], width, device="cuda").to(torch.bfloat16)
        base = base.permute(0, *range(len(batch), 0, -1), len(batch) + 1)
    elif layout == "feature-strided":
        base = torch.randn(sources, width, *batch, device="cuda").to(torch.bfloat16)
        base = base.permute(0, *range(2, len(batch) + 2), 1)
    else:  # a transposed batch needs two batch axes: a strided row selection instead
        base = torch.randn(sources, *batch[:-1], 2 * batch[-1], width, device="cuda").to(torch.bfloat16)
        base = base[..., ::2, :]
    assert base.shape == (sources, *batch, width)
    leaf = base.clone(memory_format=torch.preserve_format).requires_grad_() if layout == "contiguous" \
        else base.detach().requires_grad_()
    query = (torch.randn(rank, device="cuda") / rank ** 0.5).to(torch.bfloat16).requires_grad_()
    upstream = torch.randn(*batch, width, device="cuda").to(torch.bfloat16)
    out = attnres(leaf, query)
    dv, dq = torch.autograd.grad(out, (leaf, query), upstream)
    assert out.shape == (*batch, width) and dv.shape == leaf.shape

    from attnres import _ops  # noqa: F401  (registers the ops)
    flat = leaf.detach().reshape(sources, -1, width).contiguous()
    q = query.detach()
    saved = torch.ops.attnres_hip.packed_forward(flat, q, 2**-23, 1.0)
    grads = torch.ops.attnres_hip.packed_backward(flat, q, saved[0], saved[1], upstream.reshape(-1, width),
                                                  *saved[2:], 1.0)
    assert torch.equal(out.reshape(-1, width), saved[0]), "out differs from the ops"
    assert torch.equal(dv.reshape(sources, -1, width), grads[0]), "dv differs from the ops"
    assert torch.equal(dq, grads[1]), "dq differs from the ops"
    with torch.no_grad():
        assert torch.equal(attnres(leaf, query), out.detach()), "the no-grad forward differs"


@pytest.mark.parametrize("sources,batch,width,rank,layout", _random_layout_cases()[:12])
def test_eager_list_node_random_layouts_match_the_ops(sources, batch, width, rank, layout):
    """The same random layouts as a source list (each source a view of the
    packed tensor, addressable or not): the eager list node against the list
    ops, bit for bit, and the forward without gradients against the training
    forward."""
    torch.manual_seed(sources * 1000 + width + rank + 1)
    print(f"random list layout S={sources} batch={batch} D={width} R={rank} {layout}", flush=True)
    if layout == "feature-strided":
        packed = torch.randn(sources, width, *batch, device="cuda").to(torch.bfloat16)
        packed = packed.permute(0, *range(2, len(batch) + 2), 1)
    elif layout == "batch-transposed" and len(batch) >= 2:
        packed = torch.randn(sources, *batch[::-1], width, device="cuda").to(torch.bfloat16)
        packed = packed.permute(0, *range(len(batch), 0, -1), len(batch) + 1)
    else:
        packed = torch.randn(sources, *batch, width, device="cuda").to(torch.bfloat16)
    leaves = [packed[s].detach().requires_grad_() for s in range(sources)]
    query = (torch.randn(rank, device="cuda") / rank ** 0.5).to(torch.bfloat16).requires_grad_()
    upstream = torch.randn(*batch, width, device="cuda").to(torch.bfloat16)
    out = attnres(leaves, query)
    grads = torch.autograd.grad(out, (*leaves, query), upstream)

    from attnres import _ops  # noqa: F401  (registers the ops)
    listed = [leaf.detach() for leaf in leaves]
    q = query.detach()
    saved = torch.ops.attnres_hip.sources_forward(listed, q, 2**-23, 1.0)
    expected = torch.ops.attnres_hip.sources_backward(listed, q, saved[0], saved[1], upstream, *saved[2:], 1.0)
    assert torch.equal(out, saved[0]), "out differs from the list ops"
    for s in range(sources):
        assert torch.equal(grads[s], expected[s]), f"dv of source {s} differs from the list ops"
    assert torch.equal(grads[-1], expected[-1]), "dq differs from the list ops"
    with torch.no_grad():
        assert torch.equal(attnres(leaves, query), out.detach()), "the no-grad forward differs"


@pytest.mark.parametrize("sources", [5, 9, 25])
@pytest.mark.parametrize("use_reentrant", [True, False])
def test_checkpointed_read_matches_the_plain_read(sources, use_reentrant):
    """torch.utils.checkpoint around a read: the reentrant form runs the first
    forward under no_grad (the forward alone) and recomputes it with
    gradients in the backward; both forms give the plain read's output and
    gradients, bit for bit."""
    from torch.utils.checkpoint import checkpoint

    torch.manual_seed(17 + sources)
    print(f"checkpointed read S={sources} reentrant={use_reentrant}", flush=True)
    values = torch.randn(sources, 2, 150, 2048, device="cuda").to(torch.bfloat16)
    query = (torch.randn(2048, device="cuda") / 2048 ** 0.5).to(torch.bfloat16)
    upstream = torch.randn(2, 150, 2048, device="cuda").to(torch.bfloat16)

    def run(wrapped):
        leaf, q = values.clone().requires_grad_(), query.clone().requires_grad_()
        out = checkpoint(attnres, leaf, q, use_reentrant=use_reentrant) if wrapped else attnres(leaf, q)
        out.backward(upstream)
        return out.detach(), leaf.grad, q.grad

    for name, a, b in zip(("out", "dv", "dq"), run(False), run(True)):
        assert torch.equal(a, b), f"{name} differs under checkpointing"


@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("sources", [5, 9, 25])
def test_frozen_values_give_the_same_query_gradient(layout, sources):
    """Values that do not require grad (frozen sources) with a trainable
    query: the node returns no value gradient and the query gradient of the
    read where both require grad, bit for bit."""
    torch.manual_seed(23 + sources)
    print(f"frozen values {layout} S={sources}", flush=True)
    values = torch.randn(sources, 300, 2048, device="cuda").to(torch.bfloat16)
    query = (torch.randn(2048, device="cuda") / 2048 ** 0.5).to(torch.bfloat16)
    upstream = torch.randn(300, 2048, device="cuda").to(torch.bfloat16)

    def read(v, q):
        return attnres(v if layout == "packed" else list(v.unbind(0)), q)

    both = values.clone().requires_grad_()
    q_both = query.clone().requires_grad_()
    out = read(both, q_both)
    _, dq = torch.autograd.grad(out, (both, q_both), upstream)
    q_only = query.clone().requires_grad_()
    frozen = values.clone()
    out_frozen = read(frozen, q_only)
    (dq_frozen,) = torch.autograd.grad(out_frozen, (q_only,), upstream)
    assert torch.equal(out_frozen, out)
    assert torch.equal(dq_frozen, dq)
    assert frozen.grad is None
