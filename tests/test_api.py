"""Public API behaviour on CPU: signature, validation order, error classes
and message substrings, container handling and the ops' fake kernels.

Mirrors the reference's tests/test_api.py (CPU part) and the fake-kernel
checks of tests/test_softmax_stats.py:18-25 and
tests/test_fla_production_autotune.py:65-130.  No GPU and no kernel launch:
device rejection happens before the native library is loaded.
"""

from __future__ import annotations

import inspect
import sys

import pytest
import torch

import attnres as package
from attnres import LearnedQuery, attnres


def test_public_surface():
    # the reference's surface plus SharedSources (an addition with no reference counterpart)
    assert set(package.__all__) == {"attnres", "LearnedQuery", "__version__", "SharedSources", "SourceBank"}
    parameters = inspect.signature(attnres).parameters
    assert list(parameters) == ["values", "query", "eps", "scale"]
    assert parameters["eps"].kind is inspect.Parameter.KEYWORD_ONLY
    assert parameters["eps"].default == 2**-23
    assert parameters["scale"].default == 1.0
    assert "keys" not in parameters
    with pytest.raises(TypeError, match="keys"):
        attnres(torch.randn(3, 8, dtype=torch.bfloat16), torch.randn(2, dtype=torch.bfloat16),
                keys=torch.randn(3, 2))


@pytest.mark.parametrize("container", [list, tuple])
def test_cpu_source_list_is_rejected_without_loading_the_native_library(container, monkeypatch):
    for name in [n for n in sys.modules if n.startswith("attnres._ops")]:
        monkeypatch.delitem(sys.modules, name)
    from attnres import _native
    monkeypatch.setattr(_native, "_library", None)
    values = container(torch.randn(2, 8, dtype=torch.bfloat16, requires_grad=True) for _ in range(3))
    query = torch.randn(4, dtype=torch.bfloat16, requires_grad=True)
    with pytest.raises(RuntimeError, match="CUDA"):
        attnres(values, query)
    assert _native._library is None


def test_cpu_packed_and_fp32_inputs_are_rejected_explicitly():
    values = torch.randn(5, 2, 13, dtype=torch.bfloat16)
    query = torch.randn(4, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="CUDA"):
        attnres(values, query)
    with pytest.raises(TypeError, match="BF16"):
        attnres(values.float(), query)
    with pytest.raises(TypeError, match="BF16"):
        attnres(values, query.float())


def test_numeric_options_are_validated_before_the_device():
    values = torch.randn(4, 3, 9, dtype=torch.bfloat16)
    query = torch.randn(3, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="eps"):
        attnres(values, query, eps=0.0)
    with pytest.raises(RuntimeError, match="CUDA"):
        attnres(values, query, eps=2**-20, scale=0.75)


@pytest.mark.parametrize("values,query,error", [
    (torch.randn(4), torch.randn(2), ValueError),
    (torch.randn(4, 8, dtype=torch.bfloat16), torch.randn(2, 1, dtype=torch.bfloat16), ValueError),
    (torch.randn(4, 8, dtype=torch.float16), torch.randn(2), TypeError),
    (torch.randn(4, 8, dtype=torch.bfloat16), torch.randn(2, dtype=torch.float16), TypeError),
    (torch.randn(130, 8, dtype=torch.bfloat16), torch.randn(2, dtype=torch.bfloat16), ValueError),
    (torch.randn(3, 8193, dtype=torch.bfloat16), torch.randn(2, dtype=torch.bfloat16), ValueError),
    (torch.randn(3, 8, dtype=torch.bfloat16), torch.randn(9, dtype=torch.bfloat16), ValueError),
    (torch.randn(3, 0, 8, dtype=torch.bfloat16), torch.randn(2, dtype=torch.bfloat16), ValueError),
])
def test_packed_rejects_invalid_shapes_and_storage(values, query, error):
    with pytest.raises(error):
        attnres(values, query)


@pytest.mark.parametrize("kwargs", [{"eps": 0.0}, {"eps": -1.0}, {"eps": float("nan")},
                                    {"scale": float("inf")}, {"scale": float("nan")}])
@pytest.mark.parametrize("sequence", [False, True])
def test_invalid_numeric_options(kwargs, sequence):
    values = torch.randn(3, 8, dtype=torch.bfloat16)
    query = torch.randn(4, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        attnres(list(values.unbind(0)) if sequence else values, query, **kwargs)


@pytest.mark.parametrize("values,query,error", [
    ([], torch.randn(2, dtype=torch.bfloat16), ValueError),
    ([torch.randn(2, 5, dtype=torch.bfloat16), torch.randn(3, 5, dtype=torch.bfloat16)],
     torch.randn(2, dtype=torch.bfloat16), ValueError),
    ([torch.randn(2, 5, dtype=torch.bfloat16), 3], torch.randn(2, dtype=torch.bfloat16), TypeError),
    ([torch.randn(2, 5, dtype=torch.bfloat16)], torch.randn(6, dtype=torch.bfloat16), ValueError),
    ({"source": torch.randn(2, 5, dtype=torch.bfloat16)}, torch.randn(2, dtype=torch.bfloat16), TypeError),
    ([torch.randn(2, 5, dtype=torch.bfloat16)], torch.randn(2, device="meta", dtype=torch.bfloat16), TypeError),
    ([torch.randn(2, 5, dtype=torch.bfloat16)] * 130, torch.randn(2, dtype=torch.bfloat16), ValueError),
    ([torch.randn(2, 5, dtype=torch.bfloat16), torch.randn(2, 5)], torch.randn(2, dtype=torch.bfloat16), TypeError),
    ([torch.randn(2, 5)], torch.randn(2, dtype=torch.bfloat16), TypeError),
    ([torch.randn((), dtype=torch.bfloat16)], torch.randn(1, dtype=torch.bfloat16), ValueError),
])
def test_source_containers_reject_malformed_inputs(values, query, error):
    with pytest.raises(error):
        attnres(values, query)


@pytest.mark.parametrize("container", [None, list, tuple])
@pytest.mark.parametrize("query", [None, 2, [1.0, 2.0]])
def test_query_type_errors_are_consistent_across_containers(container, query):
    values = torch.randn(3, 8, dtype=torch.bfloat16)
    with pytest.raises(TypeError, match="query"):
        attnres(container(values.unbind(0)) if container else values, query)


@pytest.mark.parametrize("container", [None, list, tuple])
@pytest.mark.parametrize("name", ["eps", "scale"])
@pytest.mark.parametrize("value", [True, "0.5", torch.tensor(0.5)])
def test_scalar_type_errors_are_consistent_across_containers(container, name, value):
    values = torch.randn(3, 8, dtype=torch.bfloat16)
    query = torch.randn(2, dtype=torch.bfloat16)
    with pytest.raises(TypeError):
        attnres(container(values.unbind(0)) if container else values, query, **{name: value})


@pytest.mark.parametrize("container", [None, list, tuple])
def test_real_integer_and_numpy_scalars_are_accepted(container):
    np = pytest.importorskip("numpy")
    values = torch.randn(3, 8, dtype=torch.bfloat16)
    query = torch.randn(2, dtype=torch.bfloat16)
    source = container(values.unbind(0)) if container else values
    for eps, scale in ((1, 2), (np.float32(1e-3), np.int64(3))):
        with pytest.raises(RuntimeError, match="CUDA"):  # validation passed; only the device fails
            attnres(source, query, eps=eps, scale=scale)


def test_learned_query_parameter():
    torch.manual_seed(0)
    module = LearnedQuery(96, init_std=0.02)
    query = module()
    assert query.dtype == torch.bfloat16 and query.shape == (96,)
    assert isinstance(module.query, torch.nn.Parameter)
    assert 0.005 < float(query.detach().float().std()) < 0.05
    for bad, error in ((0, ValueError), (True, TypeError), (2.5, TypeError)):
        with pytest.raises(error):
            LearnedQuery(bad)
    with pytest.raises(ValueError):
        LearnedQuery(4, init_std=0.0)


# ---------------------------------------------------------------- fake ops

def _ops():
    from attnres import _ops
    return _ops


def test_packed_fake_kernels_give_shapes_and_dtypes():
    ops = _ops()
    values = torch.empty(8, 7, 48, dtype=torch.bfloat16, device="meta")
    query = torch.empty(16, dtype=torch.bfloat16, device="meta")
    out, refine, logit, inv_rms, stats = ops.packed_forward(values, query, 2**-23, 1.0)
    assert out.shape == (7, 48) and out.dtype == torch.bfloat16
    assert refine.shape == (7, 48) and refine.dtype == torch.int8
    assert logit.shape == inv_rms.shape == (7, 8) and logit.dtype == torch.float32
    assert stats.shape == (2, 7) and stats.dtype == torch.float32
    grad_values, grad_query = ops.packed_backward(values, query, out, refine, out, logit, inv_rms,
                                                  stats, 1.0)
    assert grad_values.shape == values.shape and grad_values.dtype == torch.bfloat16
    assert grad_query.shape == query.shape and grad_query.dtype == torch.bfloat16


@pytest.mark.parametrize("count", [1, 2, 6, 7, 9])
def test_source_fake_kernels_give_one_gradient_per_position(count):
    ops = _ops()
    sources = [torch.empty(2, 3, 64, dtype=torch.bfloat16, device="meta")] * count
    query = torch.empty(16, dtype=torch.bfloat16, device="meta")
    out, refine, logit, inv_rms, stats = ops.sources_forward(sources, query, 2**-23, 1.0)
    assert out.shape == (2, 3, 64) and refine.shape == ((6 if count > 6 else 0), 64)
    assert logit.shape == (6, count) and stats.shape == (2, 6) and stats.dtype == torch.float32
    grads = ops.sources_backward(sources, query, out, refine, out, logit, inv_rms, stats, 1.0)
    assert len(grads) == count + 1
    assert all(g.shape == (2, 3, 64) for g in grads[:count]) and grads[count].shape == (16,)


@pytest.mark.parametrize("count", [1, 6, 7, 9])
@pytest.mark.parametrize("layout", ["packed", "list"])
def test_saved_state_follows_the_recompute_policy(count, layout):
    """Reads of at most 6 sources keep neither the output nor its refinement
    for the backward; larger reads keep both (1 + 2 bytes per element besides
    the inputs and the per-token statistics).  Reference policy:
    fla_full_sources.py:146-161."""
    ops = _ops()
    tokens, width = 6, 64
    values = torch.empty(count, tokens, width, dtype=torch.bfloat16, device="meta", requires_grad=True)
    query = torch.empty(16, dtype=torch.bfloat16, device="meta", requires_grad=True)
    saved = []
    inputs = [values, query] if layout == "packed" else [*values.unbind(0), query]
    with torch.autograd.graph.saved_tensors_hooks(lambda t: saved.append(t) or t, lambda t: t):
        if layout == "packed":
            out, refine, *_ = ops.packed_forward(values, query, 2**-23, 1.0)
        else:
            out, refine, *_ = ops.sources_forward(inputs[:-1], query, 2**-23, 1.0)
    saves = count > 6
    assert refine.shape == ((tokens if saves else 0), width)
    state = [t for t in saved if not any(t is x for x in inputs)]
    row_state = [t for t in state if t.dim() == 2 and t.shape[-1] == width]
    assert sum(t.numel() * t.element_size() for t in row_state) == (3 * tokens * width if saves else 0)


def test_row_layout_flattening():
    """Rows of [..., D] flatten to one row stride when the batch axes are
    affine (size-1 axes are free), else the tensor is copied (reference
    src/attnres/_kernels/fla_full_sources.py:164-178)."""
    ops = _ops()
    base = torch.empty(4, 6, 10)
    assert ops.row_stride(base) == 10
    assert ops.row_stride(base[:, :, :7]) == 10          # padded rows stay addressable
    assert ops.row_stride(base.transpose(0, 1)) is None   # batch axes out of order
    assert ops.row_stride(base[..., ::2]) is None         # features not unit-stride
    assert ops.row_stride(torch.empty(1, 1, 9)) == 0      # single row
    single = torch.empty(8, 1, 5).as_strided((8, 1, 5), (5, 999, 1))
    assert ops.row_stride(single) == 5
    tensor, stride = ops.prepare_rows(base.transpose(0, 1))
    assert tensor.is_contiguous() and stride == 10


def test_shared_sources_rejects_bad_inputs_on_the_host():
    from attnres import SharedSources

    cpu = [torch.zeros(4, 8, dtype=torch.bfloat16) for _ in range(2)]
    with pytest.raises(RuntimeError, match="CUDA"):
        SharedSources(cpu)
    with pytest.raises(TypeError):
        SharedSources([])
    with pytest.raises(TypeError):
        SharedSources(torch.zeros(2, 4, 8, dtype=torch.bfloat16))
    with pytest.raises(TypeError, match="BF16"):
        SharedSources([torch.zeros(4, 8), torch.zeros(4, 8)])
    with pytest.raises(ValueError):
        SharedSources([torch.zeros(4, 8, dtype=torch.bfloat16), torch.zeros(4, 9, dtype=torch.bfloat16)])


def test_eager_path_choice():
    """Plain tensors and parameters take the direct autograd path; a compiler's
    fake tensors take the registered ops (their fake kernels give the shapes)."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    from attnres import _ops

    plain = torch.empty(3)
    assert _ops._eager(plain, torch.nn.Parameter(torch.empty(2)))
    with FakeTensorMode():
        fake = torch.empty(3)
    assert not _ops._eager(plain, fake)


@pytest.mark.parametrize("save", [False, True])
@pytest.mark.parametrize("tokens,sources,width", [(1, 1, 1), (7, 9, 33), (300, 25, 2048), (5, 129, 8192)])
def test_pooled_saved_state_layout(tokens, sources, width, save):
    """The eager read's C++ autograd node keeps its saved state in one byte
    pool at the offsets of its `pool_layout`; the ops' pooled views
    (`_saved_state(pooled=True)`, used by the shared-source reads) follow the
    Python `_pool_layout`.  Both must state the same layout: the refinement at
    byte 0, the FP32 statistics from a 16-byte aligned offset, no overlap, all
    inside the pool."""
    ops = _ops()
    from attnres import _native

    head, block, size = ops._pool_layout(tokens, sources, width, save)
    assert _native.load_autograd().pool_layout(tokens, sources, width, save) == (head, block, size)
    refine, logit, inv_rms, stats = ops._saved_state(tokens, sources, width, save, "cpu", pooled=True)
    base = refine.untyped_storage().data_ptr()
    assert refine.untyped_storage().nbytes() == size
    assert refine.shape == ((tokens if save else 0), width) and logit.shape == inv_rms.shape == (tokens, sources)
    assert stats.shape == (2, tokens)
    assert (logit.data_ptr(), inv_rms.data_ptr(), stats.data_ptr()) == (base + head, base + head + 4 * block,
                                                                        base + head + 8 * block)
    if save:
        assert refine.data_ptr() == base
    spans = [(t.data_ptr(), t.data_ptr() + t.numel() * t.element_size())
             for t in (refine, logit, inv_rms, stats) if t.numel()]  # an empty view reports address 0
    assert all(base <= lo <= hi <= base + size for lo, hi in spans)
    assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:]))
    assert head % 16 == 0 and head >= (tokens * width if save else 0)
