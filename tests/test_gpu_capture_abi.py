"""Graph capture at the C ABI: the library's entry points recorded into a HIP
graph with the runtime's stream-capture API and replayed.

The C ABI promises that a call only enqueues kernels on the caller's stream
(no allocation, synchronisation, memset or host read of device memory), which
is what stream capture needs.  Here every buffer is allocated beforehand, the
forward and backward calls of both layouts are captured on a side stream
(`hipStreamBeginCapture` / `hipStreamEndCapture`, relaxed mode), the graph is
instantiated and replayed several times with the outputs cleared between
replays, and every replay must reproduce the eager calls bit for bit.  The
runtime functions are bound from the HIP runtime the process already loaded
(the one torch uses), so both share one runtime instance.
"""

from __future__ import annotations

import ctypes
import math
import re

import pytest
import torch

from attnres import _native

pytestmark = pytest.mark.gpu

_CAPTURE_MODE_RELAXED = 2


def _hip_runtime() -> ctypes.CDLL:
    loaded = sorted(set(re.findall(r"\S*libamdhip64\.so\S*", open("/proc/self/maps").read())))
    assert loaded, "the HIP runtime is not loaded in this process"
    hip = ctypes.CDLL(loaded[0])
    vp, i = ctypes.c_void_p, ctypes.c_int
    for name, args in {
        "hipStreamBeginCapture": [vp, i],
        "hipStreamEndCapture": [vp, ctypes.POINTER(vp)],
        "hipGraphInstantiate": [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t],
        "hipGraphLaunch": [vp, vp],
        "hipGraphExecDestroy": [vp],
        "hipGraphDestroy": [vp],
        "hipStreamSynchronize": [vp],
    }.items():
        fn = getattr(hip, name)
        fn.restype, fn.argtypes = i, args
    return hip


class _Buffers:
    """Inputs, outputs and workspace of one read (packed or list)."""

    def __init__(self, layout: str, sources=5, tokens=515, width=1024, rank=384, seed=7):
        torch.manual_seed(seed)
        dev = "cuda"
        self.layout, self.S, self.N, self.D, self.R = layout, sources, tokens, width, rank
        self.values = torch.randn(sources, tokens, width, device=dev).to(torch.bfloat16)
        self.query = (torch.randn(rank, device=dev) / math.sqrt(rank)).to(torch.bfloat16)
        self.grad_out = torch.randn(tokens, width, device=dev).to(torch.bfloat16)
        self.out = torch.empty(tokens, width, device=dev, dtype=torch.bfloat16)
        self.refine = torch.empty(tokens, width, device=dev, dtype=torch.int8)
        self.logit = torch.empty(tokens, sources, device=dev)
        self.inv_rms = torch.empty(tokens, sources, device=dev)
        self.stats = torch.empty(2, tokens, device=dev)
        self.dv = torch.empty(sources, tokens, width, device=dev, dtype=torch.bfloat16)
        self.dq = torch.empty(rank, device=dev, dtype=torch.bfloat16)
        lib = _native.load()
        self.ws = torch.empty(lib.attnres_hip_dq_workspace_elems(tokens, width, rank), device=dev)
        rows = [self.values[s].data_ptr() for s in range(sources)]
        self.src_ptrs = (ctypes.c_void_p * sources)(*rows)
        self.src_strides = (ctypes.c_int64 * sources)(*([width] * sources))
        self.grad_ptrs = (ctypes.c_void_p * sources)(*[self.dv[s].data_ptr() for s in range(sources)])

    def outputs(self):
        return (self.out, self.refine, self.logit, self.inv_rms, self.stats, self.dv, self.dq)

    def enqueue(self, stream: int) -> None:
        lib = _native.load()
        S, N, D, R = self.S, self.N, self.D, self.R
        if self.layout == "packed":
            st = lib.attnres_hip_packed_forward(
                self.values.data_ptr(), N * D, D, S, N, D, self.query.data_ptr(), R, 2.0**-23, 1.0,
                self.out.data_ptr(), self.refine.data_ptr(), self.logit.data_ptr(), self.inv_rms.data_ptr(),
                self.stats.data_ptr(), stream)
            assert st == 0, lib.attnres_hip_last_error()
            st = lib.attnres_hip_packed_backward(
                self.values.data_ptr(), N * D, D, S, N, D, self.query.data_ptr(), R, 1.0, self.out.data_ptr(),
                self.refine.data_ptr(), self.grad_out.data_ptr(), self.logit.data_ptr(), self.inv_rms.data_ptr(),
                self.stats.data_ptr(), self.dv.data_ptr(), self.dq.data_ptr(), self.ws.data_ptr(),
                self.ws.numel(), stream)
        else:
            st = lib.attnres_hip_sources_forward(
                self.src_ptrs, self.src_strides, S, N, D, self.query.data_ptr(), R, 2.0**-23, 1.0,
                self.out.data_ptr(), self.refine.data_ptr(), self.logit.data_ptr(), self.inv_rms.data_ptr(),
                self.stats.data_ptr(), stream)
            assert st == 0, lib.attnres_hip_last_error()
            st = lib.attnres_hip_sources_backward(
                self.src_ptrs, self.src_strides, S, N, D, self.query.data_ptr(), R, 1.0, self.out.data_ptr(),
                self.refine.data_ptr(), self.grad_out.data_ptr(), self.logit.data_ptr(), self.inv_rms.data_ptr(),
                self.stats.data_ptr(), self.grad_ptrs, self.dq.data_ptr(), self.ws.data_ptr(), self.ws.numel(),
                stream)
        assert st == 0, lib.attnres_hip_last_error()


@pytest.mark.parametrize("layout", ["packed", "list"])
def test_abi_calls_replay_from_a_hip_graph(layout):
    hip = _hip_runtime()
    buffers = _Buffers(layout)
    side = torch.cuda.Stream()
    handle = side.cuda_stream
    print(f"abi capture layout={layout}", flush=True)
    with torch.cuda.stream(side):
        buffers.enqueue(handle)  # eager reference (also warms the occupancy caches)
    torch.cuda.synchronize()
    eager = [t.clone() for t in buffers.outputs()]
    torch.cuda.synchronize()  # the clones (default stream) finish before the replays zero the outputs (side stream)

    graph, exec_ = ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipStreamBeginCapture(handle, _CAPTURE_MODE_RELAXED) == 0
    buffers.enqueue(handle)
    assert hip.hipStreamEndCapture(handle, ctypes.byref(graph)) == 0
    try:
        assert hip.hipGraphInstantiate(ctypes.byref(exec_), graph, None, None, 0) == 0
        for replay in range(3):
            with torch.cuda.stream(side):
                for t in buffers.outputs():
                    t.zero_()
            assert hip.hipGraphLaunch(exec_, handle) == 0
            assert hip.hipStreamSynchronize(handle) == 0
            for t, e in zip(buffers.outputs(), eager):
                assert torch.equal(t, e), f"replay {replay}"
    finally:
        if exec_.value:
            hip.hipGraphExecDestroy(exec_)
        if graph.value:
            hip.hipGraphDestroy(graph)


@pytest.mark.parametrize("shape", [(25, 4096, 2048, 2048), (5, 515, 1024, 384)], ids=lambda s: "x".join(map(str, s)))
def test_no_alloc_backward_replays_from_a_hip_graph(shape):
    """The no-allocation backward under stream capture: its first call on the
    device (which looks up the library's scratch array) is made eagerly, then
    a call is captured and the graph replayed on changed upstream gradients;
    every replay must equal an eager call on the same inputs bit for bit.
    The saved-refinement path (S = 25) and the recompute path (S = 5)."""
    hip = _hip_runtime()
    lib = _native.load()
    sources, tokens, width, rank = shape
    torch.manual_seed(11)
    dev = "cuda"
    values = torch.randn(sources, tokens, width, device=dev).to(torch.bfloat16)
    query = (torch.randn(rank, device=dev) / math.sqrt(rank)).to(torch.bfloat16)
    grad_out = torch.randn(tokens, width, device=dev).to(torch.bfloat16)
    from attnres import _ops

    saved = _ops.saves_refinement(sources, width, rank)
    out, refine, logit, inv_rms, stats = _ops.packed_forward_impl(values, query, 2**-23, 1.0, saved)
    dv = torch.empty_like(values)
    dq = torch.empty(rank, device=dev, dtype=torch.bfloat16)
    side = torch.cuda.Stream()
    handle = side.cuda_stream

    def call():
        st = lib.attnres_hip_packed_backward_noalloc(
            values.data_ptr(), tokens * width, width, sources, tokens, width, query.data_ptr(), rank, 1.0,
            out.data_ptr() if saved else None, refine.data_ptr() if saved else None, grad_out.data_ptr(),
            logit.data_ptr(), inv_rms.data_ptr(), stats.data_ptr(), dv.data_ptr(), dq.data_ptr(), handle)
        assert st == 0, lib.attnres_hip_last_error()

    print(f"no-alloc capture S,N,D,R={shape}", flush=True)
    torch.cuda.synchronize()
    call()  # first call on the device, outside capture
    assert hip.hipStreamSynchronize(handle) == 0
    graph, exec_ = ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipStreamBeginCapture(handle, _CAPTURE_MODE_RELAXED) == 0
    call()
    assert hip.hipStreamEndCapture(handle, ctypes.byref(graph)) == 0
    try:
        assert hip.hipGraphInstantiate(ctypes.byref(exec_), graph, None, None, 0) == 0
        for replay in range(3):
            with torch.cuda.stream(side):
                grad_out.copy_(torch.randn(tokens, width, device=dev).to(torch.bfloat16))
            call()  # eager on the new inputs
            with torch.cuda.stream(side):  # snapshot and clear in stream order
                eager = (dv.clone(), dq.clone())
                dv.zero_()
                dq.zero_()
            assert hip.hipGraphLaunch(exec_, handle) == 0
            assert hip.hipStreamSynchronize(handle) == 0
            assert torch.equal(dv, eager[0]) and torch.equal(dq, eager[1]), f"replay {replay}"
    finally:
        if exec_.value:
            hip.hipGraphExecDestroy(exec_)
        if graph.value:
            hip.hipGraphDestroy(graph)
