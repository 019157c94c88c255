"""The backward entry point that allocates nothing
(`attnres_hip_packed_backward_noalloc`) against the workspace entry point
(`attnres_hip_packed_backward`), called through the C ABI.

Its dq partial rows live in the library's own 4 MiB device array, shared by
every call on a GPU, so two calls run back to back, the second on a smaller
input: stale rows of the first must not reach the second.  dv must be the
same bits (the grid never changes a token's arithmetic); dq must be the same
bits when the array holds every partial row of the grid the workspace entry
point launched, and within one BF16 ulp (floor 2^-16 of the largest
component) when the grid is cut to fit it.  The launched grid is read off the
workspace: it is filled with NaN first, and the launch writes exactly its
leading partial rows.  The saved-refinement backward (streaming and
token-block kernels), the recompute backward (S <= 6) and the key-resident
backward (out_refine = NULL for 7..16 sources of a 512/1024 key) are covered;
the c2-sized pair launches more token-block workgroups (two per CU) than the
array holds rows for, so its grid is really cut.
"""

from __future__ import annotations

import math

import pytest
import torch

from attnres import _native, _ops
from helpers import ulp_error

pytestmark = pytest.mark.gpu

# (S, N, D, R): the first call of each pair is the larger one
PAIRS = [
    ((25, 4096, 2048, 2048), (9, 300, 1024, 256)),     # saved path, then a smaller saved read
    ((12, 2048, 8192, 8192), (5, 64, 2048, 2048)),     # capped grid (R = 8192), then the recompute path
    ((4, 3000, 4096, 1024), (2, 17, 96, 40)),          # recompute (wide groups), then a tiny read
    ((25, 16384, 2048, 2048), (13, 4096, 2048, 2048)),  # c2: the token-block grid cut to 511 rows, then uncut
    ((16, 8192, 4096, 1024), (9, 999, 2048, 512)),     # key-resident backward, both widths
    ((12, 16384, 2048, 2048), (7, 999, 2048, 2048)),   # key-resident, the whole row as key (grid cut, then not)
]
CUT_EXPECTED = {(25, 16384, 2048, 2048)}  # shapes whose launch must exceed the array's rows on an MI355X


def _inputs(shape, seed):
    sources, tokens, width, rank = shape
    generator = torch.Generator(device="cuda").manual_seed(seed)
    values = (torch.randn(sources, tokens, width, generator=generator, device="cuda")
              * (torch.rand(sources, 1, 1, generator=generator, device="cuda") * 3.5 + 0.5)).to(torch.bfloat16)
    query = (torch.randn(rank, generator=generator, device="cuda") / math.sqrt(rank)).to(torch.bfloat16)
    grad_out = torch.randn(tokens, width, generator=generator, device="cuda").to(torch.bfloat16)
    return values, query, grad_out


def _both(shape, seed):
    lib = _native.load()
    values, query, grad_out = _inputs(shape, seed)
    sources, tokens, width, rank = shape
    out, refine, logit, inv_rms, stats = _ops.packed_forward_impl(values, query, 2**-23, 1.0,
                                                                   _ops.saves_refinement(sources, width, rank))
    saved = refine.numel() > 0
    stream = torch.cuda.current_stream().cuda_stream
    common = (values.data_ptr(), values.stride(0), values.stride(1), sources, tokens, width, query.data_ptr(), rank,
              1.0, out.data_ptr() if saved else None, refine.data_ptr() if saved else None, grad_out.data_ptr(),
              logit.data_ptr(), inv_rms.data_ptr(), stats.data_ptr())
    dv_ref = torch.empty_like(values)
    dq_ref = torch.empty(rank, device="cuda", dtype=torch.bfloat16)
    workspace = torch.full((lib.attnres_hip_dq_workspace_elems(tokens, width, rank),), float("nan"), device="cuda")
    _native.check(lib.attnres_hip_packed_backward(*common, dv_ref.data_ptr(), dq_ref.data_ptr(),
                                                  workspace.data_ptr(), workspace.numel(), stream),
                  "workspace backward")
    dv = torch.full_like(values, float("nan"))
    dq = torch.full((rank,), float("nan"), device="cuda", dtype=torch.bfloat16)
    _native.check(lib.attnres_hip_packed_backward_noalloc(*common, dv.data_ptr(), dq.data_ptr(), stream),
                  "no-alloc backward")
    torch.cuda.synchronize()
    partial_rows = workspace.numel() // rank - 1
    written = torch.isfinite(workspace[:partial_rows * rank].view(partial_rows, rank)).all(dim=1)
    launched = int(written.to(torch.int32).argmin()) if not bool(written.all()) else partial_rows
    assert bool(written[:launched].all()) and not bool(written[launched:].any()), "partial rows not a prefix"
    return (dv, dq), (dv_ref, dq_ref), launched


@pytest.mark.parametrize("pair", PAIRS, ids=lambda p: f"{p[0]}-then-{p[1]}")
def test_no_alloc_backward_matches_the_workspace_entry_point(pair):
    for index, shape in enumerate(pair):
        print(f"no-alloc backward call {index}: S,N,D,R={shape}", flush=True)
        (dv, dq), (dv_ref, dq_ref), launched = _both(shape, seed=1000 + index + shape[0])
        assert torch.equal(dv, dv_ref), f"dv differs for {shape}"
        rank = shape[3]
        fits = (launched + 1) * rank <= 2**20  # partial rows plus the total in the library's array
        print(f"  launched {launched} workgroups; {'fits' if fits else 'cut to fit'}", flush=True)
        if shape in CUT_EXPECTED:
            assert not fits, f"{shape}: the launch ({launched} workgroups) was expected to exceed the array"
        if fits:  # the same grid: same sums, same order
            assert torch.equal(dq, dq_ref), f"dq differs for {shape}"
        else:
            assert ulp_error(dq, dq_ref.double()) <= 1.0, f"dq beyond one ulp for {shape}"


def test_no_alloc_backward_rejects_bad_arguments_before_launching():
    lib = _native.load()
    status = lib.attnres_hip_packed_backward_noalloc(None, 0, 0, 2, 4, 64, None, 65, 1.0, None, None, None, None,
                                                     None, None, None, None, None)
    assert status == _native.ERR_SHAPE
    assert b"rank" in lib.attnres_hip_last_error()
