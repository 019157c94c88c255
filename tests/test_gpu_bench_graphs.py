"""bench.py's graph-replay boundary (the C-ABI read captured into HIP graphs
and replayed) on small cases: the packed form the c2/c3 lines use, the
list form of the c4 line (three reads of one source list, one query each)
and the whole-step graph of the c5 sweep (the reads of S = 1..n in one
graph).
The replayed calls must succeed and every part must carry ordered
quartiles; the numerics of captured reads are covered by test_gpu_graphs.
"""

from __future__ import annotations

import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402

pytestmark = pytest.mark.gpu


def _check(record: dict) -> None:
    for part in ("forward", "backward", "read"):
        r = record[part]
        assert 0 < r["us_best"] <= r["us_q1"] <= r["us_median"] <= r["us_q3"], (part, r)
        assert r["TB/s"] > 0
    assert record["replays"] == 3 and record["rounds"] == 3


@pytest.mark.parametrize("sources,tokens,width,rank", [
    (9, 256, 2048, 2048),   # c4's form: the whole row as key
    (4, 130, 1024, 256),    # recompute policy, key masks, a partial token group
])
def test_graph_replay_list_times_every_part(sources, tokens, width, rank):
    print(f"graph_replay_list S={sources} N={tokens} D={width} R={rank}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(0)
    dev = torch.device("cuda:0")
    rows = [torch.randn(tokens, width, device=dev, generator=g).to(torch.bfloat16) for _ in range(sources)]
    queries = [(torch.randn(rank, device=dev, generator=g) / rank**0.5).to(torch.bfloat16) for _ in range(3)]
    grads = [torch.randn(tokens, width, device=dev, generator=g).to(torch.bfloat16) for _ in range(3)]
    record = bench.graph_replay_list(rows, queries, grads, {"width": width, "rank": rank}, replays=3, rounds=3)
    _check(record)
    assert "3 reads" in record["boundary"]


def test_graph_replay_packed_times_every_part():
    print("graph_replay packed S=6 N=300 D=2048 R=512", flush=True)
    g = torch.Generator(device="cuda").manual_seed(1)
    dev = torch.device("cuda:0")
    values = torch.randn(6, 300, 2048, device=dev, generator=g).to(torch.bfloat16)
    query = (torch.randn(512, device=dev, generator=g) / 512**0.5).to(torch.bfloat16)
    grad_out = torch.randn(300, 2048, device=dev, generator=g).to(torch.bfloat16)
    record = bench.graph_replay(values, query, grad_out, {"sources": 6, "width": 2048, "rank": 512},
                                replays=3, rounds=3)
    _check(record)


@pytest.mark.parametrize("width,rank", [(1024, 256), (2048, 2048)])
def test_sweep_graph_step_replays_every_read(width, rank):
    """c5's whole-step graph: the reads of S = 1..14 (recompute, key-resident,
    saved-path and, at 2048, token-block backwards) in one captured graph."""
    print(f"sweep graph step S=1..14 N=200 D={width} R={rank}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(2)
    dev = torch.device("cuda:0")
    values = torch.randn(14, 200, width, device=dev, generator=g).to(torch.bfloat16)
    query = (torch.randn(rank, device=dev, generator=g) / rank**0.5).to(torch.bfloat16)
    grad_out = torch.randn(200, width, device=dev, generator=g).to(torch.bfloat16)
    record = bench._sweep_graph_step(values, query, grad_out, 14, width, rank, replays=2, rounds=3)
    assert 0 < record["ms_q1"] <= record["ms_per_step"] <= record["ms_q3"], record
    assert record["TB/s"] > 0
