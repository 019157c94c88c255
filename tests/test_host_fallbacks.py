"""Host-side fallbacks for torch builds without the private queries the
launch path prefers (CPU only: the queries are replaced, nothing launches)."""

from __future__ import annotations

import types

import pytest
import torch

from attnres import _ops, shared


def test_stream_handle_falls_back_to_the_public_stream(monkeypatch):
    seen = []

    def current_stream(device):
        seen.append(device)
        return types.SimpleNamespace(cuda_stream=0x1234)

    monkeypatch.setattr(_ops, "_RAW_STREAM", None)
    monkeypatch.setattr(torch.cuda, "current_stream", current_stream)
    device = torch.device("cuda", 0)
    assert _ops._stream(device) == 0x1234
    assert seen == [device]


def test_stream_handle_prefers_the_raw_query(monkeypatch):
    monkeypatch.setattr(_ops, "_RAW_STREAM", lambda index: 100 + index)
    monkeypatch.setattr(torch.cuda, "current_stream", lambda device: pytest.fail("public Stream built"))
    assert _ops._stream(torch.device("cuda", 3)) == 103


def test_shared_reads_without_the_graph_task_query_raise(monkeypatch):
    monkeypatch.setattr(shared, "_GRAPH_TASK_ID", None)
    with pytest.raises(RuntimeError, match="_current_graph_task_id"):
        shared._pass_id()


def test_pass_id_outside_a_backward_pass():
    assert shared._pass_id() == -1
