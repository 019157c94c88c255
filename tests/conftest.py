"""Test configuration: import paths, the `gpu` marker and GPU availability.

`gpu` tests run the HIP kernels on an MI355X and compare them with the CPU
oracle in `oracle/`; everything else runs on a CPU-only machine.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT, ROOT / "fast-attnres_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(autouse=True)
def _gpu_required(request):
    """A `gpu` test on a machine without a GPU fails loudly instead of skipping."""
    if request.node.get_closest_marker("gpu") is not None:
        import torch

        assert torch.cuda.is_available(), "gpu test selected but no ROCm GPU is visible"
        torch.compiler.reset()
    yield


def pytest_sessionfinish(session, exitstatus):
    """With ATTNRES_PARITY_TABLE=<path>, write the recorded error metrics of
    every comparison (tests/helpers.py) as JSON."""
    import json
    import os

    path = os.environ.get("ATTNRES_PARITY_TABLE")
    if not path:
        return
    helpers = sys.modules.get("helpers")
    records = getattr(helpers, "RECORDS", []) if helpers else []
    Path(path).parent.mkdir(parents=True, exist_ok=True)
    Path(path).write_text(json.dumps(records, indent=1))
