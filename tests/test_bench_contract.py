"""bench.py's contract on the CPU: the algorithmic byte counts its roofline
uses, and the one-GPU rule.

The byte counts are the ones the headline metric is defined on (forward:
values read + output written; backward: values and dO read, dvalues
written); the expected figures are the per-config numbers the benchmark's
roofline targets are stated in, so a dropped or doubled term fails here.
"""

from __future__ import annotations

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


@pytest.mark.parametrize("sources,tokens,width,forward,backward", [
    (25, 16384, 2048, 1_744_830_464, 3_422_552_064),   # c2
    (16, 16384, 4096, 2_281_701_376, 4_429_185_024),   # c3
    (9, 32768, 2048, 1_342_177_280, 2_550_136_832),    # c4, one read
])
def test_read_bytes_match_the_stated_config_figures(sources, tokens, width, forward, backward):
    assert bench.read_bytes(sources, tokens, width) == (forward, backward)


def test_c5_bytes_per_step_match_the_sweep_formula():
    """Per read N*D*2*(3S+2) bytes; over S = 1..48 that is N*D*2*3624."""
    for width, total in ((1024, 121_601_261_568), (4096, 486_405_046_272)):
        assert sum(sum(bench.read_bytes(s, 16384, width)) for s in range(1, 49)) == total
        assert sum(16384 * width * 2 * (3 * s + 2) for s in range(1, 49)) == total


def test_more_than_one_gpu_is_refused_with_a_message():
    result = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                            capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert result.returncode != 0
    assert "one GPU" in result.stderr
    assert result.stdout.strip() == ""  # no JSON line
