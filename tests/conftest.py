"""Shared pytest setup.

Marker `gpu`: needs an MI355X (the HIP library's kernels run); everything else
runs on the CPU.  The oracle (oracle/liboracle.so) is test infrastructure and
is built here with g++ if it is missing.
"""
from __future__ import annotations

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "qwen3-asr-wgpu_amd")
for p in (os.path.join(REPO, "oracle"), PKG, os.path.join(REPO, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the HIP kernels)")


def pytest_sessionfinish(session, exitstatus):
    """Write every parity check's figures (workloads.REPORT) to
    $QASR_PARITY_REPORT, if set."""
    path = os.environ.get("QASR_PARITY_REPORT")
    if not path:
        return
    import json

    import workloads

    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "w") as f:
        json.dump(workloads.REPORT, f, indent=1)


def _ensure_oracle():
    import oracle

    if not os.path.exists(os.path.join(REPO, "oracle", "liboracle.so")):
        oracle.build()
    return oracle


@pytest.fixture(scope="session")
def O():
    """The CPU oracle module (ctypes over liboracle.so)."""
    return _ensure_oracle()


@pytest.fixture(scope="session")
def gpu():
    """The HIP binding; skips nothing -- a gpu-marked test without a GPU fails."""
    import torch

    import qasr_attn

    if not torch.cuda.is_available():
        pytest.fail("gpu-marked test run without a visible GPU")
    qasr_attn.load()
    return qasr_attn
