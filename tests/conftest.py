"""Shared pytest setup: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs the oracle, host-logic and C-ABI load tests on CPU;
``-m gpu`` runs the parity tests through the C ABI on an MI355X.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "nano-vllm-jax_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libnvjsel.so")


def pytest_collection_modifyitems(config, items):
    import pytest

    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Every row a GPU parity checker exempted (tests/gpu_helpers.report)."""
    try:
        from tests.gpu_helpers import REPORTS
    except Exception:  # pragma: no cover
        return
    if REPORTS:
        terminalreporter.section("parity exemptions (rows reported, not hidden)")
        for line in REPORTS:
            terminalreporter.write_line(line)
