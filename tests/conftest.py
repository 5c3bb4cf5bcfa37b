from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU visible to torch")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O

    O.build()
    return O


def pytest_terminal_summary(terminalreporter):
    """One line per elementwise parity comparison that passed: the largest
    |dV|, |dtau|, |dR|/||a_j|| and the worst error-to-tolerance ratio."""
    from tests import parity

    if not parity.MARGINS:
        return
    terminalreporter.section(f"parity margins ({len(parity.MARGINS)} comparisons)")
    for line in parity.MARGINS:
        terminalreporter.write_line(line)
    worst = max(float(line.rsplit("=", 1)[1]) for line in parity.MARGINS)
    terminalreporter.write_line(f"largest error/tolerance over all comparisons: {worst:.3f}")
