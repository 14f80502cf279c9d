import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """The largest output errors the GEMM parity checks measured."""
    try:
        from tests.util import MEASURED
    except ImportError:
        return
    if not MEASURED:
        return
    tr = terminalreporter
    tr.section("largest measured GEMM errors (bounds: max-rel 1e-2, elementwise 1e-2)")
    for what, g, e in sorted(MEASURED, key=lambda t: -t[2])[:8]:
        tr.write_line(f"elementwise {e:.3e}  max-rel {g:.3e}  {what}")
    worst = max(MEASURED, key=lambda t: t[1])
    tr.write_line(f"largest max-rel {worst[1]:.3e} ({worst[0]}); {len(MEASURED)} checks")
