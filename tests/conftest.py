import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built libdrt_rocm.so")
    config.addinivalue_line("markers", "slow: long CPU oracle runs")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(autouse=True)
def _parity_log_test_id(request):
    """Names the running test in the parity exemption log (tests/helpers.py)."""
    import helpers

    helpers.CURRENT_TEST[0] = request.node.nodeid
    yield
    helpers.CURRENT_TEST[0] = ""


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """One line with every reported parity exemption of the run (count, kind,
    bound, largest gap and its test), so that a -q run's tail carries it."""
    import helpers

    terminalreporter.write_line(helpers.parity_summary())


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
