import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "vllm-cpp_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on the GPU)")


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def pytest_terminal_summary(terminalreporter):
    """Max-abs and normwise relative error of every GPU parity check run."""
    try:
        import gpu_util
    except Exception:
        return
    log = getattr(gpu_util, "PARITY_LOG", [])
    if not log:
        return
    tr = terminalreporter
    tr.section("parity: max-abs / normwise relative error (bound)")
    for what, ma, rel, atol, rtol in log:
        tr.write_line("%-60s max-abs %.3e (<= %.0e)  rel %.3e (<= %.0e)" % (what[:60], ma, atol, rel, rtol))
