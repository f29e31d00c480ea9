"""pytest configuration: import paths and the `gpu` marker.

CPU tests (-m "not gpu") check the oracle against the reference's golden
vectors and known answers, the host logic, and that libgk_fp8.so loads and
exports its C ABI.  GPU tests (-m gpu) run the gfx950 kernels through the C
ABI and compare them with the oracle.
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "gaudi-kernels_amd", "python")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built libgk_fp8.so")


def pytest_report_header(config):
    return f"gaudi-kernels_amd tests (root {ROOT})"
