"""Test configuration: import paths and the `gpu` marker.

`-m "not gpu"` runs on the CPU (oracle pinning, host logic, C-ABI load and exports);
`-m gpu` runs the parity tests on an MI355X through the C-ABI library.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PACKAGE = os.path.join(ROOT, "official-mira-llm_amd")
for path in (ROOT, PACKAGE):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")
