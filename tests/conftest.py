"""pytest configuration: the `gpu` marker and import paths.

`-m "not gpu"` runs on a machine without a GPU (oracle, host logic, C-ABI
validation); `-m gpu` runs the parity tests on an MI355X through the C ABI.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_PARENT = os.path.join(ROOT, "flash-attn-volta_amd")
for p in (ROOT, PKG_PARENT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (gfx950) GPU")
