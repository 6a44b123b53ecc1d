"""pytest configuration: the `gpu` marker and import paths.

`-m gpu` tests need an MI355X (gfx950) and the built libmynah_hip.so; they call
the kernels through the C ABI. Everything else runs on the CPU: the oracle
against the golden vectors, host logic, and the library's exported symbols.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "tests"), os.path.join(ROOT, "mynah-slm_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")
