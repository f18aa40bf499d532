"""Test setup: the `ultrametric` drop-in package lives in sparse-ai_amd/ (the
role of the reference's src/, tests/conftest.py:4-9 there), the CPU oracle in
oracle/. Tests marked `gpu` need an MI355X; everything else runs on CPU."""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "sparse-ai_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built libsparseattn.so")
