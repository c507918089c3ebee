"""pytest configuration: the `gpu` marker and import paths (repository root, the package directory
causal-conv1d-triton_amd/ and oracle/)."""

import os
import sys

_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "causal-conv1d-triton_amd", "oracle", "tests"):
    p = os.path.join(_ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built libccv1d.so")
