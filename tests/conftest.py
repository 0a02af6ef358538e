"""Test configuration: import paths and the `gpu` marker.

`-m "not gpu"` runs the oracle pinning, host-logic and C-ABI export checks on CPU;
`-m gpu` runs the HIP parity tests (they fail, not skip, when no GPU is visible so a
silent CPU run can never count as parity).
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "rdna4-vllm_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
