"""Pytest configuration: import paths and the `gpu` marker.

Tests marked `gpu` need an MI355X (they run the HIP kernels); everything
else runs on the CPU: the oracle against the reference's golden vectors,
host logic, and the C ABI surface of the built library.
"""

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "associative-scan-triton_amd", ROOT, ROOT / "tests"):
  if str(p) not in sys.path:
    sys.path.insert(0, str(p))


def pytest_configure(config):
  config.addinivalue_line(
    "markers", "gpu: needs a HIP device (MI355X); runs the gfx950 kernels")
