"""Test configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs the oracle, fixture and host-side checks on any machine;
``-m gpu`` runs the HIP parity tests through the C ABI on an MI355X.
"""

import os
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "algebraic-transformer_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")
