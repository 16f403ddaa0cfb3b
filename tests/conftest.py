"""pytest configuration: the ``gpu`` marker and the repository root on sys.path.

``-m "not gpu"`` runs the oracle, host-logic and C-ABI-loading tests on any
machine; ``-m gpu`` runs the parity tests of the HIP kernels on a MI355X.
"""

from __future__ import annotations

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built libtkv_hip.so")
