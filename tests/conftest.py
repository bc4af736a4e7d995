"""Test configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs the oracle pins, host logic and C-ABI load checks on
any machine; ``-m gpu`` runs the parity tests of the HIP kernels against the
oracle on a real MI355X.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "gmdn-gated-muon-deltanet_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built native library")
