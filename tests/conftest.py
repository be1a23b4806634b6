"""Shared test set-up: import paths and the `gpu` marker.

`-m "not gpu"` runs the oracle checks, host logic and C-ABI export checks on
any CPU host; `-m gpu` runs the parity tests through libpcl_hip on a gfx950
GPU (they fail, never skip, when the library or device is unusable).
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for d in (ROOT, os.path.join(ROOT, "pure-c-llm_amd"), os.path.join(ROOT, "oracle")):
    if d not in sys.path:
        sys.path.insert(0, d)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs through libpcl_hip)")
