"""Shared pytest setup: the `gpu` marker and import paths.

`-m "not gpu"` runs the oracle pins, host logic and ABI-export checks on any
CPU; `-m gpu` runs the parity tests proper, through the C-ABI, on an MI355X.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "glacier.tune_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
