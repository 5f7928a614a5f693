"""Shared pytest configuration.

Markers:
  gpu -- needs an MI355X: runs the HIP path through the C-ABI of
         libtemplit_hip.so and compares it with the CPU oracle.
Everything unmarked runs on a CPU-only machine.
"""
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for p in (str(ROOT), str(ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X GPU (HIP path vs the CPU oracle)")
