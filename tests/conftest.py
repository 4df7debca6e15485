"""Test configuration: put the repo root (oracle/) and the package directory on sys.path
and register the `gpu` marker (tests that need a ROCm MI355X device)."""

from __future__ import annotations

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "speedup-thingy_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm gfx950 device and the built librte_hip.so")
