"""Test configuration: the repository root on sys.path and the `gpu` marker.

Tests marked `gpu` need an MI355X (gfx950) and the built HIP library; everything else runs on a
CPU-only host."""
from __future__ import annotations

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built HIP library")
