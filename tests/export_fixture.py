"""The small board export of tests/golden/export_small.npz (written by make_export_fixture.py from
the reference's lowering and runtime) unpacked into a directory, and the results recorded on it."""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np

NPZ = Path(__file__).resolve().parent / "golden" / "export_small.npz"


def unpack(dst: Path) -> Path:
    """The export's files into dst; returns dst."""
    with np.load(NPZ) as z:
        for name in z.files:
            (dst / name).write_bytes(z[name].tobytes())
    return dst


def expected(d: Path) -> list:
    return json.loads((d / "expected.json").read_text())


def sha(logits: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(logits, np.float32).tobytes()).hexdigest()
