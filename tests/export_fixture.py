"""The small board exports of tests/golden/export_*.npz (written by make_export_fixture.py from the
reference's lowering and runtime) unpacked into a directory, and the results recorded on them."""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"
KINDS = {"qwen3": "export_small.npz", "qwen35_mtp": "export_qwen35_mtp.npz", "gemma4": "export_gemma4.npz",
         "gemma3_ksplit": "export_gemma3_ksplit.npz", "gemma4_w4": "export_gemma4_w4.npz"}


def unpack(dst: Path, kind: str = "qwen3") -> Path:
    """The export's files into dst; returns dst."""
    with np.load(GOLDEN / KINDS[kind]) as z:
        for name in z.files:
            (dst / name).write_bytes(z[name].tobytes())
    return dst


def expected(d: Path) -> list:
    return json.loads((d / "expected.json").read_text())


def sha(logits: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(logits, np.float32).tobytes()).hexdigest()
