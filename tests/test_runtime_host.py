"""The model runtime's host logic on the CPU: the schedule cover that picks prefill chunks and the
MTP head's catch-up runs, and the manifest parse, on the committed exports (tests/golden). The
device side runs in tests/test_gpu_runtime.py."""
from __future__ import annotations

import itertools
import json

import numpy as np

from export_fixture import KINDS, unpack
from opentars_amd.runtime import ExportLayout, cover


def brute_cover(start, stop, sizes_at):
    """The greedy rule stated step by step: at each position the largest offered length that fits."""
    runs, t = [], start
    while t < stop:
        fits = sorted((s for s in sizes_at(t) if t + s <= stop), reverse=True)
        n = fits[0] if fits else 1
        runs.append((t, n))
        t += n
    return runs


def test_cover_runs_are_consecutive_and_greedy():
    rng = np.random.default_rng(7)
    for trial in range(300):
        table = {int(t): tuple(int(s) for s in rng.choice([2, 4, 8], size=rng.integers(0, 3), replace=False))
                 for t in rng.integers(0, 40, size=rng.integers(0, 20))}
        start = int(rng.integers(0, 20))
        stop = start + int(rng.integers(0, 25))
        runs = cover(start, stop, lambda t: table.get(t, ()))
        assert runs == brute_cover(start, stop, lambda t: table.get(t, ()))
        pos = start
        for t, n in runs:
            assert t == pos and n >= 1 and (n == 1 or n in table.get(t, ()))
            pos += n
        assert pos == max(start, stop)


def test_cover_known_cases():
    chunks = {0: (8, 4), 8: (8, 4), 12: (4,)}
    at = lambda t: chunks.get(t, ())
    assert cover(0, 13, at) == [(0, 8), (8, 4), (12, 1)]
    assert cover(0, 7, at) == [(0, 4), (4, 1), (5, 1), (6, 1)]
    assert cover(3, 3, at) == []
    assert cover(0, 3, lambda t: ()) == [(0, 1), (1, 1), (2, 1)]
    # the MTP head's catch-up: runs of 4 where the export has that queue, single rows elsewhere
    four = {0, 4, 8}
    assert cover(0, 9, lambda r: (4,) if r in four else ()) == [(0, 4), (4, 4), (8, 1)]
    assert cover(2, 9, lambda r: (4,) if r in four else ()) == [(2, 1), (3, 1), (4, 4), (8, 1)]


def test_layout_parses_every_committed_export(tmp_path):
    for kind in KINDS:
        (tmp_path / kind).mkdir()
        d = unpack(tmp_path / kind, kind)
        m = json.loads((d / "manifest.json").read_text())
        lay = ExportLayout.parse(m)
        assert (lay.positions, lay.hidden, lay.vocab) == (m["max_tokens"], m["hidden"], m["vocab"])
        assert lay.mem_bytes >= lay.image_bytes == (d / "image.bin").stat().st_size
        assert lay.x0 == (m["x0_off"], m["x0_ld"]) and lay.logits == m["logits_off"]
        assert sum(lay.head_blocks) == lay.vocab
        assert (lay.ple is None) == (not m.get("ple_cols"))
        assert (d / "embed_bf16.bin").stat().st_size == 2 * lay.vocab * lay.hidden
        if lay.ple:
            assert (d / "ple_bf16.bin").stat().st_size == 2 * lay.vocab * lay.ple[2]
        # every queue entry lies inside its file
        for t, (off, n) in enumerate(m["queue_index"]):
            assert off + 64 * n <= (d / "queues.bin").stat().st_size
        for c, index in itertools.chain(m.get("chunks", {}).items(),
                                        ((f"s_{k}", v) for k, v in m.get("spec", {}).items())):
            f = d / (f"queues_c{c}.bin" if not str(c).startswith("s_") else f"queues_{c}.bin")
            for _, off, n in index:
                assert off + 64 * n <= f.stat().st_size


def test_layout_raises_the_firmware_level_for_fp16_states(tmp_path):
    m = json.loads((unpack(tmp_path) / "manifest.json").read_text())
    assert ExportLayout.parse(m).min_firmware == m["min_firmware"] == 0
    m["state_dtype"] = "fp16"
    assert ExportLayout.parse(m).min_firmware == 0x30400
