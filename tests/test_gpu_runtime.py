"""The export loader and runtime on the GPU (opentars_amd.runtime): the small Qwen3, Qwen3.5
(DeltaNet, MTP head) and Gemma 4 (per-layer embeddings, scaled input embedding) exports of
tests/golden/export_*.npz (the reference's lowering) run by Model, and by the reference-style
device interface GpuDevice, reproduce the logits the reference's runtime recorded on its golden
backend, bit for bit (the SHA-256 of every step's fp32 logits), token by token, in prefill chunks
and in speculative rounds. Needs a gfx950 GPU."""
from __future__ import annotations

import json

import numpy as np
import pytest

from export_fixture import KINDS, expected, sha, unpack

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def export_dir(tmp_path_factory):
    return unpack(tmp_path_factory.mktemp("export"))


@pytest.fixture(scope="module", params=list(KINDS))
def any_export(request, tmp_path_factory):
    return unpack(tmp_path_factory.mktemp(request.param), request.param)


def check_case(model, exp):
    model.new_conversation()
    for s in exp["steps"]:
        lg = model.step(s["token"])
        assert (int(np.argmax(lg)), sha(lg)) == (s["argmax"], s["sha256"]), f"{exp['name']} step {s['pos']}"
    model.new_conversation()
    lg = model.prefill(exp["ids"], chunked=True)
    first = exp["prefill"][0]
    assert (int(np.argmax(lg)), sha(lg)) == (first["argmax"], first["sha256"]), f"{exp['name']} prefill"
    for s in exp["prefill"][1:]:
        lg = model.step(s["token"])
        assert (int(np.argmax(lg)), sha(lg)) == (s["argmax"], s["sha256"]), f"{exp['name']} after prefill {s['pos']}"


def test_model_reproduces_the_reference_runtime(any_export):
    from opentars_amd.runtime import Model
    model = Model(any_export, log=None)
    for exp in expected(any_export):
        check_case(model, exp)


def test_speculative_rounds_reproduce_the_reference_runtime(tmp_path):
    """The MTP export: prefill, the first draft, verify rounds on both state copies (hits and
    misses), the swap back; the same tokens and verify rows as the reference's runtime."""
    from opentars_amd.runtime import Model
    d = unpack(tmp_path, "qwen35_mtp")
    model = Model(d, log=None)
    for exp in expected(d):
        spec = exp["spec"]
        model.new_conversation()
        lg = model.prefill(exp["ids"], chunked=True)
        cur = model.begin_spec(lg)
        toks = [cur]
        assert cur == spec["first"]
        for r in spec["rounds"]:
            assert model.can_spec()
            assert model.draft == r["draft"]
            new, rows = model.spec_round(cur)
            assert (model.pos, new, sha(rows)) == (r["pos"], r["new"], r["rows_sha256"]), r
            toks += new
            cur = new[-1]
        model.end_spec()
        assert toks == spec["tokens"]
        greedy = [s["argmax"] for s in exp["steps"][len(exp["ids"]) - 1:]]
        assert toks[:len(greedy)] == greedy[:len(toks)]       # the tokens of plain greedy decoding


def test_prefill_without_chunks_and_queue_parts(export_dir, tmp_path):
    """Every prompt token a step (chunked=False), and queues run in parts of 29 descriptors
    through the queue region (a manifest with a smaller queue_cap): the same bits."""
    from opentars_amd.runtime import Model
    d = unpack(tmp_path)
    m = json.loads((d / "manifest.json").read_text())
    m["queue_cap"] = 29
    (d / "manifest.json").write_text(json.dumps(m))
    model = Model(d, log=None)
    exp = expected(export_dir)[0]
    lg = model.prefill(exp["ids"], chunked=False)
    assert sha(lg) == exp["steps"][len(exp["ids"]) - 1]["sha256"]
    check_case(model, exp)


def test_context_overflow_and_a_wrong_image_size(export_dir, tmp_path):
    from opentars_amd.runtime import Model
    model = Model(export_dir, log=None)
    model.pos = model.T - 1
    with pytest.raises(OverflowError):
        model.prefill([1, 2])
    d = unpack(tmp_path)
    with open(d / "image.bin", "ab") as f:
        f.write(b"\0" * 16)
    with pytest.raises(RuntimeError, match="the manifest says"):
        Model(d, log=None)


class DeviceDriver:
    """The reference runtime's use of a board device (tars_board.Qwen: the image into dev.mem,
    to_dev; per token the embedding row and the queue into dev.mem, to_dev, run, from_dev of the
    logits), over GpuDevice."""

    def __init__(self, dev, d):
        self.dev, self.m = dev, json.loads((d / "manifest.json").read_text())
        img = np.fromfile(d / "image.bin", np.uint8)
        dev.mem[:img.size] = img
        dev.mem[img.size:] = 0
        dev.to_dev(0, dev.mem.size)
        self.state0 = dev.mem[:self.m["state_end"]].copy()
        self.embed = np.fromfile(d / "embed_bf16.bin", np.uint16).reshape(self.m["vocab"], self.m["hidden"])
        self.queues = np.fromfile(d / "queues.bin", np.uint8)
        self.pos = 0

    def new_conversation(self):
        self.dev.mem[:self.m["state_end"]] = self.state0
        self.dev.to_dev(0, self.m["state_end"])
        self.pos = 0

    def step(self, tok):
        m, dev = self.m, self.dev
        a = m["x0_off"] + self.pos * m["x0_ld"]
        x = (self.embed[tok].astype(np.uint32) << 16).view(np.float32)
        dev.mem[a:a + 4 * m["hidden"]] = np.frombuffer(x.tobytes(), np.uint8)
        dev.to_dev(a, 4 * m["hidden"])
        off, n = m["queue_index"][self.pos]
        q = m["qbase"]
        dev.mem[q:q + 64 * n] = self.queues[off:off + 64 * n]
        dev.to_dev(q, 64 * n)
        done, err, op, _ = dev.run(q, n)
        assert done and not err, (err, op)
        self.pos += 1
        lo = m["logits_off"]
        dev.from_dev(lo, 4 * m["vocab"])
        return dev.mem[lo:lo + 4 * m["vocab"]].view(np.float32).copy()


def test_gpu_device_under_the_reference_runtime_calls(export_dir):
    from opentars_amd.runtime import GpuDevice
    m = json.loads((export_dir / "manifest.json").read_text())
    drv = DeviceDriver(GpuDevice(mem_bytes=m["mem_bytes"]), export_dir)
    for exp in expected(export_dir):
        drv.new_conversation()
        for s in exp["steps"]:
            lg = drv.step(s["token"])
            assert (int(np.argmax(lg)), sha(lg)) == (s["argmax"], s["sha256"]), f"{exp['name']} step {s['pos']}"


def test_embed_rows_matches_the_host_lookup():
    """tars_embed_rows against numpy's bf16 -> fp32 shift and float32 multiply (the board runtime's
    host lookup, tars_board.py:298-314): random bf16 bits with zeros, infinities, subnormals and
    products that round into the subnormal range; scaled and unscaled; the 16-byte vector path
    (256 and 512 columns) and the element path (odd widths, a strided table); more ids than one
    launch takes; repeated ids."""
    import torch
    from opentars_amd import ops
    rng = np.random.default_rng(11)
    for rows, cols, ld_extra in ((512, 256, 0), (300, 512, 0), (97, 37, 3), (64, 8, 8)):
        bits = rng.integers(0, 1 << 16, (rows, cols + ld_extra), dtype=np.uint32).astype(np.uint16)
        bits = np.where((bits & 0x7F80) == 0x7F80, bits & 0x807F, bits)        # no NaN / inf ...
        bits[0, :4] = [0x0000, 0x8000, 0x7F80, 0xFF80]                        # ... but zeros and infinities
        bits[1, :4] = [0x0001, 0x807F, 0x0080, 0x3F80]                        # subnormal, min normal, 1.0
        table = torch.from_numpy(bits.view(np.int16)).cuda()[:, :cols]
        ids = rng.integers(0, rows, 150)
        ids[:3] = [0, 1, 0]
        ref32 = (bits[:, :cols][ids].astype(np.uint32) << 16).view(np.float32)
        for scale in (None, 16.0, 11.313708305358887, 3.0e-30):
            got = ops.embed_rows(table, ids, scale).cpu().numpy()
            with np.errstate(over="ignore"):
                want = ref32 if scale is None else (ref32 * np.float32(scale)).astype(np.float32)
            assert got.view(np.uint32).tobytes() == want.view(np.uint32).tobytes(), (rows, cols, scale)
