"""The oracle's descriptor-queue walk over whole board exports: the small Qwen3, Qwen3.5 (DeltaNet
and full attention) and Gemma 4 (sliding / full attention, shared KV, per-layer embeddings)
exports of tests/golden/export_*.npz run token by token and in prefill chunks reproduce, bit for
bit, the logits the reference's runtime recorded on its golden backend (the SHA-256 of every
step's fp32 logits, tools/export_kv260.py:320-347). This pins the oracle's row, elementwise, RoPE,
FDOT, quantizer and GEMM steps together, in the orders the reference's lowering emits them."""
from __future__ import annotations

import json

import numpy as np
import pytest

from oracle import queue as Q
from export_fixture import KINDS, expected, sha, unpack


class OracleBoard:
    """A minimal board runtime over the oracle (the steps of tars_board.Qwen: embedding rows into
    x0, the position's queue into the queue region, the run, the logits)."""

    def __init__(self, d):
        m = self.m = json.loads((d / "manifest.json").read_text())
        img = (d / "image.bin").read_bytes()
        assert len(img) == m["image_bytes"]
        self.ddr = bytearray(max(len(img), m["mem_bytes"]))
        self.ddr[:len(img)] = img
        self.state0 = bytes(self.ddr[:m["state_end"]])
        self.embed = np.fromfile(d / "embed_bf16.bin", np.uint16).reshape(m["vocab"], m["hidden"])
        self.ple = np.fromfile(d / "ple_bf16.bin", np.uint16).reshape(m["vocab"], m["ple_cols"]) \
            if m.get("ple_cols") else None
        self.queues = (d / "queues.bin").read_bytes()
        self.chunks = {int(n): ((d / f"queues_c{n}.bin").read_bytes(), {t0: (o, k) for t0, o, k in idx})
                       for n, idx in m["chunks"].items()}
        self.pos = 0

    def new_conversation(self):
        self.ddr[:self.m["state_end"]] = self.state0
        self.pos = 0

    def _put(self, t, tokens):
        m = self.m
        for i, tok in enumerate(tokens):
            x = (self.embed[tok].astype(np.uint32) << 16).view(np.float32)
            if m["embed_scale"] is not None:
                x = x * np.float32(m["embed_scale"])
            a = m["x0_off"] + (t + i) * m["x0_ld"]
            self.ddr[a:a + 4 * m["hidden"]] = x.astype(np.float32).tobytes()
            if self.ple is not None:
                p = (self.ple[tok].astype(np.uint32) << 16).view(np.float32) * np.float32(m["ple_scale"])
                a = m["ple0_off"] + (t + i) * m["ple0_ld"]
                self.ddr[a:a + 4 * m["ple_cols"]] = p.astype(np.float32).tobytes()

    def _run(self, queues, off, n):
        q, cap = self.m["qbase"], self.m["queue_cap"]
        for s in range(0, n, cap):
            k = min(cap, n - s)
            self.ddr[q:q + 64 * k] = queues[off + 64 * s:off + 64 * (s + k)]
            mach = Q.Machine(self.ddr)
            st = mach.run_queue(q, k)
            assert st.done and st.err_code == 0, st
            self.ddr = mach.ddr

    def logits(self):
        lo = self.m["logits_off"]
        return np.frombuffer(bytes(self.ddr[lo:lo + 4 * self.m["vocab"]]), np.float32).copy()

    def step(self, tok):
        self._put(self.pos, [tok])
        off, n = self.m["queue_index"][self.pos]
        self._run(self.queues, off, n)
        self.pos += 1
        return self.logits()

    def prefill(self, tokens):
        i = 0
        while i < len(tokens):
            n = next((n for n in sorted(self.chunks, reverse=True)
                      if i + n <= len(tokens) and self.pos in self.chunks[n][1]), 1)
            if n == 1:
                self.step(tokens[i])
            else:
                self._put(self.pos, tokens[i:i + n])
                qs, idx = self.chunks[n]
                off, k = idx[self.pos]
                self._run(qs, off, k)
                self.pos += n
            i += n
        return self.logits()


@pytest.fixture(scope="module", params=list(KINDS))
def export_dir(request, tmp_path_factory):
    return unpack(tmp_path_factory.mktemp(request.param), request.param)


@pytest.mark.parametrize("case", [0, 1])
def test_oracle_reproduces_the_reference_runtime_on_an_export(export_dir, case):
    exp = expected(export_dir)[case]
    b = OracleBoard(export_dir)
    b.new_conversation()
    for s in exp["steps"]:
        lg = b.step(s["token"])
        assert (int(np.argmax(lg)), sha(lg)) == (s["argmax"], s["sha256"]), f"{exp['name']} step {s['pos']}"
    b.new_conversation()
    lg = b.prefill(exp["ids"])
    first = exp["prefill"][0]
    assert (int(np.argmax(lg)), sha(lg)) == (first["argmax"], first["sha256"])
    for s in exp["prefill"][1:]:
        lg = b.step(s["token"])
        assert (int(np.argmax(lg)), sha(lg)) == (s["argmax"], s["sha256"]), f"{exp['name']} after prefill {s['pos']}"


def test_runtime_needs_a_gpu(export_dir):
    """No CPU fallback: without a GPU the loader refuses to start."""
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from opentars_amd.runtime import GpuDevice, Model
    with pytest.raises(RuntimeError, match="needs a ROCm GPU"):
        Model(export_dir, log=None)
    with pytest.raises(RuntimeError, match="needs a ROCm GPU"):
        GpuDevice(1 << 20)


def _descs(export_dir, pos):
    m = json.loads((export_dir / "manifest.json").read_text())
    off, n = m["queue_index"][pos]
    raw = (export_dir / "queues.bin").read_bytes()[off:off + 64 * n]
    return [Q.decode(raw[64 * i:64 * i + 64]) for i in range(n)]


def test_ksplit_export_holds_two_block_down_projections(tmp_path):
    """export_gemma3_ksplit.npz pins the K split end to end: every layer's down projection is two
    QM_ROWCOL GEMMs over K = 2304 blocks of one quantized row (the same row scale and per-channel
    scales), their partials added by an fp32 ELT ADD (llm.py:303-321, 627-635)."""
    d = unpack(tmp_path, "gemma3_ksplit")
    ds = _descs(d, 5)
    blocks = [i for i, x in enumerate(ds) if x["OPCODE"] == Q.OP_GEMM and x["K"] == 2304]
    assert len(blocks) == 2 * 2                                      # two layers, two blocks each
    for i in blocks[::2]:
        a, b = ds[i], ds[i + 1]
        assert b["OPCODE"] == Q.OP_GEMM and b["K"] == 2304 and a["N"] == b["N"] == 256
        assert a["SCALE_OFF"] == b["SCALE_OFF"] and a["A_OFF"] != b["A_OFF"]       # shared scales, the row's halves
        adds = [x for x in ds[i + 2:i + 6] if x["OPCODE"] == Q.OP_ELT and x["CTRL"] & 3 == Q.ELT_ADD]
        assert adds, "the block partials are added by an ELT ADD"


def test_w4_export_runs_every_linear_as_w4a16_with_k_blocks(tmp_path):
    """export_gemma4_w4.npz: every GEMM of a decode step is W4A16 (QM_GROUP, int4 weights), and
    the KV-shared layers' double-wide down projections (K = 4608) are two W4 K blocks with their
    own group scales (llm.py:120-132, 306-313)."""
    d = unpack(tmp_path, "gemma4_w4")
    ds = _descs(d, 3)
    gemms = [x for x in ds if x["OPCODE"] == Q.OP_GEMM]
    assert gemms and all(Q.is_w4(x) for x in gemms)
    kb = [i for i, x in enumerate(ds) if Q.is_w4(x) and x["K"] == 2304 and x["N"] == 256]
    pairs = [(ds[i], ds[i + 1]) for i in kb if i + 1 < len(ds) and Q.is_w4(ds[i + 1]) and ds[i + 1]["K"] == 2304]
    assert len(pairs) >= 2
    for a, b in pairs:
        assert a["SCALE_OFF"] != b["SCALE_OFF"] and a["W_OFF"] != b["W_OFF"]         # each block its own scales
