"""Board exports on one MI355X: a device with the board runtime's interface, and the loader and
model runtime of an export directory.

An export (tools/export_kv260.py:13-32, 141-247) is a directory: image.bin (the DDR image from
address 0: zeroed states, the queue region, scratch, quantized weights), embed_bf16.bin (the
embedding table [vocab, hidden] as bf16), ple_bf16.bin (Gemma 4's per-layer embeddings),
queues.bin (one descriptor queue per token position), queues_c<n>.bin (prefill chunks of n
tokens), queues_s_*.bin (speculative decoding) and manifest.json (addresses, sizes, the queue
indexes, tokenizer settings).

GpuDevice is a device of the board runtime (deploy/kv260/sw/tars_board.py:4-12: mem, to_dev,
from_dev, run(q, n) -> (done, err, op_idx, cycles), like Fpga :50-152 and Golden :155-178) whose
image lives in HBM and whose queues run through the library's executor (tars_run_queue), so the
reference's runtime (tars_board.Qwen) runs on it as it is.

Model is that runtime's own counterpart (tars_board.py:212-435: Qwen) with the export resident on
the GPU: image.bin is read straight into device memory through a pinned staging buffer, the
initial states stay on the device for new conversations, each position's queue is copied into the
image's queue region and run by the executor with the host's copy of its bytes, and the logits
come back. The embedding lookup (bf16 -> fp32, exact; Gemma's fp32 scale) is done on the host from
the memory-mapped table, as the reference's runtime does, and only the rows cross to the device.
Every device step is the executor's, bit-identical to the golden model, so each step's logits are
the bits the reference's runtime gets on its golden backend.
"""
from __future__ import annotations

import ctypes
import json
import time
from pathlib import Path

import numpy as np
import torch

from . import _lib
from .contract import DESC_BYTES, ERR_NAMES
from .queue import _raise
from .ops import _device

STAGING = 64 << 20           # pinned staging buffer for reading image.bin


def _host_ptr(addr: int) -> ctypes.c_char_p:
    return ctypes.cast(ctypes.c_void_p(addr), ctypes.c_char_p)


def _run_queue(image: torch.Tensor, q: int, n: int, host_addr: int) -> tuple[int, int, int, int]:
    """n descriptors at image address q through tars_run_queue, their bytes also at host_addr:
    (done, err_code, op_idx, host_op). Raises on a refusal (an output over an input) or a device
    error."""
    st = _lib.QueueStatus()
    rc = _lib.lib().tars_run_queue(image.data_ptr(), image.numel(), q, n, _host_ptr(host_addr), 0, 0,
                                   ctypes.byref(st), torch.cuda.current_stream().cuda_stream)
    if rc != _lib.OK:
        _raise(rc)
    return int(st.done), int(st.err_code), int(st.op_idx), int(st.host_op)


class GpuDevice:
    """The board runtime's device on one MI355X (tars_board.py:4-12).

    mem: numpy uint8 view of a pinned host mirror of the device image [0, mem_bytes); to_dev(a, n)
    copies the mirror's bytes [a, a + n) to the device, from_dev(a, n) the device's to the mirror;
    run(q, n) runs the n descriptors the mirror holds at q (copied to the device before) on the
    device image and returns (done, err, op_idx, cycles), cycles 0 (the device keeps no cycle count).
    A descriptor the executor leaves to the host (a convolution: the language-model exports hold
    none) ends the run with done = 0 and err = 0 at its index."""
    # version: the firmware level whose features the executor covers (the W4A16 unit of v4.0, bit 0,
    # FP16 states and images over 1 GB): tars_board.Qwen checks an export's min_firmware against it
    params = dict(backend="mi355x executor", version=0x00040001)

    def __init__(self, mem_bytes: int = 1 << 30):
        dev = _device()
        self.image = torch.zeros(int(mem_bytes), dtype=torch.uint8, device=dev)
        self._host = torch.zeros(int(mem_bytes), dtype=torch.uint8, pin_memory=True)
        self.mem = self._host.numpy()

    def to_dev(self, a: int, n: int) -> None:
        self.image[a:a + n].copy_(self._host[a:a + n])

    def from_dev(self, a: int, n: int) -> None:
        self._host[a:a + n].copy_(self.image[a:a + n])

    def run(self, q: int, n: int, timeout=None):
        if q < 0 or q + DESC_BYTES * n > self.mem.size:
            raise ValueError("the queue lies outside the device buffer")
        done, err, op, _ = _run_queue(self.image, q, n, self._host.data_ptr() + q)
        return done, err, op, 0


def _read_into(path: Path, dst: torch.Tensor, log=None) -> None:
    """path's bytes into the device tensor dst (exactly its size) through a pinned staging buffer."""
    size = dst.numel()
    stage = torch.empty(min(STAGING, max(size, 1)), dtype=torch.uint8, pin_memory=True)
    view = memoryview(stage.numpy())
    pos = 0
    with open(path, "rb") as f:
        while pos < size:
            k = f.readinto(view[:min(stage.numel(), size - pos)])
            if not k:
                raise IOError(f"short read of {path}")
            dst[pos:pos + k].copy_(stage[:k])
            pos += k
            if log:
                log(f"\r  loading {path.name} {pos >> 20} / {size >> 20} MiB", end="")
    if log:
        log("")


class Model:
    """An export directory on one MI355X: the loader and runtime of tars_board.Qwen
    (tars_board.py:212-435) with the same methods, arguments and errors.

    step(token) -> logits (fp32 [vocab]) of the token at the next position; prefill(tokens,
    chunked) -> the logits after the last one, in prefill chunks where the export has a queue for
    the position (every chunk size it holds: the GPU's GEMMs take any number of rows) and single
    steps elsewhere; new_conversation(); encode(tokenizer, text, chat); the speculative decoding of
    an export with MTP queues (begin_spec, spec_round, end_spec, can_spec). self.seconds: host
    wall time of the last step / prefill / speculative round."""

    def __init__(self, data: str | Path, log=print):
        self.d = Path(data)
        m = json.loads((self.d / "manifest.json").read_text())
        self.m = m
        self.T, self.H, self.vocab = int(m["max_tokens"]), int(m["hidden"]), int(m["vocab"])
        t = time.time()
        img = self.d / "image.bin"
        size = img.stat().st_size
        if size != m["image_bytes"]:
            raise RuntimeError(f"{img}: {size} bytes, the manifest says {m['image_bytes']}")
        dev = _device()
        self.image = torch.empty(max(size, int(m.get("mem_bytes", size))), dtype=torch.uint8, device=dev)
        _read_into(img, self.image[:size], log)
        self.image[size:].zero_()
        self.state_end = int(m["state_end"])
        st = self.image[:self.state_end]
        self.state0 = st.clone() if bool(st.any()) else None
        self.embed = np.memmap(self.d / "embed_bf16.bin", np.uint16, "r", shape=(self.vocab, self.H))
        self.ple_cols = int(m.get("ple_cols", 0))
        self.ple = np.memmap(self.d / "ple_bf16.bin", np.uint16, "r", shape=(self.vocab, self.ple_cols)) \
            if self.ple_cols else None
        self.ple_scale = np.float32(m["ple_scale"]) if self.ple_cols else None
        self.qidx = np.asarray(m["queue_index"], np.int64)
        self.queues = np.memmap(self.d / "queues.bin", np.uint8, "r")
        self.chunks = {int(n): (np.memmap(self.d / f"queues_c{n}.bin", np.uint8, "r"),
                                {int(t0): (int(o), int(k)) for t0, o, k in index})
                       for n, index in m.get("chunks", {}).items() if (self.d / f"queues_c{n}.bin").exists()}
        self.spec = {n: (np.memmap(self.d / f"queues_s_{n}.bin", np.uint8, "r"),
                         {int(r): (int(o), int(k)) for r, o, k in index})
                     for n, index in m.get("spec", {}).items()}
        s = m.get("embed_scale")
        self.embed_scale = None if s is None else np.float32(s)
        self.bos = [int(v) for v in m.get("bos_ids", [])]
        self.turn_end = m.get("turn_end", "<|im_end|>\n")
        self.pos, self.par, self.mrow, self.draft = 0, 0, 0, None
        self.seconds = 0.0
        torch.cuda.synchronize()
        if log:
            log(f"  ready in {time.time() - t:.1f} s ({size >> 20} MiB image, {self.T} positions, "
                f"prefill chunks {sorted(self.chunks) or 'none'})")

    # ------------------------------------------------------------------ conversation state
    def new_conversation(self) -> None:
        if self.state0 is None:
            self.image[:self.state_end].zero_()
        else:
            self.image[:self.state_end].copy_(self.state0)
        self.pos, self.par, self.mrow, self.draft = 0, 0, 0, None

    def encode(self, tk, text: str, chat: bool = True) -> list[int]:
        """Token ids of `text` at the next position: in the export's chat template with `chat` (a
        later turn closes the model's turn first), the BOS tokens at position 0."""
        if chat:
            text = self.m["chat_prefix"] + text + self.m["chat_suffix"]
            if self.pos:
                text = self.turn_end + text
        return (self.bos if self.pos == 0 else []) + list(tk.encode(text, add_special_tokens=False).ids)

    # ------------------------------------------------------------------ device transfers
    def _write_rows(self, off: int, ld: int, rows: np.ndarray) -> None:
        rows = np.ascontiguousarray(rows, np.float32)
        nb = rows.shape[1] * 4
        src = torch.from_numpy(rows.view(np.uint8).reshape(rows.shape[0], nb))
        if ld == nb:
            self.image[off:off + rows.shape[0] * nb].copy_(src.reshape(-1))
        else:
            for i in range(rows.shape[0]):
                self.image[off + i * ld:off + i * ld + nb].copy_(src[i])

    def _put(self, t: int, tokens) -> None:
        """The embeddings of `tokens` into the input rows t, t + 1, ... (bf16 -> fp32 exactly; Gemma:
        times the manifest's embed_scale, one fp32 multiply)."""
        m = self.m
        if t + len(tokens) > self.T:
            raise OverflowError(f"context full ({self.T} tokens)")
        ids = np.asarray(tokens, np.int64)
        x = (self.embed[ids].astype(np.uint32) << 16).view(np.float32)
        if self.embed_scale is not None:
            x = (x * self.embed_scale).astype(np.float32)
        self._write_rows(int(m["x0_off"]) + t * int(m["x0_ld"]), int(m["x0_ld"]), x)
        if self.ple is not None:
            p = ((self.ple[ids].astype(np.uint32) << 16).view(np.float32) * self.ple_scale).astype(np.float32)
            self._write_rows(int(m["ple0_off"]) + t * int(m["ple0_ld"]), int(m["ple0_ld"]), p)

    def _run(self, queues: np.ndarray, off: int, n: int, what: str) -> None:
        """n descriptors from queues[off:], through the image's queue region in parts of at most
        queue_cap descriptors (the descriptors keep nothing from one part to the next)."""
        q, cap = int(self.m["qbase"]), int(self.m["queue_cap"])
        for s in range(0, n, cap):
            k = min(cap, n - s)
            part = np.array(queues[off + DESC_BYTES * s:off + DESC_BYTES * (s + k)])   # a writable copy
            self.image[q:q + part.size].copy_(torch.from_numpy(part))
            done, err, op, host_op = _run_queue(self.image, q, k, part.ctypes.data)
            if host_op:
                raise RuntimeError(f"{what}: descriptor {s + op} is a convolution, which this executor leaves "
                                   f"to a host")
            if not done or err:
                raise RuntimeError(f"{what}: the core stopped at descriptor {s + op} with error "
                                   f"{ERR_NAMES.get(err, err)}")

    def _logits(self) -> np.ndarray:
        lo = int(self.m["logits_off"])
        return self.image[lo:lo + 4 * self.vocab].cpu().numpy().view(np.float32).copy()

    def _rows(self, n: int) -> np.ndarray:
        """The logits rows [n, vocab] of a verify (each head block holds its n rows densely)."""
        lo = int(self.m["logits_off"])
        flat = self.image[lo:lo + 4 * self.vocab * n].cpu().numpy().view(np.float32)
        out, c0 = np.empty((n, self.vocab), np.float32), 0
        for b in self.m["head_blocks"]:
            out[:, c0:c0 + b] = flat[c0 * n:(c0 + b) * n].reshape(n, b)
            c0 += b
        return out

    # ------------------------------------------------------------------ decoding
    def step(self, token: int) -> np.ndarray:
        """`token` at the next position; returns the logits (fp32, vocab)."""
        t0 = time.perf_counter()
        t = self.pos
        self._put(t, [token])
        off, n = (int(v) for v in self.qidx[t])
        self._run(self.queues, off, n, f"position {t}")
        self.pos += 1
        lg = self._logits()
        self.seconds = time.perf_counter() - t0
        return lg

    def prefill(self, tokens, chunked: bool = True) -> np.ndarray:
        """`tokens` at the next positions; returns the logits after the last one. chunked: the
        largest chunk the export has a queue for at each position (bit-identical to one token at a
        time), single steps elsewhere; chunked=False: every token a step."""
        tokens = [int(v) for v in tokens]
        if not tokens:
            raise ValueError("no tokens")
        t_start = time.perf_counter()
        i, lg = 0, None
        while i < len(tokens):
            t = self.pos
            n = next((n for n in sorted(self.chunks, reverse=True)
                      if chunked and i + n <= len(tokens) and t in self.chunks[n][1]), 1)
            if n == 1:
                lg = self.step(tokens[i])
            else:
                self._put(t, tokens[i:i + n])
                queues, index = self.chunks[n]
                off, k = index[t]
                self._run(queues, off, k, f"positions {t}..{t + n - 1}")
                self.pos += n
                lg = None
            i += n
        lg = lg if lg is not None else self._logits()
        self.seconds = time.perf_counter() - t_start
        return lg

    # ------------------------------------------------------------------ speculative decoding (MTP exports)
    def _spec_run(self, name: str, r: int) -> None:
        queues, index = self.spec[name]
        off, k = index[r]
        self._run(queues, off, k, f"{name} at {r}")

    def begin_spec(self, lg: np.ndarray) -> int:
        """After a prefill with logits lg: the first new token (not yet in the cache); the MTP head
        takes the rows it has not seen and drafts the token after it."""
        t_start = time.perf_counter()
        cur = int(np.argmax(lg))
        t = self.pos
        self._put(t, [cur])
        while self.mrow < t - 1:
            n = 4 if self.mrow + 4 <= t - 1 and self.mrow in self.spec["mp4"][1] else 1
            self._spec_run(f"mp{n}", self.mrow)
            self.mrow += n
        self._spec_run("m1", t - 1)
        self.mrow = t
        self.draft = int(np.argmax(self._logits()))
        self.seconds = time.perf_counter() - t_start
        return cur

    def can_spec(self) -> bool:
        return self.pos + 3 <= self.T

    def spec_round(self, cur: int) -> tuple[list[int], np.ndarray]:
        """Verify [cur, draft] at the next position: the new tokens (2 on a hit, 1 on a miss; the last
        is not yet in the cache) and the verify's logits rows; the tokens of plain greedy decoding."""
        t_start = time.perf_counter()
        t, d = self.pos, self.draft
        self._put(t + 1, [d])
        self._spec_run(f"v2p{self.par}", t)
        rows = self._rows(2)
        x = int(np.argmax(rows[0]))
        if x == d and x not in self.m["eos_ids"]:
            y = int(np.argmax(rows[1]))
            self.par ^= 1
            self._put(t + 2, [y])
            self._spec_run("m2", t)
            self.pos, new = t + 2, [x, y]
        else:
            self._put(t + 1, [x])
            self._spec_run("m1", t)
            self.pos, new = t + 1, [x]
        self.mrow = self.pos
        self.draft = int(np.argmax(self._logits()))
        self.seconds = time.perf_counter() - t_start
        return new, rows

    def end_spec(self) -> None:
        """Back to the plain queues (they use the first state copy)."""
        if self.par:
            self._spec_run("swap", 0)
            self.par = 0


__all__ = ["GpuDevice", "Model"]
