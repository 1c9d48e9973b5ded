"""Board exports on one MI355X: a device with the board runtime's interface, and a model runtime
of its own design that keeps a whole export resident in HBM.

An export (tools/export_kv260.py:13-32, 141-247) is a directory: image.bin (the DDR image from
address 0: zeroed states, the queue region, scratch, quantized weights), embed_bf16.bin (the input
embedding table [vocab, hidden] as bf16), ple_bf16.bin (Gemma 4's per-layer embeddings),
queues.bin (one descriptor queue per token position), queues_c<n>.bin (prefill chunks of n
tokens), queues_s_<name>.bin (speculative decoding with an MTP head) and manifest.json.

GpuDevice is a device of the board runtime's interface (deploy/kv260/sw/tars_board.py:4-12:
mem, to_dev, from_dev, run(q, n) -> (done, err, op_idx, cycles)) over the library's executor.

Model runs an export with everything on the device. What crosses PCIe per step is the token ids
(kernel arguments of the embedding lookup), the descriptors' host copy the executor decodes (it
never copies them back), and the logits:

  ExportLayout  the manifest, parsed once into typed fields.
  QueueStore    every queue file in one HBM buffer, read once at load; each schedule entry (the
                queue of a position, a prefill chunk, a speculative step) is precomputed as its
                executor runs: parts of at most queue_cap descriptors, each a device-to-device copy
                into the image's queue region and one tars_run_queue.
  TokenRows     the bf16 embedding tables resident in HBM; a token's fp32 input rows are written
                into the image by tars_embed_rows (the bf16 -> fp32 shift and Gemma's one fp32
                multiply, as the board runtime computes them on its host, tars_board.py:298-314).
  Speculation   the state of MTP speculative decoding as one object: which state copy the verify
                queues read, how far the MTP head has consumed the cache, and its current draft.
  Model         schedules the entries: a step, a prefill covered greedily by the longest chunk
                queue the export holds at each position, the MTP rounds. The export's queue
                protocol (which queue runs at which position, and the verify / accept / reject
                sequence of a speculative round) is the export's own and is followed as
                tars_board.Qwen (tars_board.py:212-435) defines it; each step's logits are the bits
                the reference's runtime gets on its golden backend.
"""
from __future__ import annotations

import ctypes
import json
import time
from dataclasses import dataclass
from pathlib import Path
from typing import Iterable, NamedTuple

import numpy as np
import torch

from . import _lib
from .contract import DESC_BYTES, ERR_NAMES
from .ops import _check, _device
from .queue import _raise

STAGING = 64 << 20           # pinned staging buffer for reading files into device memory
# The executor's feature level, in the board firmware's numbering (the W4A16 unit of v4.0, FP16
# states, images over 1 GB): an export whose min_firmware is above it is refused.
EXECUTOR_LEVEL = 0x00040001


def _run_queue(image: torch.Tensor, q: int, n: int, host_addr: int) -> tuple[int, int, int, int]:
    """n descriptors at image address q through tars_run_queue, their bytes also at host_addr:
    (done, err_code, op_idx, host_op). Raises on a refusal (an output over an input) or a device
    error."""
    st = _lib.QueueStatus()
    rc = _lib.lib().tars_run_queue(image.data_ptr(), image.numel(), q, n,
                                   ctypes.cast(ctypes.c_void_p(host_addr), ctypes.c_char_p), 0, 0,
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
    params = dict(backend="mi355x executor", version=EXECUTOR_LEVEL)

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


def _load(path: Path, dst: torch.Tensor, stage: torch.Tensor, log=None) -> None:
    """The file's bytes into the device tensor dst (exactly its size) through the pinned stage."""
    size, pos = dst.numel(), 0
    view = memoryview(stage.numpy())
    with open(path, "rb") as f:
        while pos < size:
            k = f.readinto(view[:min(stage.numel(), size - pos)])
            if not k:
                raise IOError(f"short read of {path}")
            dst[pos:pos + k].copy_(stage[:k])            # synchronous: the stage is free again after it
            pos += k
            if log:
                log(f"\r  loading {path.name} {pos >> 20} / {size >> 20} MiB", end="")
    if log:
        log("")


# ---------------------------------------------------------------------------------- layout
@dataclass(frozen=True)
class ExportLayout:
    """The manifest's fields the runtime uses (tools/export_kv260.py:248-295 writes them)."""
    positions: int                 # max_tokens
    hidden: int
    vocab: int
    image_bytes: int
    mem_bytes: int                 # the device image's size (>= image_bytes)
    state_end: int                 # [0, state_end): the conversation state (KV caches, DeltaNet states)
    qbase: int                     # the image's queue region
    queue_cap: int                 # descriptors it holds
    x0: tuple[int, int]            # input rows: (offset, row stride)
    ple: tuple[int, int, int] | None   # per-layer embedding rows: (offset, row stride, columns)
    embed_scale: float | None
    ple_scale: float | None
    logits: int                    # logits offset
    head_blocks: tuple[int, ...]   # the head's row blocks (a verify's rows are dense per block)
    bos: tuple[int, ...]
    eos: frozenset
    turn_end: str
    chat: tuple[str, str]          # chat template: (prefix, suffix)
    min_firmware: int

    @staticmethod
    def parse(m: dict) -> "ExportLayout":
        ple_cols = int(m.get("ple_cols", 0))
        level = int(m.get("min_firmware", 0))
        if m.get("state_dtype") == "fp16":
            level = max(level, 0x30400)         # FP16 states need firmware 3.4
        es = m.get("embed_scale")
        return ExportLayout(
            positions=int(m["max_tokens"]), hidden=int(m["hidden"]), vocab=int(m["vocab"]),
            image_bytes=int(m["image_bytes"]), mem_bytes=max(int(m["image_bytes"]), int(m.get("mem_bytes", 0))),
            state_end=int(m["state_end"]), qbase=int(m["qbase"]), queue_cap=int(m["queue_cap"]),
            x0=(int(m["x0_off"]), int(m["x0_ld"])),
            ple=(int(m["ple0_off"]), int(m["ple0_ld"]), ple_cols) if ple_cols else None,
            embed_scale=None if es is None else float(es),
            ple_scale=float(m["ple_scale"]) if ple_cols else None,
            logits=int(m["logits_off"]), head_blocks=tuple(int(b) for b in m["head_blocks"]),
            bos=tuple(int(v) for v in m.get("bos_ids", [])), eos=frozenset(int(v) for v in m.get("eos_ids", [])),
            turn_end=m.get("turn_end", "<|im_end|>\n"),
            chat=(m.get("chat_prefix", ""), m.get("chat_suffix", "")), min_firmware=level)


# ---------------------------------------------------------------------------------- queues
class Run(NamedTuple):
    """One tars_run_queue call: `count` descriptors at byte `src` of the store, the first of them
    descriptor `first` of its schedule entry; `host` is their bytes for the executor to decode."""
    src: int
    count: int
    first: int
    host: np.ndarray


class QueueStore:
    """The export's queue files in one HBM buffer, and the runs of every schedule entry.

    books: name -> (file name, [(key, byte offset, descriptors), ...]). An entry (name, key)
    becomes ceil(descriptors / queue_cap) runs (a queue longer than the image's queue region runs
    in parts; the descriptors keep nothing from one part to the next)."""

    def __init__(self, d: Path, books: dict, cap: int, stage: torch.Tensor, log=None):
        files = sorted({f for f, _ in books.values()})
        base, total = {}, 0
        for f in files:
            base[f] = total
            total += ((d / f).stat().st_size + 255) // 256 * 256
        self.dev = torch.empty(max(total, 1), dtype=torch.uint8, device=_device())
        host = {}
        for f in files:
            size = (d / f).stat().st_size
            _load(d / f, self.dev[base[f]:base[f] + size], stage, log)
            host[f] = np.fromfile(d / f, np.uint8)          # read-only bytes for the executor
        self._runs: dict[tuple[str, int], tuple[Run, ...]] = {}
        self._keys: dict[str, frozenset] = {}
        for name, (f, index) in books.items():
            keys = []
            for key, off, n in index:
                off, n = int(off), int(n)
                self._runs[(name, int(key))] = tuple(
                    Run(base[f] + off + DESC_BYTES * s, min(cap, n - s), s,
                        host[f][off + DESC_BYTES * s:off + DESC_BYTES * (s + min(cap, n - s))])
                    for s in range(0, n, cap))
                keys.append(int(key))
            self._keys[name] = frozenset(keys)

    def keys(self, name: str) -> frozenset:
        return self._keys.get(name, frozenset())

    def runs(self, name: str, key: int) -> tuple[Run, ...]:
        return self._runs[(name, key)]


def cover(start: int, stop: int, sizes_at) -> list[tuple[int, int]]:
    """Positions [start, stop) as consecutive (position, length) runs: at each position the largest
    length sizes_at(position) offers that still fits, else 1 (a single step)."""
    out, t = [], start
    while t < stop:
        n = max((s for s in sizes_at(t) if t + s <= stop), default=1)
        out.append((t, n))
        t += n
    return out


# ---------------------------------------------------------------------------------- token rows
class TokenRows:
    """The input embedding table (and Gemma 4's per-layer embedding table) resident in HBM; write()
    puts the fp32 rows of token ids into the image's input rows on the device."""

    def __init__(self, d: Path, lay: ExportLayout, stage: torch.Tensor, log=None):
        self.lay = lay
        dev = _device()
        self.embed = torch.empty((lay.vocab, lay.hidden), dtype=torch.int16, device=dev)
        _load(d / "embed_bf16.bin", self.embed.view(torch.uint8).view(-1), stage, log)
        self.ple = None
        if lay.ple is not None:
            self.ple = torch.empty((lay.vocab, lay.ple[2]), dtype=torch.int16, device=dev)
            _load(d / "ple_bf16.bin", self.ple.view(torch.uint8).view(-1), stage, log)

    @staticmethod
    def _gather(table: torch.Tensor, ids: np.ndarray, scale, dst: int, ld: int) -> None:
        bits = 0 if scale is None else int(np.float32(scale).view(np.uint32))
        _check(_lib.lib().tars_embed_rows(table.data_ptr(), 2 * table.shape[1], table.shape[0], table.shape[1],
                                          ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), ids.size,
                                          int(scale is not None), bits, dst, ld,
                                          torch.cuda.current_stream().cuda_stream))

    def write(self, image: torch.Tensor, pos: int, tokens: Iterable[int]) -> None:
        wide = np.fromiter((int(t) for t in tokens), np.int64)
        if wide.size and (wide.min() < 0 or wide.max() >= self.lay.vocab):
            bad = wide[(wide < 0) | (wide >= self.lay.vocab)][0]
            raise IndexError(f"token id {bad} is outside the vocabulary of {self.lay.vocab} rows")
        ids = np.ascontiguousarray(wide, np.int32)
        if pos + ids.size > self.lay.positions:
            raise OverflowError(f"context full ({self.lay.positions} tokens)")
        off, ld = self.lay.x0
        self._gather(self.embed, ids, self.lay.embed_scale, image.data_ptr() + off + pos * ld, ld)
        if self.ple is not None:
            off, ld, _ = self.lay.ple
            self._gather(self.ple, ids, self.lay.ple_scale, image.data_ptr() + off + pos * ld, ld)


# ---------------------------------------------------------------------------------- model
@dataclass
class Speculation:
    """MTP speculative decoding state. parity: which of the two state copies the verify queue of
    the next round reads (v2p0 / v2p1); an accepted draft leaves its update in the other copy, so
    parity flips. seen: the positions below it have been consumed by the MTP head. draft: the MTP
    head's proposal for the token after the current one."""
    parity: int = 0
    seen: int = 0
    draft: int | None = None


class Model:
    """An export directory run on one MI355X, with the board runtime's methods (tars_board.Qwen:
    step, prefill, new_conversation, encode, begin_spec / spec_round / end_spec / can_spec) and
    their results and errors.

    step(token) -> logits (fp32 [vocab]) of `token` at the next position; prefill(tokens, chunked)
    -> the logits after the last token, the positions covered by the longest prefill-chunk queue
    the export holds at each position (any number of rows runs on the GPU's GEMMs) and single steps
    elsewhere (bit-identical either way). self.seconds: host wall time of the last call."""

    def __init__(self, data: str | Path, log=print):
        t_start = time.time()
        self.d = Path(data)
        self.manifest = json.loads((self.d / "manifest.json").read_text())
        lay = self.lay = ExportLayout.parse(self.manifest)
        if lay.min_firmware > EXECUTOR_LEVEL:
            raise RuntimeError(f"export requires firmware >= 0x{lay.min_firmware:08x}; the executor "
                               f"covers 0x{EXECUTOR_LEVEL:08x}")
        self.T, self.H, self.vocab = lay.positions, lay.hidden, lay.vocab
        img = self.d / "image.bin"
        if img.stat().st_size != lay.image_bytes:
            raise RuntimeError(f"{img}: {img.stat().st_size} bytes, the manifest says {lay.image_bytes}")
        dev = _device()                       # raises first when there is no GPU
        stage = torch.empty(STAGING, dtype=torch.uint8, pin_memory=True)
        self.image = torch.zeros(lay.mem_bytes, dtype=torch.uint8, device=dev)
        _load(img, self.image[:lay.image_bytes], stage, log)
        state = self.image[:lay.state_end]
        self._state0 = state.clone() if bool(state.any()) else None   # None: the state starts zeroed

        m = self.manifest
        books = {"pos": ("queues.bin", [(t, off, n) for t, (off, n) in enumerate(m["queue_index"])])}
        for n, index in m.get("chunks", {}).items():
            if (self.d / f"queues_c{n}.bin").exists():
                books[f"c{int(n)}"] = (f"queues_c{n}.bin", index)
        for name, index in m.get("spec", {}).items():
            books[f"s:{name}"] = (f"queues_s_{name}.bin", index)
        self.store = QueueStore(self.d, books, lay.queue_cap, stage, log)
        self.chunk_sizes = sorted(int(k[1:]) for k in books if k[0] == "c")
        self._chunks_at = {}
        for n in self.chunk_sizes:
            for t in self.store.keys(f"c{n}"):
                self._chunks_at.setdefault(t, []).append(n)
        self.rows = TokenRows(self.d, lay, stage, log)
        del stage
        self.pos = 0
        self.spec = Speculation()
        self.seconds = 0.0
        torch.cuda.synchronize()
        if log:
            log(f"  ready in {time.time() - t_start:.1f} s ({lay.image_bytes >> 20} MiB image, {self.T} positions, "
                f"prefill chunks {self.chunk_sizes or 'none'})")

    # ------------------------------------------------------------------ device work
    def _execute(self, book: str, key: int, what: str) -> None:
        """The schedule entry's runs through the executor, in order; raises where the core stops."""
        q = self.lay.qbase
        for r in self.store.runs(book, key):
            nb = DESC_BYTES * r.count
            self.image[q:q + nb].copy_(self.store.dev[r.src:r.src + nb])
            done, err, op, host_op = _run_queue(self.image, q, r.count, r.host.ctypes.data)
            if host_op:
                raise RuntimeError(f"{what}: descriptor {r.first + op} is a convolution, which this "
                                   f"executor leaves to a host")
            if not done or err:
                raise RuntimeError(f"{what}: the core stopped at descriptor {r.first + op} with error "
                                   f"{ERR_NAMES.get(err, err)}")

    def _logits(self) -> np.ndarray:
        lo = self.lay.logits
        return self.image[lo:lo + 4 * self.vocab].view(torch.float32).cpu().numpy()

    def _verify_rows(self, n: int) -> np.ndarray:
        """The logits rows [n, vocab] of an n-token verify: each head block holds its n rows
        densely, one after the other; the blocks are put side by side on the device."""
        lo = self.lay.logits
        flat = self.image[lo:lo + 4 * self.vocab * n].view(torch.float32)
        parts, c0 = [], 0
        for b in self.lay.head_blocks:
            parts.append(flat[c0 * n:(c0 + b) * n].view(n, b))
            c0 += b
        return torch.cat(parts, dim=1).cpu().numpy()

    # ------------------------------------------------------------------ conversation
    def new_conversation(self) -> None:
        state = self.image[:self.lay.state_end]
        if self._state0 is None:
            state.zero_()
        else:
            state.copy_(self._state0)
        self.pos = 0
        self.spec = Speculation()

    def encode(self, tk, text: str, chat: bool = True) -> list[int]:
        """Token ids of `text` at the next position: in the export's chat template with `chat`
        (a turn after the first closes the model's turn first), the BOS tokens at position 0."""
        if chat:
            prefix, suffix = self.lay.chat
            text = (self.lay.turn_end if self.pos else "") + prefix + text + suffix
        lead = list(self.lay.bos) if self.pos == 0 else []
        return lead + list(tk.encode(text, add_special_tokens=False).ids)

    # ------------------------------------------------------------------ decoding
    def _timed(self, t0: float, value):
        self.seconds = time.perf_counter() - t0
        return value

    def step(self, token: int) -> np.ndarray:
        """`token` at the next position; returns the logits (fp32, vocab)."""
        t0 = time.perf_counter()
        self.rows.write(self.image, self.pos, [token])
        self._execute("pos", self.pos, f"position {self.pos}")
        self.pos += 1
        return self._timed(t0, self._logits())

    def prefill(self, tokens, chunked: bool = True) -> np.ndarray:
        """`tokens` at the next positions; returns the logits after the last one. chunked: each
        position covered by the longest chunk queue the export holds there that fits (bit-identical
        to single steps); chunked=False: every token a step."""
        tokens = [int(v) for v in tokens]
        if not tokens:
            raise ValueError("no tokens")
        t0 = time.perf_counter()
        start = self.pos
        if start + len(tokens) > self.T:
            raise OverflowError(f"context full ({self.T} tokens)")
        sizes = (lambda t: self._chunks_at.get(t, ())) if chunked else (lambda t: ())
        for t, n in cover(start, start + len(tokens), sizes):
            self.rows.write(self.image, t, tokens[t - start:t - start + n])
            if n == 1:
                self._execute("pos", t, f"position {t}")
            else:
                self._execute(f"c{n}", t, f"positions {t}..{t + n - 1}")
            self.pos = t + n
        return self._timed(t0, self._logits())

    # ------------------------------------------------------------------ speculative decoding (MTP exports)
    @property
    def draft(self) -> int | None:
        return self.spec.draft

    def _mtp(self, name: str, t: int) -> None:
        self._execute(f"s:{name}", t, f"{name} at {t}")

    def _redraft(self) -> None:
        self.spec.seen = self.pos
        self.spec.draft = int(np.argmax(self._logits()))

    def begin_spec(self, lg: np.ndarray) -> int:
        """After a prefill with logits lg: the first new token (written at the next position, not
        yet run). The MTP head consumes the cache rows it has not seen (in runs of 4 where the
        export has that queue) and the last one with that token, and drafts the token after it."""
        t0 = time.perf_counter()
        cur = int(np.argmax(lg))
        t = self.pos
        self.rows.write(self.image, t, [cur])
        four = self.store.keys("s:mp4")
        for r, n in cover(self.spec.seen, t - 1, lambda r: (4,) if r in four else ()):
            self._mtp(f"mp{n}", r)
        self._mtp("m1", t - 1)
        self._redraft()
        return self._timed(t0, cur)

    def can_spec(self) -> bool:
        """Room for a verify of two tokens and the MTP step after it."""
        return self.pos + 3 <= self.T

    def spec_round(self, cur: int) -> tuple[list[int], np.ndarray]:
        """Verify [cur, draft] at the next position. Returns the new tokens and the verify's logits
        rows [2, vocab]: on a hit (the model's own next token is the draft, and not an end token)
        two tokens, else one; the last is written at its position but not yet run. The tokens are
        those of plain greedy decoding."""
        t0 = time.perf_counter()
        t, sp = self.pos, self.spec
        self.rows.write(self.image, t + 1, [sp.draft])
        self._mtp(f"v2p{sp.parity}", t)
        rows = self._verify_rows(2)
        best = [int(v) for v in rows.argmax(axis=1)]
        hit = best[0] == sp.draft and best[0] not in self.lay.eos
        new = best if hit else best[:1]
        if hit:
            sp.parity ^= 1                   # the verify's update of the draft row is the state now
        self.rows.write(self.image, t + len(new), [new[-1]])
        self._mtp("m2" if hit else "m1", t)
        self.pos = t + len(new)
        self._redraft()
        return self._timed(t0, (new, rows))

    def end_spec(self) -> None:
        """Back to the plain queues, which read the first state copy."""
        if self.spec.parity:
            self._mtp("swap", 0)
            self.spec.parity = 0


__all__ = ["GpuDevice", "Model", "ExportLayout", "QueueStore", "TokenRows", "Speculation", "cover"]
