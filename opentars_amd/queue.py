"""The descriptor-queue executor on MI355X, with the golden Machine's interface.

`Machine(ddr)` holds the DDR byte image in device memory and runs descriptor queues on it through
the C ABI's tars_run_queue (include/opentars_amd.h), the replacement of tars_mini/golden.py:41-62
(Machine: ddr, read, write) and :450-492 (run_queue -> Status). Descriptors are validated in the
contract's order on the host; every kind but a convolution runs on the GPU, in queue order,
bit-identical to the golden model: OP_GEMM (W8A8 QM_TENSOR / QM_CHANNEL / QM_ROWCOL and W4A16),
the row functions (ROW_QUANT, softmax, the norms), RELU, ELT, ROPE and FDOT.

A valid convolution (OP_CONV, OP_CONV_ACT) is not run here. Without a `host` the queue stops there
and the returned Status has host_op set. With a `host` -- a factory taking a host bytearray and
returning an object with a `ddr` image and a run_queue(addr, 1) that executes one descriptor on it,
e.g. the reference's own `tars_mini.golden.Machine` -- the image is copied to the host, that
descriptor runs there, the image is copied back and the GPU queue resumes. The language-model
lowering emits no convolutions. `run(ddr, q, n, host)` is the `run(ddr, q, n) -> bytes` seam of
QwenLowering.generate (tars_mini/llm.py:815-836).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Callable

import numpy as np
import torch

from . import _lib
from .contract import DESC_BYTES, ERR_NAMES
from .ops import ContractError, TarsError, _device


@dataclass
class Status:
    """golden.py:23-30, plus host_op: the queue stopped at a valid descriptor left to the host."""
    done: bool = False
    err_code: int = 0
    op_idx: int = 0
    host_op: bool = False

    def __str__(self) -> str:
        s = f"done={int(self.done)} err={ERR_NAMES.get(self.err_code, self.err_code)} op_idx={self.op_idx}"
        return s + (" host_op=1" if self.host_op else "")


def _raise(rc: int) -> None:
    msg = _lib.last_error()
    if rc == _lib.E_OVERLAP:
        raise ContractError(rc, msg)
    raise TarsError(rc, msg)


class Machine:
    """A DDR image in device memory and its descriptor queues (golden.py:41-62, 450-492).

    ddr: bytes-like (copied to the GPU) or a 1-D torch.uint8 tensor on the GPU (used in place).
    core_id / gemv_only: the executing core's CORE_ID and the KV260 profile (golden.py:43-50).
    host: optional factory host(bytearray) -> object with .ddr and run_queue(addr, n), for the
    descriptors the GPU does not run (see the module docstring).
    """

    def __init__(self, ddr, core_id: int = 0, gemv_only: bool = False,
                 host: Callable[[bytearray], object] | None = None):
        dev = _device()
        if isinstance(ddr, torch.Tensor):
            if ddr.dtype != torch.uint8 or ddr.dim() != 1 or not ddr.is_cuda or not ddr.is_contiguous():
                raise ValueError("a tensor image must be a contiguous 1-D torch.uint8 tensor on the GPU")
            self.image = ddr
        else:
            host_bytes = np.frombuffer(bytes(ddr) if not isinstance(ddr, (bytearray, np.ndarray)) else ddr, np.uint8)
            self.image = torch.from_numpy(host_bytes.copy()).to(dev)
        self.core_id, self.gemv_only, self.host = core_id, bool(gemv_only), host
        self.status = Status()

    # ------------------------------------------------------------------ memory
    @property
    def ddr(self) -> bytearray:
        """The image as host bytes (waits for the queued work)."""
        torch.cuda.synchronize()
        return bytearray(self.image.cpu().numpy().tobytes())

    def read(self, addr: int, n: int) -> bytes:
        torch.cuda.synchronize()
        return self.image[addr:addr + n].cpu().numpy().tobytes()

    def write(self, addr: int, data: bytes) -> None:
        self.image[addr:addr + len(data)] = torch.frombuffer(bytearray(data), dtype=torch.uint8).to(self.image.device)

    # ------------------------------------------------------------------ the queue
    def _gpu(self, queue_addr: int, n: int, descs: bytes | None = None) -> Status:
        st = _lib.QueueStatus()
        rc = _lib.lib().tars_run_queue(self.image.data_ptr(), self.image.numel(), queue_addr, n, descs, self.core_id,
                                       int(self.gemv_only), ctypes.byref(st), torch.cuda.current_stream().cuda_stream)
        if rc != _lib.OK:
            _raise(rc)
        return Status(bool(st.done), st.err_code, st.op_idx, bool(st.host_op))

    def _on_host(self, addr: int) -> Status:
        m = self.host(self.ddr)
        st = m.run_queue(addr, 1)
        after = np.frombuffer(bytes(m.ddr), np.uint8)         # the host machine's image after the descriptor
        if after.size != self.image.numel():
            raise ValueError("the host machine changed the image size")
        self.image.copy_(torch.from_numpy(after.copy()).to(self.image.device))
        return Status(bool(st.done), int(st.err_code), 0)

    def run_queue(self, queue_addr: int, queue_len: int, descs: bytes | None = None) -> Status:
        """Runs queue_len descriptors at queue_addr in order; the GPU work is stream-ordered on the
        current stream (read the image through .ddr / .read, which synchronize). An output that
        overlaps an input raises ContractError, as the golden does. descs: optionally the caller's
        host copy of the queue's bytes (then the call does not wait to read them from the image)."""
        base = 0
        while True:
            part = None if descs is None else descs[DESC_BYTES * base:DESC_BYTES * queue_len]
            st = self._gpu(queue_addr + DESC_BYTES * base, queue_len - base, part)
            st.op_idx += base
            if st.done or not st.host_op or self.host is None:
                self.status = st
                return st
            hs = self._on_host(queue_addr + DESC_BYTES * st.op_idx)
            descs = None                                      # the host step may have rewritten the queue
            if not hs.done:
                self.status = Status(False, hs.err_code, st.op_idx)
                return self.status
            base = st.op_idx + 1
            if base == queue_len:
                self.status = Status(True, 0, queue_len)
                return self.status


def run(ddr, q: int, n: int, host: Callable[[bytearray], object] | None = None, core_id: int = 0,
        gemv_only: bool = False) -> bytearray:
    """The executor seam of QwenLowering.generate (llm.py:815-836): runs the queue and returns the
    image bytes. Raises RuntimeError when the queue does not complete."""
    m = Machine(ddr, core_id=core_id, gemv_only=gemv_only, host=host)
    st = m.run_queue(q, n)
    if not st.done:
        raise RuntimeError(f"queue stopped: {st}")
    return m.ddr


def check_descriptor(desc: bytes, image_len: int, core_id: int = 0, gemv_only: bool = False) -> tuple[int, bool]:
    """(ERR_CODE, runs on the GPU) of one 64-byte descriptor against an image of image_len bytes
    (host only). Raises ContractError when a valid descriptor's output overlaps an input."""
    if len(desc) != DESC_BYTES:
        raise ValueError("a descriptor is 64 bytes")
    err, gpu = ctypes.c_int32(), ctypes.c_int32()
    rc = _lib.lib().tars_check_descriptor(bytes(desc), image_len, core_id, int(gemv_only), ctypes.byref(err),
                                          ctypes.byref(gpu))
    if rc != _lib.OK:
        _raise(rc)
    return err.value, bool(gpu.value)


def decode_descriptor(desc: bytes) -> list[int]:
    """The 23 field values of a 64-byte descriptor in layout order (host only)."""
    out = (ctypes.c_uint64 * 23)()
    rc = _lib.lib().tars_decode_descriptor(bytes(desc), out)
    if rc != _lib.OK:
        _raise(rc)
    return list(out)


def descriptor_crc(desc: bytes) -> int:
    return int(_lib.lib().tars_descriptor_crc(bytes(desc)))


FIELDS = ("MAGIC", "VERSION", "CORE_ID", "HDR_RSV", "OPCODE", "CTRL", "GROUP_SIZE", "EPI", "BASE_ADDR", "A_OFF",
          "W_OFF", "Y_OFF", "SCALE_OFF", "BIAS_OFF", "M", "N", "K", "LDA16", "OUT_SCALE", "CRC32", "VALID", "LDY16",
          "DEP_SIG")


def encode_descriptor(fields: dict, fix_crc: bool = True) -> bytes:
    """A 64-byte descriptor from field values by name (absent fields are 0), its CRC fixed
    (contract.py:154-167 encode). Host only."""
    unknown = set(fields) - set(FIELDS)
    if unknown:
        raise ValueError(f"unknown descriptor fields {sorted(unknown)}")
    vals = (ctypes.c_uint64 * 23)(*[int(fields.get(n, 0)) for n in FIELDS])
    out = ctypes.create_string_buffer(DESC_BYTES)
    rc = _lib.lib().tars_encode_descriptor(vals, int(fix_crc), out)
    if rc != _lib.OK:
        _raise(rc)
    return out.raw


def set_fusion(on: bool) -> bool:
    """Peephole fusion of decode-row ROW_QUANT + its QM_ROWCOL GEMMs in run_queue (default on);
    returns the previous setting."""
    return bool(_lib.lib().tars_set_queue_fusion(int(on)))


FUSION_KINDS = ("quant_gemm", "attention", "add_norm", "norm_rope", "gated_mlp", "norm_rope_two", "norm_quant",
                "rope_attention")


def fusion_counts(reset: bool = False) -> dict:
    """Fused launches run_queue has run since the last reset, per kind (FUSION_KINDS). A gated_mlp
    launch (an MLP's ELT MUL folded into its gate / up GEMMs) and a norm_quant launch (a norm, and
    the residual add before it, run in front of a quantizer group) also count as quant_gemm;
    norm_rope counts (norm, RoPE) pairs and norm_rope_two the launches that ran two of them; a
    rope_attention launch (an attention whose scores kernel ran the layer's q and k norm + RoPE pairs)
    also counts as attention and as two norm_rope pairs. A
    replayed launch plan counts its fused launches again. Diagnostics for tests and benchmarks."""
    arr = (ctypes.c_int64 * len(FUSION_KINDS))()
    _lib.lib().tars_queue_fusion_counts(arr, len(FUSION_KINDS), int(reset))
    return dict(zip(FUSION_KINDS, (int(v) for v in arr)))


def set_graphs(on: bool) -> bool:
    """Launch plans replayed as HIP graphs for repeated queues in run_queue (default on); returns
    the previous setting. Turning it off drops the kept plans."""
    return bool(_lib.lib().tars_set_queue_graphs(int(on)))


__all__ = ["Machine", "Status", "run", "check_descriptor", "decode_descriptor", "descriptor_crc", "fusion_counts",
           "encode_descriptor", "set_fusion", "set_graphs", "FIELDS", "ERR_NAMES"]
