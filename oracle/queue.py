"""The golden model's descriptor contract and queue walk, restated -- TEST INFRASTRUCTURE ONLY.

  LAYOUT / encode / decode / crc_ok   the 512-bit descriptor               contract.py:14-38,154-181
  validate                            checks in the contract's order       golden.py:59-169
  strides / bstride / segments        row strides and byte segments        golden.py:172-248
  extra_out, overlaps, in_place       ROW_QUANT scales, overlap rules      golden.py:250-267,440-448
  Machine.run_queue                   in-order execution and end status    golden.py:450-492

The executor here runs the descriptors the GPU library runs (OP_GEMM: W8A8 in QM_TENSOR /
QM_CHANNEL / QM_ROWCOL and W4A16; OP_ROW: softmax, causal softmax, LayerNorm, RMSNorm, L2Norm and
ROW_QUANT; OP_RELU; OP_ELT; OP_ROPE; OP_FDOT) through the oracle's arithmetic, and stops at a
valid convolution descriptor with `host_op` set, exactly as the GPU executor hands such
descriptors back. It is the reference the GPU queue executor is compared with, byte for byte and
status for status; only the tests may import it.

Pinning: the layout, codec and CRC by the contract document's worked example (descriptor bytes
and CRC 0x3784C47F, tests/test_contract.py:12-14,47-84) and the reference's round-trip and bit-flip
tests; the validation order by the reference's error-code tables (test_golden.py:92-136,
test_v04.py:175-211, test_w4a16.py:182-216) transcribed as data into
tests/golden/descriptor_cases.json; the segment and range rules by the reference's own range
cases (test_golden.py:113-115, test_w4a16.py:219-238) and by brute force (a byte-map of every
segment) on random descriptors.
"""
from __future__ import annotations

import bisect
import struct
import zlib
from dataclasses import dataclass

import numpy as np

from . import golden as G
from . import numerics as F
from . import rowops as R

LAYOUT = {
    "MAGIC": (511, 496), "VERSION": (495, 480), "CORE_ID": (479, 472), "HDR_RSV": (471, 448),
    "OPCODE": (447, 432), "CTRL": (431, 416), "GROUP_SIZE": (415, 400), "EPI": (399, 384),
    "BASE_ADDR": (383, 320), "A_OFF": (319, 288), "W_OFF": (287, 256), "Y_OFF": (255, 224),
    "SCALE_OFF": (223, 192), "BIAS_OFF": (191, 160), "M": (159, 144), "N": (143, 128),
    "K": (127, 112), "LDA16": (111, 96), "OUT_SCALE": (95, 64), "CRC32": (63, 32),
    "VALID": (31, 31), "LDY16": (30, 16), "DEP_SIG": (15, 0),
}
FIELDS = list(LAYOUT)
DESC_BYTES = 64
MAGIC, VERSION = 0xAA55, 0x0002
OP_CONV, OP_GEMM, OP_RELU, OP_ROW, OP_CONV_ACT, OP_ELT, OP_ROPE, OP_FDOT = 1, 2, 3, 4, 5, 6, 7, 8
CONV_OPS, V04_OPS = (OP_CONV, OP_CONV_ACT), (OP_ELT, OP_ROPE, OP_FDOT)
QM_NONE, QM_TENSOR, QM_CHANNEL, QM_ROWCOL = 0, 1, 2, 3
QM_GROUP = QM_ROWCOL
DT_BF16, DT_INT8, DT_INT4, DT_FP8, DT_FP32 = 0, 1, 2, 3, 4
OUT_FP32, OUT_BF16, OUT_INT8, OUT_FP16 = 0, 1, 2, 3
ESIZE = {OUT_FP32: 4, OUT_BF16: 2, OUT_INT8: 1, OUT_FP16: 2}
ROW_SOFTMAX, ROW_LAYERNORM, ROW_RMSNORM, ROW_L2NORM, ROW_QUANT = 0, 1, 2, 3, 4
ELT_MUL, ELT_ADD, ELT_MULADD, ELT_SUB = 0, 1, 2, 3
BM_DENSE, BM_ROW, BM_COL, BM_SCALAR = 0, 1, 2, 3
STATE_FP16 = 1 << 3
W4_GROUP = 128
E_OK, E_MAGIC, E_VERSION, E_CRC, E_VALID, E_OPCODE, E_FIELD, E_ALIGN, E_RANGE = range(9)


class ContractError(Exception):
    """An output overlaps an input (golden.py:17-18, 473-479)."""


def ctrl(qmode=QM_TENSOR, symmetric=1, a_dtype=DT_INT8, w_dtype=DT_INT8, fusion=0) -> int:
    """CTRL bits (contract.py:121-124): qmode[2:0] sym[3] a_dtype[7:4] w_dtype[11:8] fusion[12]."""
    return (qmode & 7) | (symmetric & 1) << 3 | (a_dtype & 15) << 4 | (w_dtype & 15) << 8 | (fusion & 1) << 12


def epi(act=0, out=OUT_FP32, bias=0) -> int:
    """EPI bits (contract.py:127-133): act[1:0] out[3:2] bias[4] act[2] at bit 5."""
    return (act & 3) | (out & 3) << 2 | (bias & 1) << 4 | (act >> 2 & 1) << 5


def act_of(e: int) -> int:
    return (e & 3) | (e >> 5 & 1) << 2


def crc(raw: bytes) -> int:
    z = bytearray(raw)
    z[4:8] = b"\0\0\0\0"
    return zlib.crc32(bytes(z)) & 0xFFFFFFFF


def encode(fields: dict, fix_crc: bool = True) -> bytes:
    """64 little-endian bytes, byte i = bits 8i+7..8i; the CRC over the bytes with 4..7 zeroed."""
    v = 0
    for name, val in fields.items():
        hi, lo = LAYOUT[name]
        if not 0 <= val < 1 << (hi - lo + 1):
            raise ValueError(f"{name}={val} does not fit")
        v |= val << lo
    raw = bytearray(v.to_bytes(DESC_BYTES, "little"))
    if fix_crc:
        raw[4:8] = struct.pack("<I", crc(bytes(raw)))
    return bytes(raw)


def decode(raw: bytes) -> dict:
    v = int.from_bytes(raw, "little")
    return {n: (v >> lo) & ((1 << (hi - lo + 1)) - 1) for n, (hi, lo) in LAYOUT.items()}


def crc_ok(raw: bytes) -> bool:
    return struct.unpack("<I", raw[4:8])[0] == crc(raw)


def conv_params(d: dict) -> dict:
    """contract.py:62-72: H, W, KH, KW, stride, pad from HDR_RSV / GROUP_SIZE; Cin, OH, OW."""
    g = d["HDR_RSV"]
    h, kh, kw, s, p, w = g >> 12, g >> 8 & 15, g >> 4 & 15, (g >> 2 & 3) + 1, g & 3, d["GROUP_SIZE"]
    cin = d["K"] // (kh * kw) if kh and kw else 0
    return dict(H=h, W=w, KH=kh, KW=kw, S=s, P=p, Cin=cin, OH=(h + 2 * p - kh) // s + 1,
                OW=(w + 2 * p - kw) // s + 1)


def is_w4(d: dict) -> bool:
    return d["OPCODE"] == OP_GEMM and d["CTRL"] & 7 == QM_GROUP and d["CTRL"] >> 8 & 15 == DT_INT4


def validate(raw: bytes, core_id: int = 0, gemv_only: bool = False) -> tuple[int, dict]:
    """golden.py:59-169."""
    d = decode(raw)
    if d["MAGIC"] != MAGIC:
        return E_MAGIC, d
    if d["VERSION"] != VERSION:
        return E_VERSION, d
    if not crc_ok(raw):
        return E_CRC, d
    if d["VALID"] != 1:
        return E_VALID, d
    op = d["OPCODE"]
    if op not in (OP_GEMM, OP_RELU, OP_ROW) + CONV_OPS + V04_OPS:
        return E_OPCODE, d
    if gemv_only and (op in CONV_OPS or (op == OP_GEMM and d["K"] > 4096)):
        return E_OPCODE, d
    conv = op in CONV_OPS
    c, e = d["CTRL"], d["EPI"]
    qmode, sym, adt, wdt, fus = c & 7, c >> 3 & 1, c >> 4 & 15, c >> 8 & 15, c >> 12 & 1
    act, out, bias = act_of(e), e >> 2 & 3, e >> 4 & 1
    w4 = is_w4(d)
    hdr_ok = conv or (op == OP_GEMM and qmode == QM_ROWCOL and not w4) \
        or (op == OP_ELT and d["HDR_RSV"] < 16) or (op == OP_FDOT and c & 1 and d["HDR_RSV"] == STATE_FP16)
    grp_ok = conv or op in V04_OPS or w4
    if d["CORE_ID"] != core_id or d["DEP_SIG"] or (d["HDR_RSV"] and not hdr_ok) or (d["GROUP_SIZE"] and not grp_ok):
        return E_FIELD, d
    if c >> 13 or e >> 6 or (out == OUT_FP16 and op != OP_ELT):
        return E_FIELD, d
    if out != OUT_INT8 and d["OUT_SCALE"]:
        return E_FIELD, d
    gemm = op == OP_GEMM or conv
    if gemm:
        if w4:
            if sym != 1 or adt not in (DT_FP32, DT_BF16) or d["HDR_RSV"] != 0 or d["GROUP_SIZE"] != W4_GROUP:
                return E_FIELD, d
        elif qmode not in (QM_TENSOR, QM_CHANNEL, QM_ROWCOL) or sym != 1 or adt != DT_INT8 or wdt != DT_INT8 \
                or (conv and qmode == QM_ROWCOL):
            return E_FIELD, d
        if (act != 0) != (fus == 1):
            return E_FIELD, d
        if op == OP_CONV_ACT and act == 0:
            return E_FIELD, d
        if conv:
            g = conv_params(d)
            if not (g["H"] and g["W"] and g["KH"] and g["KW"]) or g["OH"] < 1 or g["OW"] < 1 \
                    or d["M"] != g["OH"] * g["OW"]:
                return E_FIELD, d
    elif op == OP_RELU:
        if c != 0 or bias or d["K"] or d["W_OFF"] or d["SCALE_OFF"] or d["BIAS_OFF"] or act == 0:
            return E_FIELD, d
    elif op == OP_ROW:
        fn = c & 7
        if c >> 3 or fn > ROW_QUANT or act != 0 or (d["K"] and fn != ROW_SOFTMAX):
            return E_FIELD, d
        if fn == ROW_SOFTMAX and (bias or d["W_OFF"] or d["SCALE_OFF"] or d["BIAS_OFF"]):
            return E_FIELD, d
        if fn == ROW_QUANT and (bias or d["W_OFF"] or d["BIAS_OFF"] or out != OUT_INT8 or d["OUT_SCALE"]):
            return E_FIELD, d
        if not bias and d["BIAS_OFF"]:
            return E_FIELD, d
    elif op == OP_ELT:
        eop = c & 3
        if c >> 2 or d["K"] or d["SCALE_OFF"] or bias != (eop == ELT_MULADD) \
                or (eop == ELT_MULADD and out not in (OUT_FP32, OUT_FP16)) or (not bias and d["BIAS_OFF"]):
            return E_FIELD, d
    elif op == OP_ROPE:
        if c or act != 0 or bias or d["SCALE_OFF"] or d["BIAS_OFF"] or d["GROUP_SIZE"] == 0:
            return E_FIELD, d
    else:
        if c >> 1 or act != 0 or bias or d["SCALE_OFF"] or d["BIAS_OFF"]:
            return E_FIELD, d
    M, N, K = d["M"], d["N"], d["K"]
    if M == 0 or N == 0 or N % 16 or ((gemm or op == OP_FDOT) and (K == 0 or K % 16)):
        return E_ALIGN, d
    if w4 and (K < 2 * W4_GROUP or K % (2 * W4_GROUP) or K > 64 * W4_GROUP or d["W_OFF"] % 128):
        return E_ALIGN, d
    if op == OP_ROPE and (K == 0 or K % 32 or K > N):
        return E_ALIGN, d
    if conv:
        g = conv_params(d)
        if K % (g["KH"] * g["KW"]) or g["Cin"] % 16:
            return E_ALIGN, d
    for off in ("A_OFF", "Y_OFF", "SCALE_OFF", "BIAS_OFF") + (() if op == OP_ROW else ("W_OFF",)):
        al = 4 if (off == "W_OFF" and op == OP_ELT and d["HDR_RSV"] & 3 in (BM_COL, BM_SCALAR)) else 16
        if d[off] % al:
            return E_ALIGN, d
    lda, ldy, arow, yrow = strides(d)
    if lda < arow or ldy < yrow:
        return E_ALIGN, d
    if op in (OP_ELT, OP_FDOT):
        ldb, brow = bstride(d)
        if ldb < brow:
            return E_ALIGN, d
    return E_OK, d


def bstride(d: dict) -> tuple[int, int]:
    """golden.py:172-179."""
    if d["OPCODE"] == OP_FDOT:
        brow = (2 if d["HDR_RSV"] & STATE_FP16 else 4) * (d["N"] if d["CTRL"] & 1 else d["K"])
    else:
        brow = 4 * d["N"] if (d["HDR_RSV"] & 3) == BM_DENSE else 0
    return (16 * d["GROUP_SIZE"] if d["GROUP_SIZE"] else brow), brow


def strides(d: dict) -> tuple[int, int, int, int]:
    """golden.py:181-193: (lda, ldy, input row bytes, output row bytes)."""
    op = d["OPCODE"]
    aes = 4 if d["CTRL"] >> 4 & 15 == DT_FP32 else 2
    if is_w4(d):
        arow = aes * d["K"]
    elif op == OP_GEMM:
        arow = d["K"]
    elif op in CONV_OPS:
        arow = conv_params(d)["Cin"]
    elif op == OP_FDOT:
        arow = 4 * d["K"]
    else:
        arow = (2 if op == OP_ELT and d["HDR_RSV"] & STATE_FP16 else 4) * d["N"]
    yrow = d["N"] * ESIZE[d["EPI"] >> 2 & 3]
    return (16 * d["LDA16"] if d["LDA16"] else arow), (16 * d["LDY16"] if d["LDY16"] else yrow), arow, yrow


def segments(d: dict) -> tuple[list, list]:
    """golden.py:195-248: the byte segments each input tensor occupies and the output rows."""
    B, M, N, K = d["BASE_ADDR"], d["M"], d["N"], d["K"]
    lda, ldy, arow, yrow = strides(d)

    def rows(off, ld, n, nb):
        return [(B + off + m * ld, B + off + m * ld + nb) for m in range(n)]

    y = rows(d["Y_OFF"], ldy, M, yrow)
    op = d["OPCODE"]
    if op in V04_OPS:
        a = [(B + d["A_OFF"], B + d["A_OFF"] + arow)] if op == OP_ELT and d["HDR_RSV"] >> 2 & 1 \
            else rows(d["A_OFF"], lda, M, arow)
        reads = [a]
        w0 = B + d["W_OFF"]
        if op == OP_ELT:
            bm = d["HDR_RSV"] & 3
            if bm == BM_DENSE:
                ldb = bstride(d)[0]
                reads.append([(w0 + m * ldb, w0 + m * ldb + 4 * N) for m in range(M)])
            else:
                reads.append([(w0, w0 + {BM_ROW: 4 * N, BM_COL: 4 * M, BM_SCALAR: 4}[bm])])
            if d["CTRL"] & 3 == ELT_MULADD:
                reads.append(rows(d["BIAS_OFF"], ldy, M, yrow))
        elif op == OP_ROPE:
            reads.append([(w0, w0 + 4 * K * ((M - 1) // d["GROUP_SIZE"] + 1))])
        else:
            ldb, brow = bstride(d)
            reads.append([(w0 + i * ldb, w0 + i * ldb + brow) for i in range(K if d["CTRL"] & 1 else N)])
        return reads, y
    if op in CONV_OPS:
        g = conv_params(d)
        npx = g["H"] * g["W"]
        a0 = B + d["A_OFF"]
        reads = [[(a0, a0 + npx * arow)] if lda == arow else [(a0 + p * lda, a0 + p * lda + arow) for p in range(npx)]]
    else:
        reads = [rows(d["A_OFF"], lda, M, arow)]
    if op in (OP_GEMM,) + CONV_OPS:
        w4 = is_w4(d)
        ns = 1 if d["CTRL"] & 7 == QM_TENSOR else N
        reads.append([(B + d["W_OFF"], B + d["W_OFF"] + N * K // (2 if w4 else 1))])
        reads.append([(B + d["SCALE_OFF"], B + d["SCALE_OFF"] + (2 * N * (K // W4_GROUP) if w4 else 4 * ns))])
        if d["EPI"] >> 4 & 1:
            reads.append([(B + d["BIAS_OFF"], B + d["BIAS_OFF"] + 4 * N)])
        if d["CTRL"] & 7 == QM_ROWCOL and not w4:
            r0 = B + 16 * d["HDR_RSV"]
            reads.append([(r0, r0 + 4 * M)])
    elif op == OP_ROW and d["CTRL"] & 7 in (ROW_LAYERNORM, ROW_RMSNORM, ROW_L2NORM):
        reads.append([(B + d["SCALE_OFF"], B + d["SCALE_OFF"] + 4 * N)])
        if d["EPI"] >> 4 & 1:
            reads.append([(B + d["BIAS_OFF"], B + d["BIAS_OFF"] + 4 * N)])
    return reads, y


def extra_out(d: dict) -> list:
    """golden.py:250-256: ROW_QUANT also writes 4 M bytes of row scales at SCALE_OFF."""
    if d["OPCODE"] == OP_ROW and d["CTRL"] & 7 == ROW_QUANT:
        a = d["BASE_ADDR"] + d["SCALE_OFF"]
        return [(a, a + 4 * d["M"])]
    return []


def overlaps(segs: list, y: list) -> bool:
    """golden.py:258-267 (y ascending and disjoint)."""
    yhi = [hi for _, hi in y]
    for lo, hi in segs:
        i = bisect.bisect_right(yhi, lo)
        if i < len(y) and y[i][0] < hi:
            return True
    return False


def in_place(d: dict, i: int) -> bool:
    """golden.py:440-448."""
    out = d["EPI"] >> 2 & 3
    if d["OPCODE"] != OP_ELT or out not in (OUT_FP32, OUT_FP16):
        return False
    lda, ldy = strides(d)[:2]
    if i == 0:
        afmt = OUT_FP16 if d["HDR_RSV"] & STATE_FP16 else OUT_FP32
        return afmt == out and not (d["HDR_RSV"] >> 2 & 1) and d["A_OFF"] == d["Y_OFF"] and lda == ldy
    return i == 2 and d["BIAS_OFF"] == d["Y_OFF"]


def check(raw: bytes, ddr_len: int, core_id: int = 0, gemv_only: bool = False):
    """(ERR_CODE, decoded fields, reads, y, extra) with E_RANGE against ddr_len; raises
    ContractError for an output that overlaps an input (golden.py:459-479)."""
    err, d = validate(raw, core_id, gemv_only)
    if err != E_OK:
        return err, d, None, None, None
    reads, y = segments(d)
    extra = extra_out(d)
    if any(hi > ddr_len for seg in reads + [y, extra] for _, hi in seg):
        return E_RANGE, d, None, None, None
    for j, seg in enumerate(reads):
        if overlaps(seg, y) and not in_place(d, j):
            raise ContractError("an output overlaps an input")
        if extra and overlaps(seg, extra):
            raise ContractError("an output overlaps an input")
    if extra and overlaps(extra, y):
        raise ContractError("the two outputs overlap")
    return E_OK, d, reads, y, extra


def gpu_kind(d: dict) -> bool:
    """Every opcode but the convolutions runs on the GPU."""
    return d["OPCODE"] not in CONV_OPS


@dataclass
class Status:
    done: bool = False
    err_code: int = E_OK
    op_idx: int = 0
    host_op: bool = False


class Machine:
    """A DDR byte image and the in-order queue walk of golden.py:450-492 for every descriptor but
    the convolutions (a valid conv descriptor stops the queue with host_op)."""

    def __init__(self, ddr, core_id: int = 0, gemv_only: bool = False):
        self.ddr = bytearray(ddr)
        self.core_id, self.gemv_only = core_id, gemv_only

    def read(self, addr: int, n: int) -> bytes:
        return bytes(self.ddr[addr:addr + n])

    def _rows(self, addr: int, ld: int, m: int, nbytes: int, dtype) -> np.ndarray:
        return np.stack([np.frombuffer(self.read(addr + i * ld, nbytes), dtype) for i in range(m)])

    def _exec(self, d: dict) -> tuple[np.ndarray, tuple | None]:
        """The stored output rows [M, row bytes] (and ROW_QUANT's scales) of one descriptor."""
        B, M, N, K, e = d["BASE_ADDR"], d["M"], d["N"], d["K"], d["EPI"]
        lda = strides(d)[0]
        act, out, osc = act_of(e), e >> 2 & 3, np.frombuffer(struct.pack("<I", d["OUT_SCALE"]), "<f4")[0]
        bias = np.frombuffer(self.read(B + d["BIAS_OFF"], 4 * N), "<f4") if e >> 4 & 1 else None
        op = d["OPCODE"]
        if op == OP_ROW and d["CTRL"] & 7 == ROW_QUANT:                 # golden.py:369-372
            q, s = F.quant_rows(self._rows(B + d["A_OFF"], lda, M, 4 * N, "<f4"))
            return q.view(np.uint8).reshape(M, -1), (B + d["SCALE_OFF"], F.ftz(s).astype("<f4").tobytes())
        if op in (OP_RELU, OP_ROW, OP_ELT, OP_ROPE, OP_FDOT):
            y = self._rowop(d, lda)
        elif is_w4(d):                                                     # golden.py:295-324
            bf16 = d["CTRL"] >> 4 & 15 == DT_BF16
            x = self._rows(B + d["A_OFF"], lda, M, (2 if bf16 else 4) * K, "<u2" if bf16 else "<f4")
            wp = np.frombuffer(self.read(B + d["W_OFF"], N * K // 2), np.uint8).reshape(N, K // 2)
            ws = np.frombuffer(self.read(B + d["SCALE_OFF"], 2 * N * (K // W4_GROUP)), "<u2").reshape(N, -1)
            y = G.gemm_w4(x, wp, ws, bias, act, out, osc, x_is_bf16=bf16)
        else:                                                            # golden.py:326-349
            a = self._rows(B + d["A_OFF"], lda, M, K, np.int8)
            w = np.frombuffer(self.read(B + d["W_OFF"], N * K), np.int8).reshape(N, K)
            qm = d["CTRL"] & 7
            sc = np.frombuffer(self.read(B + d["SCALE_OFF"], 4 * (1 if qm == QM_TENSOR else N)), "<f4")
            sr = np.frombuffer(self.read(B + 16 * d["HDR_RSV"], 4 * M), "<f4") if qm == QM_ROWCOL else None
            y = G.gemm_rowcol(a, sr, w, sc, bias, act, out, osc)
        dt = {OUT_FP32: "<f4", OUT_BF16: "<u2", OUT_INT8: np.int8, OUT_FP16: "<u2"}[out]
        return np.ascontiguousarray(y.astype(dt)).view(np.uint8).reshape(M, -1), None

    def _f32rows(self, addr: int, ld: int, m: int, n: int, half: bool = False) -> np.ndarray:
        if half:
            return F.from_fp16_bits(self._rows(addr, ld, m, 2 * n, "<u2"))
        return self._rows(addr, ld, m, 4 * n, "<f4").astype(np.float32)

    def _rowop(self, d: dict, lda: int) -> np.ndarray:
        """RELU, the row functions, ELT, ROPE and FDOT (golden.py:351-436), converted to the output
        format."""
        B, M, N, K, e = d["BASE_ADDR"], d["M"], d["N"], d["K"], d["EPI"]
        act, out = act_of(e), e >> 2 & 3
        osc = np.frombuffer(struct.pack("<I", d["OUT_SCALE"]), "<f4")[0]
        op = d["OPCODE"]
        if op == OP_RELU:                                                # golden.py:351-356
            y = F.act_fn(self._f32rows(B + d["A_OFF"], lda, M, N), act)
        elif op == OP_ROW:                                               # golden.py:358-380
            x = self._f32rows(B + d["A_OFF"], lda, M, N)
            fn = d["CTRL"] & 7
            if fn == ROW_SOFTMAX and K:
                y = R.softmax_rows_causal(x, np.minimum(N, K + np.arange(M)))
            elif fn == ROW_SOFTMAX:
                y = R.softmax_rows(x)
            else:
                g = np.frombuffer(self.read(B + d["SCALE_OFF"], 4 * N), "<f4").astype(np.float32)
                b = np.frombuffer(self.read(B + d["BIAS_OFF"], 4 * N), "<f4").astype(np.float32) if e >> 4 & 1 else None
                eps = np.frombuffer(struct.pack("<I", d["W_OFF"]), "<f4")[0]
                f = {ROW_LAYERNORM: R.layernorm_rows, ROW_RMSNORM: R.rmsnorm_rows, ROW_L2NORM: R.l2norm_rows}[fn]
                y = f(x, g, b, eps)
        elif op == OP_ELT:                                               # golden.py:393-418
            ldy = strides(d)[1]
            hr = d["HDR_RSV"]
            a = self._f32rows(B + d["A_OFF"], 0 if hr >> 2 & 1 else lda, M, N, bool(hr & STATE_FP16))
            bm = hr & 3
            if bm == BM_DENSE:
                bv = self._f32rows(B + d["W_OFF"], bstride(d)[0], M, N)
            else:
                cnt = {BM_ROW: N, BM_COL: M, BM_SCALAR: 1}[bm]
                bv = np.frombuffer(self.read(B + d["W_OFF"], 4 * cnt), "<f4").astype(np.float32)
            eop = d["CTRL"] & 3
            c = self._f32rows(B + d["BIAS_OFF"], ldy, M, N, out == OUT_FP16) if eop == R.ELT_MULADD else None
            y = R.elt(eop, a, R.broadcast_b(bv, bm, M, N), c, act)
        elif op == OP_ROPE:                                              # golden.py:420-424
            G_, Rr = d["GROUP_SIZE"], K
            x = self._f32rows(B + d["A_OFF"], lda, M, N)
            tab = self._f32rows(B + d["W_OFF"], 4 * Rr, (M - 1) // G_ + 1, Rr)
            y = R.rope_rows(x, tab, G_, Rr)
        else:                                                            # OP_FDOT, golden.py:426-436
            a = self._f32rows(B + d["A_OFF"], lda, M, K)
            ldb = bstride(d)[0]
            if d["CTRL"] & 1:
                y = R.fdot_nn(a, self._f32rows(B + d["W_OFF"], ldb, K, N, bool(d["HDR_RSV"] & STATE_FP16)))
            else:
                y = R.fdot_nt(a, self._f32rows(B + d["W_OFF"], ldb, N, K))
        return G.convert(y, out, osc)

    def run_queue(self, queue_addr: int, n: int) -> Status:
        for i in range(n):
            qa = queue_addr + DESC_BYTES * i
            if qa + DESC_BYTES > len(self.ddr):
                return Status(False, E_RANGE, i)
            err, d, reads, y, extra = check(self.read(qa, DESC_BYTES), len(self.ddr), self.core_id, self.gemv_only)
            if err != E_OK:
                return Status(False, err, i)
            if not gpu_kind(d):
                return Status(False, E_OK, i, host_op=True)
            rows, scales = self._exec(d)
            for m in range(rows.shape[0]):
                self.ddr[y[m][0]:y[m][1]] = rows[m].tobytes()
            if scales:
                self.ddr[scales[0]:scales[0] + len(scales[1])] = scales[1]
        return Status(True, E_OK, n)
