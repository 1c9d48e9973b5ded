"""The descriptor-queue executor on the GPU (opentars_amd.queue over tars_run_queue) against the
oracle's queue walk: whole DDR images byte for byte and end statuses, on random programs of
ROW_QUANT, W8A8 GEMM (QM_TENSOR / QM_CHANNEL / QM_ROWCOL, every epilogue and output format,
strided rows), W4A16 GEMM, the row functions (softmax, causal softmax, LayerNorm, RMSNorm,
L2Norm), RELU, ELT (every op and broadcast, fp16 states, in place), RoPE and FDOT (NT, NN, fp16 B),
with errors, host hand-offs (a convolution) and overlaps. Needs a gfx950 GPU."""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from attention_data import plant_attention_specials
from oracle import queue as Q
from opentars_amd import queue as NQ
from opentars_amd.ops import ContractError

pytestmark = pytest.mark.gpu

IMAGE = 1 << 21
QADDR = 0x1F0000


class Program:
    """A DDR image under construction: data regions allocated upward from 0x1000, descriptors
    collected in order."""

    def __init__(self, seed: int, image: int = IMAGE, qaddr: int = QADDR):
        self.rng = np.random.default_rng(seed)
        self.ddr = bytearray(image)
        self.qaddr = qaddr
        self.top = 0x1000
        self.row_scale = 1.0   # rand_rows' values are multiplied by this
        self.descs: list[bytes] = []

    def alloc(self, nbytes: int, align: int = 16) -> int:
        a = (self.top + align - 1) // align * align
        self.top = a + nbytes + 16 * int(self.rng.integers(0, 3))
        assert self.top < self.qaddr
        return a

    def put(self, data: bytes, align: int = 16) -> int:
        a = self.alloc(len(data), align)
        self.ddr[a:a + len(data)] = data
        return a

    def add(self, **f) -> None:
        self.descs.append(Q.encode({"MAGIC": Q.MAGIC, "VERSION": Q.VERSION, "VALID": 1, **f}))

    def image(self) -> bytearray:
        img = bytearray(self.ddr)
        for i, d in enumerate(self.descs):
            img[self.qaddr + 64 * i:self.qaddr + 64 * (i + 1)] = d
        return img


def stride_fields(p: Program, m: int, row: int):
    """A row region of m rows; sometimes strided (LDA16 / LDY16 given), sometimes dense."""
    extra = int(p.rng.integers(0, 3))
    ld = row + 16 * extra
    return p.alloc(ld * m), (ld // 16 if extra else 0)


def add_quant(p: Program, M: int, K: int):
    x = (p.rng.normal(0, 1, (M, K)) * np.exp2(p.rng.integers(-8, 8, (M, 1)))).astype("<f4")
    a, lda16 = stride_fields(p, M, 4 * K)
    ld = 16 * lda16 if lda16 else 4 * K
    for m in range(M):
        p.ddr[a + m * ld:a + m * ld + 4 * K] = x[m].tobytes()
    y, ldy16 = stride_fields(p, M, K)
    s = p.alloc(4 * M)
    p.add(OPCODE=Q.OP_ROW, CTRL=Q.ROW_QUANT, EPI=Q.epi(out=Q.OUT_INT8), A_OFF=a, Y_OFF=y, SCALE_OFF=s, M=M, N=K,
          LDA16=lda16, LDY16=ldy16)
    return y, (16 * ldy16 if ldy16 else K), s


def add_w8(p: Program, M: int, N: int, K: int, qmode: int, a=None, lda=None, srow=None, act=None, out=None,
           bias=None):
    rng = p.rng
    if a is None:
        A = rng.integers(-128, 128, (M, K), dtype=np.int8)
        a, lda16 = stride_fields(p, M, K)
        ld = 16 * lda16 if lda16 else K
        for m in range(M):
            p.ddr[a + m * ld:a + m * ld + K] = A[m].tobytes()
    else:
        lda16 = 0 if lda == K else lda // 16
    w = p.put(rng.integers(-128, 128, (N, K), dtype=np.int8).tobytes())
    ns = 1 if qmode == Q.QM_TENSOR else N
    sc = rng.uniform(1e-4, 2e-2, ns).astype("<f4")
    if rng.integers(0, 8) == 0:
        sc[0] = 3e30
    s = p.put(sc.tobytes())
    act = int(rng.integers(0, 8)) if act is None else act
    out = int(rng.choice([Q.OUT_FP32, Q.OUT_BF16, Q.OUT_INT8])) if out is None else out
    bias = int(rng.integers(0, 2)) if bias is None else bias
    b = p.put(rng.normal(0, 2, N).astype("<f4").tobytes()) if bias else 0
    y, ldy16 = stride_fields(p, M, N * Q.ESIZE[out])
    hdr = 0
    if qmode == Q.QM_ROWCOL:
        if srow is None:
            srow = p.put(rng.uniform(0.1, 2.0, M).astype("<f4").tobytes())
        hdr = srow // 16
    osc = struct.unpack("<I", struct.pack("<f", float(rng.uniform(0.5, 8.0))))[0] if out == Q.OUT_INT8 else 0
    p.add(OPCODE=Q.OP_GEMM, CTRL=Q.ctrl(qmode, fusion=int(act != 0)), EPI=Q.epi(act, out, bias), A_OFF=a, W_OFF=w,
          SCALE_OFF=s, BIAS_OFF=b, Y_OFF=y, HDR_RSV=hdr, M=M, N=N, K=K, LDA16=lda16, LDY16=ldy16, OUT_SCALE=osc)
    return y


def add_w4(p: Program, M: int, N: int, K: int):
    rng = p.rng
    bf16 = bool(rng.integers(0, 2))
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    if bf16:
        xb = (x.view(np.uint32) >> 16).astype("<u2")
        a, lda16 = stride_fields(p, M, 2 * K)
        ld = 16 * lda16 if lda16 else 2 * K
        for m in range(M):
            p.ddr[a + m * ld:a + m * ld + 2 * K] = xb[m].tobytes()
    else:
        a, lda16 = stride_fields(p, M, 4 * K)
        ld = 16 * lda16 if lda16 else 4 * K
        for m in range(M):
            p.ddr[a + m * ld:a + m * ld + 4 * K] = x[m].astype("<f4").tobytes()
    w = p.put(rng.integers(0, 256, (N, K // 2), dtype=np.uint8).tobytes(), align=128)
    ws = (rng.uniform(1e-3, 1e-2, (N, K // 128)).astype(np.float16)).view("<u2")
    s = p.put(ws.tobytes())
    act = int(rng.integers(0, 8))
    out = int(rng.choice([Q.OUT_FP32, Q.OUT_BF16, Q.OUT_INT8]))
    bias = int(rng.integers(0, 2))
    b = p.put(rng.normal(0, 1, N).astype("<f4").tobytes()) if bias else 0
    y, ldy16 = stride_fields(p, M, N * Q.ESIZE[out])
    osc = struct.unpack("<I", struct.pack("<f", 4.0))[0] if out == Q.OUT_INT8 else 0
    p.add(OPCODE=Q.OP_GEMM, CTRL=Q.ctrl(Q.QM_GROUP, a_dtype=Q.DT_BF16 if bf16 else Q.DT_FP32, w_dtype=Q.DT_INT4,
                                        fusion=int(act != 0)),
          EPI=Q.epi(act, out, bias), GROUP_SIZE=128, A_OFF=a, W_OFF=w, SCALE_OFF=s, BIAS_OFF=b, Y_OFF=y, M=M, N=N,
          K=K, LDA16=lda16, LDY16=ldy16, OUT_SCALE=osc)


def f32bits(v: float) -> int:
    return struct.unpack("<I", struct.pack("<f", float(v)))[0]


def put_rows(p: Program, x: np.ndarray, row_bytes: int):
    """fp32 or uint16 rows [M, n] in a (sometimes strided) region; returns (offset, ld16)."""
    a, ld16 = stride_fields(p, x.shape[0], row_bytes)
    ld = 16 * ld16 if ld16 else row_bytes
    for m in range(x.shape[0]):
        p.ddr[a + m * ld:a + m * ld + row_bytes] = x[m].tobytes()
    return a, ld16


def rand_rows(p: Program, M: int, N: int) -> np.ndarray:
    x = (p.rng.normal(0, 1, (M, N)) * np.exp2(p.rng.integers(-4, 5, (M, 1))) * p.row_scale).astype("<f4")
    if p.rng.integers(0, 6) == 0:
        x[int(p.rng.integers(0, M)), int(p.rng.integers(0, N))] = [np.inf, -np.inf, np.nan, 0.0, 1e-40][
            int(p.rng.integers(0, 5))]
    return x


def out_fields(p: Program, M: int, N: int, outs=(Q.OUT_FP32, Q.OUT_BF16, Q.OUT_INT8)):
    out = int(p.rng.choice(outs))
    y, ldy16 = stride_fields(p, M, N * Q.ESIZE[out])
    osc = f32bits(p.rng.uniform(0.5, 8.0)) if out == Q.OUT_INT8 else 0
    return out, y, ldy16, osc


def add_row(p: Program, M: int, N: int, fn: int | None = None):
    rng = p.rng
    fn = int(rng.choice([Q.ROW_SOFTMAX, Q.ROW_LAYERNORM, Q.ROW_RMSNORM, Q.ROW_L2NORM])) if fn is None else fn
    a, lda16 = put_rows(p, rand_rows(p, M, N), 4 * N)
    out, y, ldy16, osc = out_fields(p, M, N)
    f = dict(OPCODE=Q.OP_ROW, CTRL=fn, A_OFF=a, Y_OFF=y, M=M, N=N, LDA16=lda16, LDY16=ldy16, OUT_SCALE=osc)
    if fn == Q.ROW_SOFTMAX:
        f.update(EPI=Q.epi(out=out), K=int(rng.integers(1, N + 1)) if rng.integers(0, 2) else 0)
    else:
        bias = int(rng.integers(0, 2))
        g = p.put(rng.normal(1, 0.2, N).astype("<f4").tobytes())
        b = p.put(rng.normal(0, 0.1, N).astype("<f4").tobytes()) if bias else 0
        eps = float(rng.choice([1e-6, 1e-5, 0.0]))
        f.update(EPI=Q.epi(out=out, bias=bias), SCALE_OFF=g, BIAS_OFF=b, W_OFF=f32bits(eps))
    p.add(**f)
    return y


def add_relu(p: Program, M: int, N: int, src=None, lda16=0):
    if src is None:
        src, lda16 = put_rows(p, rand_rows(p, M, N), 4 * N)
    out, y, ldy16, osc = out_fields(p, M, N)
    p.add(OPCODE=Q.OP_RELU, EPI=Q.epi(int(p.rng.integers(1, 8)), out), A_OFF=src, Y_OFF=y, M=M, N=N, LDA16=lda16,
          LDY16=ldy16, OUT_SCALE=osc)


def add_elt(p: Program, M: int, N: int):
    rng = p.rng
    op = int(rng.integers(0, 4))
    bm = int(rng.integers(0, 4))
    fp16 = bool(rng.integers(0, 3) == 0)
    arow = bool(rng.integers(0, 4) == 0)
    outs = (Q.OUT_FP32, Q.OUT_FP16) if op == Q.ELT_MULADD else (Q.OUT_FP32, Q.OUT_BF16, Q.OUT_INT8, Q.OUT_FP16)
    out = int(rng.choice(outs))
    A = rand_rows(p, 1 if arow else M, N)
    if fp16:
        with np.errstate(over="ignore"):
            A = A.astype(np.float16).view("<u2")
    inplace = not arow and rng.integers(0, 3) == 0 and (out == (Q.OUT_FP16 if fp16 else Q.OUT_FP32))
    arb = (2 if fp16 else 4) * N
    a, lda16 = put_rows(p, A, arb)
    if bm == Q.BM_DENSE:
        w, gs = put_rows(p, rand_rows(p, M, N), 4 * N)
    else:
        cnt = {Q.BM_ROW: N, Q.BM_COL: M, Q.BM_SCALAR: 1}[bm]
        w = p.put(rng.normal(0, 1, cnt).astype("<f4").tobytes(), align=16 if bm == Q.BM_ROW else 4)
        gs = 0
    if inplace:
        y, ldy16 = a, lda16
    else:
        y, ldy16 = stride_fields(p, M, N * Q.ESIZE[out])
    c = 0
    if op == Q.ELT_MULADD:
        C = rand_rows(p, M, N)
        crow = C.astype(np.float16).view("<u2") if out == Q.OUT_FP16 else C
        if not inplace and rng.integers(0, 2):
            c = y                                   # C is the output itself
            ld = 16 * ldy16 if ldy16 else N * Q.ESIZE[out]
            for m in range(M):
                p.ddr[y + m * ld:y + m * ld + N * Q.ESIZE[out]] = crow[m].tobytes()
        else:
            y_ld = 16 * ldy16 if ldy16 else N * Q.ESIZE[out]
            c = p.alloc(y_ld * M)
            for m in range(M):
                p.ddr[c + m * y_ld:c + m * y_ld + N * Q.ESIZE[out]] = crow[m].tobytes()
    osc = f32bits(rng.uniform(0.5, 8.0)) if out == Q.OUT_INT8 else 0
    hdr = bm | (4 if arow else 0) | (Q.STATE_FP16 if fp16 else 0)
    p.add(OPCODE=Q.OP_ELT, CTRL=op, EPI=Q.epi(int(rng.integers(0, 8)), out, int(op == Q.ELT_MULADD)), HDR_RSV=hdr,
          A_OFF=a, W_OFF=w, BIAS_OFF=c, Y_OFF=y, M=M, N=N, LDA16=lda16, LDY16=ldy16, GROUP_SIZE=gs, OUT_SCALE=osc)


def add_rope(p: Program, M: int, N: int):
    rng = p.rng
    R = 32 * int(rng.integers(1, N // 32 + 1))
    G = int(rng.integers(1, 4))
    a, lda16 = put_rows(p, rand_rows(p, M, N), 4 * N)
    rows = (M - 1) // G + 1
    fr = (np.arange(rows, dtype=np.float32)[:, None] * rng.uniform(0.01, 1.0, R // 2).astype(np.float32)[None, :])
    t = p.put(np.concatenate([np.cos(fr), np.sin(fr)], 1).astype("<f4").tobytes())
    out, y, ldy16, osc = out_fields(p, M, N)
    p.add(OPCODE=Q.OP_ROPE, EPI=Q.epi(out=out), A_OFF=a, W_OFF=t, Y_OFF=y, M=M, N=N, K=R, GROUP_SIZE=G,
          LDA16=lda16, LDY16=ldy16, OUT_SCALE=osc)


def add_fdot(p: Program, M: int, N: int, K: int):
    rng = p.rng
    nn = int(rng.integers(0, 2))
    fp16 = bool(nn and rng.integers(0, 2))
    a, lda16 = put_rows(p, rand_rows(p, M, K), 4 * K)
    Bm = rand_rows(p, K, N) if nn else rand_rows(p, N, K)
    if fp16:
        with np.errstate(over="ignore"):
            Bm = Bm.astype(np.float16).view("<u2")
    w, gs = put_rows(p, Bm, Bm.shape[1] * Bm.dtype.itemsize)
    out, y, ldy16, osc = out_fields(p, M, N)
    p.add(OPCODE=Q.OP_FDOT, CTRL=nn, HDR_RSV=Q.STATE_FP16 if fp16 else 0, EPI=Q.epi(out=out), A_OFF=a, W_OFF=w,
          Y_OFF=y, M=M, N=N, K=K, GROUP_SIZE=gs, LDA16=lda16, LDY16=ldy16, OUT_SCALE=osc)


def random_program(seed: int) -> Program:
    p = Program(seed)
    rng = p.rng
    for _ in range(int(rng.integers(4, 9))):
        kind = int(rng.integers(0, 10))
        M = int(rng.choice([1, 2, 4, 5, 17, 40]))
        if kind == 0:                                   # ROW_QUANT feeding a QM_ROWCOL GEMM (RAW)
            K = 16 * int(rng.integers(1, 40))
            q, ldq, s = add_quant(p, M, K)
            add_w8(p, M, 16 * int(rng.integers(1, 12)), K, Q.QM_ROWCOL, a=q, lda=ldq, srow=s)
        elif kind == 1:
            add_w8(p, M, 16 * int(rng.integers(1, 12)), 16 * int(rng.integers(1, 40)),
                   int(rng.choice([Q.QM_TENSOR, Q.QM_CHANNEL, Q.QM_ROWCOL])))
        elif kind == 2:
            add_w4(p, min(M, 5), 16 * int(rng.integers(1, 8)), 256 * int(rng.integers(1, 5)))
        elif kind == 3:
            add_quant(p, M, 16 * int(rng.integers(1, 60)))
        elif kind == 4:                                 # a decode row shared by 1-5 GEMMs (fusable)
            K = 16 * int(rng.integers(1, 80))
            q, ldq, s = add_quant(p, 1, K)
            for _ in range(int(rng.integers(1, 6))):
                add_w8(p, 1, 16 * int(rng.integers(1, 12)), K, Q.QM_ROWCOL, a=q, lda=ldq, srow=s)
        elif kind == 5:
            add_row(p, M, 16 * int(rng.integers(1, 70)))
        elif kind == 6:                                 # a GEMM's fp32 output through an activation (RAW)
            N = 16 * int(rng.integers(1, 12))
            y = add_w8(p, M, N, 16 * int(rng.integers(1, 20)), Q.QM_CHANNEL, out=Q.OUT_FP32)
            add_relu(p, M, N, src=y, lda16=0)
        elif kind == 7:
            add_elt(p, M, 16 * int(rng.integers(1, 20)))
        elif kind == 8:
            add_rope(p, M, 32 * int(rng.integers(1, 6)))
        else:
            add_fdot(p, M, 16 * int(rng.integers(1, 12)), 16 * int(rng.integers(1, 20)))
    return p


def both(img: bytearray, n: int, qaddr: int = QADDR, **kw):
    o = Q.Machine(img, **kw)
    ost = o.run_queue(qaddr, n)
    g = NQ.Machine(img, **kw)
    gst = g.run_queue(qaddr, n)
    return (o, ost), (g, gst)


def same_status(a, b) -> bool:
    return (bool(a.done), a.err_code, a.op_idx, bool(a.host_op)) == (bool(b.done), b.err_code, b.op_idx, bool(b.host_op))


def first_diff(a: bytes, b: bytes) -> int:
    x = np.frombuffer(a, np.uint8) != np.frombuffer(b, np.uint8)
    return int(np.argmax(x)) if x.any() else -1


@pytest.mark.parametrize("fusion", [True, False])
@pytest.mark.parametrize("seed", range(12))
def test_random_programs_match_the_oracle(seed, fusion):
    """With and without the executor's quantizer + GEMM fusion."""
    p = random_program(seed)
    prev = NQ.set_fusion(fusion)
    try:
        (o, ost), (g, gst) = both(p.image(), len(p.descs))
    finally:
        NQ.set_fusion(prev)
    assert ost.done and same_status(ost, gst), (ost, gst)
    gd = bytes(g.ddr)
    assert gd == bytes(o.ddr), f"first differing byte at {first_diff(gd, bytes(o.ddr)):#x}"


def cancelling_rows(rng, M: int, N: int, stride: int) -> np.ndarray:
    """Rows near 2^-115 whose summation chains (elements c, c + stride, ...) pass through a
    subnormal partial sum: per chain the first two elements are a near 2^-112 and -(a - s) with
    s = k 2^-133 (|k| < 100; exact, as s is a multiple of a's ulp), whose sum is exactly the
    subnormal s, and the third is near 2^-115, so a step that keeps s instead of flushing it changes
    the sum."""
    x = (rng.normal(0, 1, (M, N)) * 2.0 ** -115).astype(np.float32)
    for c in range(min(stride, N - 2 * stride)):
        a = ((1 + rng.random(M)) * 2.0 ** -112 * rng.choice([-1, 1], M)).astype(np.float32)
        sv = (rng.integers(1, 100, M) * rng.choice([-1, 1], M) * 2.0 ** -133).astype(np.float32)
        x[:, c], x[:, c + stride] = a, -(a - sv)
        assert (np.abs(x[:, c] + x[:, c + stride]) < np.float32(2.0 ** -126)).all()
    return x


def add_w4_cancelling(p: Program, M: int, N: int, K: int):
    """A W4A16 GEMM whose fp32 bank 0 (groups 0, 4, 8, ...) passes through a subnormal sum: group 4
    holds group 0's activations (near 2^-108, element 5 at 2^-115) and group 0's weights negated
    except element 5, which differs by 1; with every group scale 2^-20 the two terms (near 2^-122)
    are exact and add to the subnormal +-aq_5 2^-20 xs (near 2^-135); group 8's term follows it."""
    rng = p.rng
    assert K >= 9 * 128
    x = (rng.normal(0, 1, (M, K)) * 2.0 ** -108).astype(np.float32)
    x[:, 5] = np.float32(2.0 ** -115)
    x[:, 512:640] = x[:, 0:128]
    w = rng.integers(-7, 8, (N, K)).astype(np.int64)
    w[:, 512:640] = -w[:, 0:128]
    w[:, 512 + 5] += np.where(w[:, 512 + 5] < 7, 1, -1)
    nib = (w & 15).astype(np.uint8)
    wp = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    a, lda16 = put_rows(p, x, 4 * K)
    wo = p.put(wp.tobytes(), align=128)
    s = p.put(np.full((N, K // 128), 0x0010, "<u2").tobytes())      # binary16 2^-20
    y, ldy16 = stride_fields(p, M, 4 * N)
    p.add(OPCODE=Q.OP_GEMM, CTRL=Q.ctrl(Q.QM_GROUP, a_dtype=Q.DT_FP32, w_dtype=Q.DT_INT4), EPI=Q.epi(),
          GROUP_SIZE=128, A_OFF=a, W_OFF=wo, SCALE_OFF=s, Y_OFF=y, M=M, N=N, K=K, LDA16=lda16, LDY16=ldy16)


@pytest.mark.parametrize("seed", range(3))
@pytest.mark.parametrize("fusion", [True, False])
def test_chains_whose_partial_sums_are_subnormal(seed, fusion):
    """Summation chains whose steps' flushes decide the result (cancelling_rows): LayerNorm's
    16-lane row sums, FDOT NT's 16-lane chains and their fold (B is 1.0 on the cancelling columns,
    so the products are the row's elements), FDOT NN's sequential chains, and the W4A16 banks of
    add_w4_cancelling; the images equal the oracle's."""
    p = Program(7000 + seed)
    rng = p.rng
    for M, N in ((1, 1024), (3, 4096), (2, 208)):
        a, lda16 = put_rows(p, cancelling_rows(rng, M, N, 16), 4 * N)
        y, ldy16 = stride_fields(p, M, 4 * N)
        g = p.put(rng.normal(1, 0.2, N).astype("<f4").tobytes())
        p.add(OPCODE=Q.OP_ROW, CTRL=Q.ROW_LAYERNORM, EPI=Q.epi(), A_OFF=a, Y_OFF=y, SCALE_OFF=g, M=M, N=N,
              LDA16=lda16, LDY16=ldy16, W_OFF=f32bits(1e-30))
    for nn, M, N, K in ((0, 1, 64, 128), (0, 2, 48, 256), (1, 1, 128, 1008), (1, 3, 48, 64)):
        A = cancelling_rows(rng, M, K, 1 if nn else 16)
        a, lda16 = put_rows(p, A, 4 * K)
        B = (rng.normal(0, 1, (K, N) if nn else (N, K)) * 0.5).astype(np.float32)
        if nn:
            B[:3] = 1.0
        else:
            B[:, :48] = 1.0
        w, gs = put_rows(p, B, 4 * B.shape[1])
        y, ldy16 = stride_fields(p, M, 4 * N)
        p.add(OPCODE=Q.OP_FDOT, CTRL=nn, EPI=Q.epi(), A_OFF=a, W_OFF=w, Y_OFF=y, M=M, N=N, K=K, GROUP_SIZE=gs,
              LDA16=lda16, LDY16=ldy16)
    # the per-lane form in 8-wave workgroups (M = 2, 4 and 6); the K split over waves (M = 1,
    # K = 6400: 50 groups, the last wave two); the INT8 MFMA form's 4-row tiles over 8 waves (M = 12
    # and 20) and over 16 waves (M = 12, K = 3072)
    for M, N, K in ((1, 256, 1280), (2, 64, 1536), (4, 32, 1280), (1, 64, 6400), (12, 32, 1280),
                    (20, 64, 1280), (6, 48, 3072), (12, 48, 3072)):
        add_w4_cancelling(p, M, N, K)
    prev = NQ.set_fusion(fusion)
    try:
        (o, ost), (g, gst) = both(p.image(), len(p.descs))
    finally:
        NQ.set_fusion(prev)
    assert ost.done and same_status(ost, gst), (ost, gst)
    gd = bytes(g.ddr)
    assert gd == bytes(o.ddr), f"first differing byte at {first_diff(gd, bytes(o.ddr)):#x}"


@pytest.mark.parametrize("fusion", [True, False])
def test_w4_banks_subnormal_on_8row_tiles(fusion):
    """add_w4_cancelling on the INT8 MFMA form's 8-row tiles, whose lanes take each row's h and l
    sums from a permlane swap: one weight tile of 8 waves (M = 20, N = 688), two weight tiles of 16
    waves (N = 1376), and past 2048 k one weight tile of 16 waves (M = 16, K = 3072, N = 1040); the
    matrices need a larger image than the other chain cases."""
    image = 1 << 23
    p = Program(7100, image=image, qaddr=image - 0x10000)
    for M, N, K in ((20, 688, 1280), (20, 1376, 1280), (16, 1040, 3072)):
        add_w4_cancelling(p, M, N, K)
    prev = NQ.set_fusion(fusion)
    try:
        (o, ost), (g, gst) = both(p.image(), len(p.descs), qaddr=p.qaddr)
    finally:
        NQ.set_fusion(prev)
    assert ost.done and same_status(ost, gst), (ost, gst)
    gd = bytes(g.ddr)
    assert gd == bytes(o.ddr), f"first differing byte at {first_diff(gd, bytes(o.ddr)):#x}"


def add_residual_norm(p: Program, M: int, N: int, inplace: bool, norm_over_b: bool = False, shift: int = 0):
    """A residual ELT ADD of dense fp32 rows (fp32 out, no activation) and a norm of its output, the
    pair the executor fuses; norm_over_b: the norm writes over the ELT's B rows (fp32), shifted by
    `shift` rows (shift 1: norm row r lands on B row r + 1, which the fused launch's row r + 1 would
    read after row r wrote it), which the executor must not fuse."""
    rng = p.rng
    a, lda16 = put_rows(p, rand_rows(p, M, N), 4 * N)
    b, ldb16 = put_rows(p, rand_rows(p, M + shift, N), 4 * N)
    y, ldy16 = (a, lda16) if inplace else stride_fields(p, M, 4 * N)
    p.add(OPCODE=Q.OP_ELT, CTRL=Q.ELT_ADD, EPI=Q.epi(), A_OFF=a, W_OFF=b, Y_OFF=y, M=M, N=N, LDA16=lda16, LDY16=ldy16,
          GROUP_SIZE=ldb16)
    fn = int(rng.choice([Q.ROW_LAYERNORM, Q.ROW_RMSNORM, Q.ROW_L2NORM]))
    if norm_over_b:
        out, yo, ldyo16, osc = Q.OUT_FP32, b + shift * (16 * ldb16 if ldb16 else 4 * N), ldb16, 0
    else:
        out, yo, ldyo16, osc = out_fields(p, M, N)
    g = p.put(rng.normal(1, 0.2, N).astype("<f4").tobytes())
    bias = int(rng.integers(0, 2))
    bb = p.put(rng.normal(0, 0.1, N).astype("<f4").tobytes()) if bias else 0
    p.add(OPCODE=Q.OP_ROW, CTRL=fn, EPI=Q.epi(out=out, bias=bias), A_OFF=y, Y_OFF=yo, SCALE_OFF=g, BIAS_OFF=bb,
          W_OFF=f32bits(float(rng.choice([1e-6, 1e-5, 0.0]))), M=M, N=N, LDA16=ldy16, LDY16=ldyo16, OUT_SCALE=osc)


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("fusion", [True, False])
def test_residual_add_then_norm(seed, fusion):
    """ELT ADD -> norm pairs, which the executor runs as one launch: in place and apart, every norm,
    with and without beta, every output format, rows up to the fused kernel's 2048 elements and one
    block past it (not fused), and a pair whose norm writes over the ELT's B rows (not fused); the
    images equal the oracle's."""
    p = Program(8100 + seed)
    for k, (M, N) in enumerate(((1, 1024), (3, 2048), (2, 224), (1, 2064), (4, 1024))):
        add_residual_norm(p, M, N, inplace=bool(k % 2))
    add_residual_norm(p, 1, 1024, inplace=True, norm_over_b=True)
    add_residual_norm(p, 3, 512, inplace=True, norm_over_b=True, shift=1)
    add_residual_norm(p, 4, 256, inplace=False, norm_over_b=True, shift=1)
    prev = NQ.set_fusion(fusion)
    NQ.fusion_counts(reset=True)
    try:
        (o, ost), (g, gst) = both(p.image(), len(p.descs))
    finally:
        NQ.set_fusion(prev)
    assert ost.done and same_status(ost, gst), (ost, gst)
    # exactly the four pairs within the fused kernel's row limit and free of hazards ran fused
    assert NQ.fusion_counts()["add_norm"] == (4 if fusion else 0)
    gd = bytes(g.ddr)
    assert gd == bytes(o.ddr), f"first differing byte at {first_diff(gd, bytes(o.ddr)):#x}"


def add_norm_then_rope(p: Program, M: int, N: int, rot: int, G: int, rope_over_x: bool = False, shift: int = 0):
    """A norm with an fp32 output and a RoPE of its output rows (fp32 out), the pair the executor
    fuses; rope_over_x: the RoPE writes over the norm's input rows, shifted by `shift` rows (shift
    1: RoPE row r lands on input row r + 1, which the fused launch's row r + 1 would read after
    row r wrote it), which the executor must not fuse."""
    rng = p.rng
    a, lda16 = put_rows(p, rand_rows(p, M + shift, N), 4 * N)
    y, ldy16 = stride_fields(p, M, 4 * N)
    g = p.put(rng.normal(1, 0.2, N).astype("<f4").tobytes())
    bias = int(rng.integers(0, 2))
    bb = p.put(rng.normal(0, 0.1, N).astype("<f4").tobytes()) if bias else 0
    fn = int(rng.choice([Q.ROW_LAYERNORM, Q.ROW_RMSNORM, Q.ROW_L2NORM]))
    p.add(OPCODE=Q.OP_ROW, CTRL=fn, EPI=Q.epi(bias=bias), A_OFF=a, Y_OFF=y, SCALE_OFF=g, BIAS_OFF=bb,
          W_OFF=f32bits(1e-6), M=M, N=N, LDA16=lda16, LDY16=ldy16)
    rows = (M - 1) // G + 1
    fr = np.arange(rows, dtype=np.float32)[:, None] * rng.uniform(0.01, 1.0, rot // 2).astype(np.float32)[None, :]
    t = p.put(np.concatenate([np.cos(fr), np.sin(fr)], 1).astype("<f4").tobytes())
    yr, ldyr16 = ((a + shift * (16 * lda16 if lda16 else 4 * N), lda16) if rope_over_x
                  else stride_fields(p, M, 4 * N))
    p.add(OPCODE=Q.OP_ROPE, EPI=Q.epi(), A_OFF=y, W_OFF=t, Y_OFF=yr, M=M, N=N, K=rot, GROUP_SIZE=G, LDA16=ldy16,
          LDY16=ldyr16)


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("fusion", [True, False])
def test_norm_then_rope(seed, fusion):
    """Norm -> RoPE pairs, which the executor runs as one launch: q / k shapes (16 and 8 rows of
    128, one table row), several table rows, partial rotation, rows up to the fused kernel's 2048
    elements and one block past it (not fused), and a RoPE over the norm's input (not fused); the
    images equal the oracle's."""
    p = Program(8300 + seed)
    for M, N, rot, G in ((16, 128, 128, 16), (8, 128, 128, 8), (6, 256, 128, 2), (3, 2048, 2048, 1), (2, 2080, 64, 1)):
        add_norm_then_rope(p, M, N, rot, G)
    add_norm_then_rope(p, 4, 128, 128, 4, rope_over_x=True)
    add_norm_then_rope(p, 4, 128, 128, 4, rope_over_x=True, shift=1)
    add_norm_then_rope(p, 3, 256, 64, 1, rope_over_x=True, shift=1)
    prev = NQ.set_fusion(fusion)
    NQ.fusion_counts(reset=True)
    try:
        (o, ost), (g, gst) = both(p.image(), len(p.descs))
    finally:
        NQ.set_fusion(prev)
    assert ost.done and same_status(ost, gst), (ost, gst)
    # exactly the four pairs within the fused kernel's row limit and free of hazards ran fused
    assert NQ.fusion_counts()["norm_rope"] == (4 if fusion else 0)
    gd = bytes(g.ddr)
    assert gd == bytes(o.ddr), f"first differing byte at {first_diff(gd, bytes(o.ddr)):#x}"


def add_norm_rope_at(p: Program, M: int, N: int, rot: int, G: int, x: int = 0, y: int = 0, yr: int = 0):
    """A (norm, RoPE) pair over dense rows of N fp32: the norm reads x and writes y, the RoPE reads
    y and writes yr; each is a fresh region (x filled with random rows) when 0. Returns (x, y, yr)."""
    rng = p.rng
    if not x:
        x, _ = stride_fields(p, M, 4 * N)
        p.ddr[x:x + 4 * M * N] = rand_rows(p, M, N).tobytes()
    y = y or p.alloc(4 * M * N)
    yr = yr or p.alloc(4 * M * N)
    g = p.put(rng.normal(1, 0.2, N).astype("<f4").tobytes())
    fn = int(rng.choice([Q.ROW_LAYERNORM, Q.ROW_RMSNORM, Q.ROW_L2NORM]))
    p.add(OPCODE=Q.OP_ROW, CTRL=fn, EPI=Q.epi(), A_OFF=x, Y_OFF=y, SCALE_OFF=g, W_OFF=f32bits(1e-6), M=M, N=N)
    rows = (M - 1) // G + 1
    fr = np.arange(rows, dtype=np.float32)[:, None] * rng.uniform(0.01, 1.0, rot // 2).astype(np.float32)[None, :]
    t = p.put(np.concatenate([np.cos(fr), np.sin(fr)], 1).astype("<f4").tobytes())
    p.add(OPCODE=Q.OP_ROPE, EPI=Q.epi(), A_OFF=y, W_OFF=t, Y_OFF=yr, M=M, N=N, K=rot, GROUP_SIZE=G)
    return x, y, yr


@pytest.mark.parametrize("seed", range(3))
@pytest.mark.parametrize("fusion", [True, False])
def test_two_norm_rope_pairs_share_a_launch(seed, fusion):
    """Adjacent (norm, RoPE) pairs, which the executor runs two to a launch when they are
    independent: q / k shapes (merged), a pair whose norm reads the previous pair's RoPE output
    (not merged), a pair whose norm writes over the previous pair's input (not merged), a pair whose
    RoPE writes over the previous pair's RoPE output (not merged), two pairs that read the same
    rows (merged) after a pair the fused kernel does not take; the images equal the oracle's."""
    p = Program(8400 + seed)
    add_norm_rope_at(p, 16, 128, 128, 16)                  # P1 + P2 merged
    add_norm_rope_at(p, 8, 128, 128, 8)
    _, _, yr3 = add_norm_rope_at(p, 4, 256, 128, 1)        # P3 alone: P4 reads its output
    x4, _, _ = add_norm_rope_at(p, 4, 256, 64, 2, x=yr3)   # P4 alone: P5 writes over its input
    _, _, yr5 = add_norm_rope_at(p, 4, 256, 256, 4, y=x4)  # P5 alone: P6 writes over its output
    add_norm_rope_at(p, 2, 256, 128, 1, yr=yr5)            # P6 + P7 merged
    add_norm_rope_at(p, 3, 1024, 1024, 3)
    add_norm_rope_at(p, 2, 2080, 64, 1)                    # P8 not fused (rows past the kernel's limit)
    x9, _, _ = add_norm_rope_at(p, 5, 512, 512, 5)         # P9 + P10 merged (both read x9)
    add_norm_rope_at(p, 5, 512, 256, 1, x=x9)
    prev = NQ.set_fusion(fusion)
    NQ.fusion_counts(reset=True)
    try:
        (o, ost), (g, gst) = both(p.image(), len(p.descs))
    finally:
        NQ.set_fusion(prev)
    assert ost.done and same_status(ost, gst), (ost, gst)
    counts = NQ.fusion_counts()
    assert (counts["norm_rope"], counts["norm_rope_two"]) == ((9, 3) if fusion else (0, 0)), counts
    gd = bytes(g.ddr)
    assert gd == bytes(o.ddr), f"first differing byte at {first_diff(gd, bytes(o.ddr)):#x}"


@pytest.mark.parametrize("seed", range(3))
def test_host_copy_of_the_queue_gives_the_same_result(seed):
    p = random_program(200 + seed)
    img = p.image()
    o = Q.Machine(img)
    assert o.run_queue(QADDR, len(p.descs)).done
    g = NQ.Machine(img)
    assert g.run_queue(QADDR, len(p.descs), descs=b"".join(p.descs)).done
    assert bytes(g.ddr) == bytes(o.ddr)


@pytest.mark.parametrize("seed", range(4))
def test_repeated_queue_replays_its_plan_on_new_data(seed):
    """A decode loop's pattern: the same descriptors run again and again while the image's data
    changes. Run 1 checks and launches (and keeps a plan), run 2 captures the plan as a HIP graph,
    later runs launch the graph; every run equals the oracle's run on that run's image."""
    p = random_program(300 + seed)
    descs = b"".join(p.descs)
    img = p.image()
    g = NQ.Machine(img)
    rng = np.random.default_rng(seed)
    for rnd in range(4):
        if rnd:
            fresh = bytearray(img)
            fresh[0x1000:p.top] = rng.integers(0, 256, p.top - 0x1000, dtype=np.uint8).tobytes()
            img = fresh
            g.write(0, bytes(img[:QADDR]))
        st = g.run_queue(QADDR, len(p.descs), descs=descs)
        o = Q.Machine(img)
        ost = o.run_queue(QADDR, len(p.descs))
        assert ost.done and st.done, (rnd, ost, st)
        gd = bytes(g.ddr)
        assert gd == bytes(o.ddr), f"run {rnd}: first differing byte at {first_diff(gd, bytes(o.ddr)):#x}"
        img = bytearray(gd)


def add_gated_mlp(p: Program, N: int, K: int, act: int = 4, inplace: bool = True, gate_out: int = Q.OUT_FP32,
                  swap: bool = False, prod_over_w: bool = False):
    """An MLP's gated product (tars_mini/llm.py:620-624): ROW_QUANT of one row, the gate GEMM with
    its activation (SiLU = 4, GELU = 3) and the up GEMM (QM_ROWCOL, fp32 out), then ELT MUL of their
    outputs, in place over the gate's rows or apart. swap: the ELT reads up as A and gate as B;
    prod_over_w: the product lands on the gate GEMM's weights (so it may only be written after the
    GEMMs: the executor then runs the ELT on its own); gate_out: the gate GEMM's format. The
    executor folds the ELT into the group only for A = gate, B = up, fp32 outputs, a product that
    overlaps no operand of the group and K with whole-wave rows of at most four chunks per lane."""
    q, ldq, s = add_quant(p, 1, K)
    g = add_w8(p, 1, N, K, Q.QM_ROWCOL, a=q, lda=ldq, srow=s, act=act, out=gate_out, bias=int(p.rng.integers(0, 2)))
    u = add_w8(p, 1, N, K, Q.QM_ROWCOL, a=q, lda=ldq, srow=s, act=0, out=Q.OUT_FP32, bias=int(p.rng.integers(0, 2)))
    y = g if inplace else Q.decode(p.descs[-2])["W_OFF"] if prod_over_w else p.alloc(4 * N)
    a, b = (u, g) if swap else (g, u)
    p.add(OPCODE=Q.OP_ELT, CTRL=Q.ELT_MUL, EPI=Q.epi(), HDR_RSV=Q.BM_DENSE, A_OFF=a, W_OFF=b, Y_OFF=y, M=1, N=N)


@pytest.mark.parametrize("seed", range(3))
@pytest.mark.parametrize("fusion", [True, False])
def test_gated_mlp_product(seed, fusion):
    """ROW_QUANT -> gate GEMM (activation) -> up GEMM -> ELT MUL, which the executor runs as one
    launch (the gate and up rows of each index on one lane, the product stored with the outputs):
    the Qwen3-0.6B shape in place and apart, K = 2048 (two chunks per lane) with GELU, a height that
    leaves a partial last block; not fused: a bf16 gate output, swapped operands, a product over the
    gate's weights, K = 512 (16-lane rows). The images equal the oracle's."""
    image = 24 << 20
    p = Program(8500 + seed, image=image, qaddr=image - 0x10000)
    add_gated_mlp(p, 3072, 1024)
    add_gated_mlp(p, 3072, 1024, inplace=False)
    add_gated_mlp(p, 512, 2048, act=3)
    add_gated_mlp(p, 112, 768)
    add_gated_mlp(p, 256, 1024, gate_out=Q.OUT_BF16)
    add_gated_mlp(p, 256, 1024, inplace=False, swap=True)
    add_gated_mlp(p, 256, 1024, inplace=False, prod_over_w=True)
    add_gated_mlp(p, 256, 512)
    prev = NQ.set_fusion(fusion)
    NQ.fusion_counts(reset=True)
    try:
        (o, ost), (g, gst) = both(p.image(), len(p.descs), qaddr=p.qaddr)
    finally:
        NQ.set_fusion(prev)
    assert ost.done and same_status(ost, gst), (ost, gst)
    counts = NQ.fusion_counts()
    assert counts["gated_mlp"] == (4 if fusion else 0) and counts["quant_gemm"] == (8 if fusion else 0), counts
    gd = bytes(g.ddr)
    assert gd == bytes(o.ddr), f"first differing byte at {first_diff(gd, bytes(o.ddr)):#x}"


def add_norm_quant_group(p: Program, K: int, Ns, add: bool = True, gated: bool = False, inplace: bool = False,
                         sum_over_gamma: bool = False, fn=None):
    """[ELT ADD of two fp32 rows ->] norm (fp32 out) -> ROW_QUANT of the norm's output -> QM_ROWCOL
    GEMMs of heights Ns reading it [-> the gated product's ELT MUL of the first two], one row: a
    decoder's residual add, next norm and projections (tars_mini/llm.py:699-705, 767 and the next
    layer's norm). inplace: the ELT writes over its A row; sum_over_gamma: over the norm's gamma.
    Both make the executor run the norm apart from the quantizer group."""
    rng = p.rng
    g = p.put(rng.normal(1, 0.2, K).astype("<f4").tobytes())
    x = p.put(rand_rows(p, 1, K).tobytes())
    if add:
        b = p.put(rand_rows(p, 1, K).tobytes())
        y = x if inplace else g if sum_over_gamma else p.alloc(4 * K)
        p.add(OPCODE=Q.OP_ELT, CTRL=Q.ELT_ADD, EPI=Q.epi(), A_OFF=x, W_OFF=b, Y_OFF=y, M=1, N=K)
        x = y
    fn = int(rng.choice([Q.ROW_LAYERNORM, Q.ROW_RMSNORM, Q.ROW_L2NORM])) if fn is None else fn
    bias = int(rng.integers(0, 2))
    bb = p.put(rng.normal(0, 0.1, K).astype("<f4").tobytes()) if bias else 0
    h = p.alloc(4 * K)
    p.add(OPCODE=Q.OP_ROW, CTRL=fn, EPI=Q.epi(bias=bias), A_OFF=x, Y_OFF=h, SCALE_OFF=g, BIAS_OFF=bb,
          W_OFF=f32bits(float(rng.choice([1e-6, 1e-5, 0.0]))), M=1, N=K)
    q, s = p.alloc(K), p.alloc(4)
    p.add(OPCODE=Q.OP_ROW, CTRL=Q.ROW_QUANT, EPI=Q.epi(out=Q.OUT_INT8), A_OFF=h, Y_OFF=q, SCALE_OFF=s, M=1, N=K)
    ys = []
    for k, N in enumerate(Ns):
        gate = gated and k == 0
        ys.append(add_w8(p, 1, N, K, Q.QM_ROWCOL, a=q, lda=K, srow=s, act=4 if gate else None,
                         out=Q.OUT_FP32 if gated else None, bias=int(rng.integers(0, 2))))
    if gated:
        p.add(OPCODE=Q.OP_ELT, CTRL=Q.ELT_MUL, EPI=Q.epi(), HDR_RSV=Q.BM_DENSE, A_OFF=ys[0], W_OFF=ys[1], Y_OFF=ys[0],
              M=1, N=Ns[0])


@pytest.mark.parametrize("seed", range(3))
@pytest.mark.parametrize("fusion", [True, False])
def test_norm_prologue_groups(seed, fusion):
    """Residual ELT ADD -> norm -> ROW_QUANT -> GEMMs, which the executor runs as one launch (every
    workgroup forms the sum and the norm, the first stores them): q/k/v-like heights at K = 1024,
    a gated MLP at K = 1024, a norm alone in front of the group (the first layer's and the final
    norm), K = 2048 (two chunks per lane) and K = 768 (a partial chunk row), LayerNorm with and
    without beta; not as one launch: an ELT in place, a sum over the norm's gamma (the ELT runs on
    its own, the norm still in front of the quantizer), K = 512 (16-lane rows) and K = 2064 (three
    chunks per lane). The images equal the oracle's."""
    image = 24 << 20
    p = Program(8700 + seed, image=image, qaddr=image - 0x10000)
    add_norm_quant_group(p, 1024, (512, 256, 256))
    add_norm_quant_group(p, 1024, (768, 768), gated=True)
    add_norm_quant_group(p, 1024, (256, 256, 256, 256), add=False)
    add_norm_quant_group(p, 2048, (256,), fn=Q.ROW_LAYERNORM)
    add_norm_quant_group(p, 768, (320, 64))
    add_norm_quant_group(p, 1024, (256,), add=False, fn=Q.ROW_LAYERNORM)
    add_norm_quant_group(p, 1024, (256, 256), inplace=True)
    add_norm_quant_group(p, 1024, (256,), sum_over_gamma=True)
    add_norm_quant_group(p, 512, (256,))
    add_norm_quant_group(p, 2064, (128,))
    prev = NQ.set_fusion(fusion)
    NQ.fusion_counts(reset=True)
    try:
        (o, ost), (g, gst) = both(p.image(), len(p.descs), qaddr=p.qaddr)
    finally:
        NQ.set_fusion(prev)
    assert ost.done and same_status(ost, gst), (ost, gst)
    counts = NQ.fusion_counts()
    # the six groups in range and free of hazards took their norm (and ELT), the sum over gamma its norm
    # alone; every group fused its GEMMs; the ELT in place and K = 512 ran as ELT + norm pairs
    expect = (7, 10, 1, 2) if fusion else (0, 0, 0, 0)
    assert tuple(counts[k] for k in ("norm_quant", "quant_gemm", "gated_mlp", "add_norm")) == expect, counts
    gd = bytes(g.ddr)
    assert gd == bytes(o.ddr), f"first differing byte at {first_diff(gd, bytes(o.ddr)):#x}"


def test_an_int8_norm_is_not_taken_for_a_quantizer():
    """A norm with an int8 output read by a QM_ROWCOL GEMM as its A row with the norm's gamma as the
    row scale has a quantizer group's addresses, but it is a norm: the executor runs it as one."""
    p = Program(8800)
    K = 1024
    x = p.put(rand_rows(p, 1, K).tobytes())
    g = p.put(p.rng.uniform(0.5, 2.0, K).astype("<f4").tobytes())
    y = p.alloc(K)
    p.add(OPCODE=Q.OP_ROW, CTRL=Q.ROW_RMSNORM, EPI=Q.epi(out=Q.OUT_INT8), A_OFF=x, Y_OFF=y, SCALE_OFF=g,
          W_OFF=f32bits(1e-6), M=1, N=K, OUT_SCALE=f32bits(0.05))
    add_w8(p, 1, 256, K, Q.QM_ROWCOL, a=y, lda=K, srow=g)
    NQ.fusion_counts(reset=True)
    (o, ost), (g2, gst) = both(p.image(), len(p.descs))
    assert ost.done and same_status(ost, gst), (ost, gst)
    assert NQ.fusion_counts()["quant_gemm"] == 0
    gd = bytes(g2.ddr)
    assert gd == bytes(o.ddr), f"first differing byte at {first_diff(gd, bytes(o.ddr)):#x}"


def test_fusion_group_with_a_hazard_runs_one_by_one():
    """A decode row read by three GEMMs where the second GEMM writes over the third's weights: the
    fused launch would race, so the group runs descriptor by descriptor (the third GEMM then reads
    the second's output as its weights, as the golden's order has it)."""
    p = Program(70)
    K = 64
    q, ldq, s = add_quant(p, 1, K)
    add_w8(p, 1, 32, K, Q.QM_ROWCOL, a=q, lda=ldq, srow=s)
    add_w8(p, 1, 16, K, Q.QM_ROWCOL, a=q, lda=ldq, srow=s, out=Q.OUT_INT8)
    add_w8(p, 1, 16, K, Q.QM_ROWCOL, a=q, lda=ldq, srow=s)
    f1, f2 = Q.decode(p.descs[2]), Q.decode(p.descs[3])
    f1.pop("CRC32")
    f1.update(Y_OFF=f2["W_OFF"], LDY16=0)              # int8 [1, 16] lands in the third matrix's weights
    p.descs[2] = Q.encode(f1)
    (o, ost), (g, gst) = both(p.image(), 4)
    assert ost.done and same_status(ost, gst)
    assert bytes(g.ddr) == bytes(o.ddr)


def test_worked_example_on_the_gpu():
    rng = np.random.default_rng(2026)
    M, N, K = 2, 16, 32
    ddr = bytearray(1 << 16)
    ddr[0x100:0x140] = rng.integers(-128, 128, (M, K), dtype=np.int8).tobytes()
    ddr[0x200:0x400] = rng.integers(-128, 128, (N, K), dtype=np.int8).tobytes()
    ddr[0x600:0x640] = (rng.uniform(0.5, 2.0, N) / 4096).astype("<f4").tobytes()
    ddr[0x700:0x740] = rng.uniform(-8, 8, N).astype("<f4").tobytes()
    ddr[0x8000:0x8040] = bytes.fromhex("000000807FC4843700000000000020001000020000070000000600000010000000020000"
                                       "000100000000000000000000150000001A11020000000000020055AA")
    m = NQ.Machine(ddr)
    assert m.run_queue(0x8000, 1).done
    assert struct.unpack("<H", m.read(0x1002, 2))[0] == 0x3F16


@pytest.mark.parametrize("bad,code", [("MAGIC", Q.E_MAGIC), ("CRC", Q.E_CRC), ("N", Q.E_ALIGN), ("Y_OFF", Q.E_RANGE)])
def test_error_mid_queue_keeps_earlier_writes_only(bad, code):
    p = random_program(50)
    i = len(p.descs) // 2
    f = Q.decode(p.descs[i])
    f.pop("CRC32")
    if bad == "CRC":
        p.descs[i] = Q.encode(f, fix_crc=False)
    else:
        f[bad] = {"MAGIC": 0x1234, "N": 8, "Y_OFF": IMAGE - 16}[bad]
        p.descs[i] = Q.encode(f)
    (o, ost), (g, gst) = both(p.image(), len(p.descs))
    assert (ost.done, ost.err_code, ost.op_idx) == (False, code, i)
    assert same_status(ost, gst) and bytes(g.ddr) == bytes(o.ddr)


def test_output_overlapping_input_raises_and_writes_nothing_of_it():
    p = random_program(51)
    i = len(p.descs) - 1
    f = Q.decode(p.descs[i])
    f.pop("CRC32")
    f["Y_OFF"] = f["A_OFF"]
    p.descs[i] = Q.encode(f)
    img = p.image()
    o = Q.Machine(img)
    with pytest.raises(Q.ContractError):
        o.run_queue(QADDR, len(p.descs))
    g = NQ.Machine(img)
    with pytest.raises(ContractError):
        g.run_queue(QADDR, len(p.descs))
    assert bytes(g.ddr) == bytes(o.ddr)           # descriptors before it ran, it did not


def conv_desc(p: Program) -> tuple[int, bytes]:
    """A valid 3x3 convolution (4x4 input, pad 1, 16 -> 16 channels): the one descriptor kind the
    executor hands to the host. Its output rows are [16, 16] fp32."""
    a = p.put(p.rng.integers(-128, 128, (16, 16), dtype=np.int8).tobytes())
    w = p.put(p.rng.integers(-128, 128, (16, 9 * 16), dtype=np.int8).tobytes())
    s = p.put(np.full(16, 1e-3, "<f4").tobytes())
    y = p.alloc(4 * 16 * 16)
    return y, Q.encode({"MAGIC": Q.MAGIC, "VERSION": Q.VERSION, "VALID": 1, "OPCODE": Q.OP_CONV,
                        "CTRL": Q.ctrl(Q.QM_CHANNEL), "EPI": Q.epi(), "A_OFF": a, "W_OFF": w, "SCALE_OFF": s,
                        "Y_OFF": y, "M": 16, "N": 16, "K": 9 * 16, "GROUP_SIZE": 4,
                        "HDR_RSV": (4 << 12) | (3 << 8) | (3 << 4) | 1})


class FakeHost:
    """A host executor for the test: runs one convolution descriptor by writing a fixed fp32
    pattern (y[i] = (i - 128) / 8) to its output rows on the host image -- a stand-in for the host's
    own convolution, enough to follow the data across the hand-off."""

    def __init__(self, ddr: bytearray):
        self.ddr = ddr

    def run_queue(self, addr: int, n: int):
        d = Q.decode(bytes(self.ddr[addr:addr + 64]))
        assert n == 1 and d["OPCODE"] == Q.OP_CONV
        y = ((np.arange(d["M"] * d["N"], dtype=np.float32) - 128) / 8).astype("<f4")
        self.ddr[d["Y_OFF"]:d["Y_OFF"] + y.nbytes] = y.tobytes()
        return Q.Status(True, Q.E_OK, 1)


def test_host_hand_off_stops_then_resumes_with_a_host():
    """A convolution between two GPU descriptors: without a host the queue stops there (host_op);
    with one it runs on the host copy and the GPU descriptors after it see its output (RAW across
    the hand-off)."""
    p = Program(60)
    add_w8(p, 1, 32, 64, Q.QM_CHANNEL, act=0, out=Q.OUT_FP32, bias=0)
    cy, cdesc = conv_desc(p)
    p.descs.append(cdesc)
    add_quant(p, 16, 16)                              # quantizes the conv output: A_OFF patched below
    f = Q.decode(p.descs[-1])
    f.pop("CRC32")
    f.update(A_OFF=cy, LDA16=0)
    p.descs[-1] = Q.encode(f)
    img = p.image()
    g = NQ.Machine(img)
    st = g.run_queue(QADDR, 3)
    assert (st.done, st.op_idx, st.host_op) == (False, 1, True)
    # the expected image: the oracle to the conv, the fake host, then the oracle for the rest
    o = Q.Machine(img)
    assert o.run_queue(QADDR, 1).done
    FakeHost(o.ddr).run_queue(QADDR + 64, 1)
    assert o.run_queue(QADDR + 128, 1).done
    g2 = NQ.Machine(img, host=FakeHost)
    st2 = g2.run_queue(QADDR, 3)
    assert st2.done and st2.op_idx == 3
    assert bytes(g2.ddr) == bytes(o.ddr)
    assert bytes(NQ.run(img, QADDR, 3, host=FakeHost)) == bytes(o.ddr)


def test_unaligned_base_goes_to_the_host():
    """BASE_ADDR 8: legal for the contract, off the kernels' 16-byte alignment -> handed to the host
    (here the oracle's machine), with the same final image as the oracle's own run."""
    p = Program(61)
    add_w8(p, 2, 32, 64, Q.QM_CHANNEL)
    f = Q.decode(p.descs[0])
    f.pop("CRC32")
    f["BASE_ADDR"] = 8
    p.descs[0] = Q.encode(f)
    add_w8(p, 3, 48, 32, Q.QM_TENSOR)
    img = p.image()
    assert NQ.Machine(img).run_queue(QADDR, 2).host_op
    o = Q.Machine(img)
    assert o.run_queue(QADDR, 2).done
    g = NQ.Machine(img, host=lambda ddr: Q.Machine(ddr))
    assert g.run_queue(QADDR, 2).done
    assert bytes(g.ddr) == bytes(o.ddr)


def test_a_descriptor_that_overwrites_the_next_one():
    """ROW_QUANT's int8 output lands on the following descriptor: both executors read the
    overwritten bytes (which no longer hold a valid descriptor) and stop with the same code."""
    p = Program(62)
    add_quant(p, 1, 64)
    f = Q.decode(p.descs[0])
    f.pop("CRC32")
    f.update(Y_OFF=QADDR + 64, LDY16=0)
    p.descs[0] = Q.encode(f)
    add_w8(p, 1, 16, 64, Q.QM_CHANNEL)
    img = p.image()
    (o, ost), (g, gst) = both(img, 2)
    assert not ost.done and ost.op_idx == 1 and same_status(ost, gst), (ost, gst)
    assert bytes(g.ddr) == bytes(o.ddr)


def test_gemv_only_profile_refuses_long_k():
    p = Program(63)
    add_w8(p, 1, 16, 4112, Q.QM_CHANNEL)
    (o, ost), (g, gst) = both(p.image(), 1, gemv_only=True)
    assert (ost.err_code, gst.err_code) == (Q.E_OPCODE, Q.E_OPCODE)


# ------------------------------------------------------------------------------ fused attention
ATT_IMAGE, ATT_QADDR = 1 << 24, (1 << 24) - 0x10000


def attention_program(seed: int, heads: int, kv_heads: int, hd: int, M: int, t0: int, v_fp16: bool,
                      out: int = Q.OUT_FP32, hazard: bool = False, specials: bool = False) -> Program:
    """One layer's attention as the reference lowers it (tars_mini/llm.py:736-746): per query head an
    FDOT_NT of its q rows with its KV head's K rows into the shared score buffer, the causal softmax
    (t0 + 1 valid keys for the first row) into the shared probability buffer, and an FDOT_NN with the
    V rows into the head's output columns. hazard: the last head's q rows are the first head's
    output, so the heads cannot run concurrently. specials: plant_attention_specials."""
    p = Program(seed, image=ATT_IMAGE, qaddr=ATT_QADDR)
    rng = p.rng
    nk = (t0 + M + 15) // 16 * 16
    qrow = 4 * heads * hd
    qv = rng.normal(0, 0.3, (M, heads * hd)).astype(np.float32)
    kv_ = rng.normal(0, 1, (nk, kv_heads * hd)).astype(np.float32)
    vv = rng.normal(0, 1, (nk, kv_heads * hd)).astype(np.float32)
    if specials:
        plant_attention_specials(rng, qv, kv_, vv, kv_heads, hd, v_fp16)
    q = p.put(qv.astype("<f4").tobytes())
    kc = p.put(kv_.astype("<f4").tobytes())
    vc = p.put(vv.astype(np.float16).view("<u2").tobytes() if v_fp16 else vv.astype("<f4").tobytes())
    ves = 2 if v_fp16 else 4
    sc = p.alloc(4 * M * nk)
    pr = p.alloc(4 * M * nk)
    arow = heads * hd * Q.ESIZE[out]
    att = p.alloc(M * arow)
    osc = f32bits(4.0) if out == Q.OUT_INT8 else 0
    for h in range(heads):
        kv = h // (heads // kv_heads)
        dep = hazard and h == heads - 1
        p.add(OPCODE=Q.OP_FDOT, CTRL=0, EPI=Q.epi(), A_OFF=att if dep else q + 4 * h * hd, W_OFF=kc + 4 * kv * hd,
              Y_OFF=sc, M=M, N=nk, K=hd, LDA16=(arow if dep else qrow) // 16, GROUP_SIZE=4 * kv_heads * hd // 16)
        p.add(OPCODE=Q.OP_ROW, CTRL=Q.ROW_SOFTMAX, EPI=Q.epi(), A_OFF=sc, Y_OFF=pr, M=M, N=nk, K=t0 + 1)
        p.add(OPCODE=Q.OP_FDOT, CTRL=1, HDR_RSV=Q.STATE_FP16 if v_fp16 else 0, EPI=Q.epi(out=out), A_OFF=pr,
              W_OFF=vc + ves * kv * hd, Y_OFF=att + Q.ESIZE[out] * h * hd, M=M, N=hd, K=nk,
              GROUP_SIZE=ves * kv_heads * hd // 16, LDY16=arow // 16, OUT_SCALE=osc)
    return p


@pytest.mark.parametrize("fusion", [True, False])
@pytest.mark.parametrize("heads,kv_heads,hd,M,t0,v_fp16,out", [
    (16, 8, 128, 1, 250, False, Q.OUT_FP32),      # Qwen3-0.6B decode
    (4, 1, 256, 1, 37, True, Q.OUT_FP32),         # head dim 256, fp16 V state
    (8, 4, 64, 3, 100, False, Q.OUT_BF16),        # a 3-token chunk, bf16 out
    (2, 2, 128, 2, 0, False, Q.OUT_INT8),         # the first position
    (2, 1, 64, 2, 2000, True, Q.OUT_FP32),        # 32 V stages per row, two query rows
    (2, 1, 128, 1, 4100, False, Q.OUT_FP32),      # past the fused kernel's 4080 keys: unfused
])
def test_attention_layer_matches_the_oracle(fusion, heads, kv_heads, hd, M, t0, v_fp16, out):
    p = attention_program(heads * 1000 + t0, heads, kv_heads, hd, M, t0, v_fp16, out)
    prev = NQ.set_fusion(fusion)
    try:
        (o, ost), (g, gst) = both(p.image(), len(p.descs), ATT_QADDR)
    finally:
        NQ.set_fusion(prev)
    assert ost.done and same_status(ost, gst), (ost, gst)
    gd = bytes(g.ddr)
    assert gd == bytes(o.ddr), f"first differing byte at {first_diff(gd, bytes(o.ddr)):#x}"


@pytest.mark.parametrize("heads,kv_heads,hd,M,t0,v_fp16", [
    (4, 2, 128, 1, 250, False),
    (4, 2, 128, 2, 40, False),
    (2, 1, 64, 1, 300, True),
    (2, 1, 256, 1, 20, False),
])
def test_attention_with_values_the_flushes_change(heads, kv_heads, hd, M, t0, v_fp16):
    """The fused kernel's chains run unflushed and are recomputed with the flushes when an input,
    product or partial sum is subnormal: planted values that take that path match the oracle."""
    p = attention_program(heads * 77 + t0, heads, kv_heads, hd, M, t0, v_fp16, specials=True)
    (o, ost), (g, gst) = both(p.image(), len(p.descs), ATT_QADDR)
    assert ost.done and same_status(ost, gst), (ost, gst)
    gd = bytes(g.ddr)
    assert gd == bytes(o.ddr), f"first differing byte at {first_diff(gd, bytes(o.ddr)):#x}"


def rope_attention_program(seed: int, heads: int, kv_heads: int, hd: int, t0: int, fn: int = Q.ROW_RMSNORM,
                           beta: bool = False, rot: int = 0, key_row: int = -1, qn_over_v: bool = False) -> Program:
    """One decode layer's q / k norms and rotations and its attention (tars_mini/llm.py:705-746): the
    q norm of a row per query head and its RoPE, the k norm of a row per K / V head and its RoPE into
    key row t0 of the cache (key_row: another row), then the per-head FDOT_NT / softmax / FDOT_NN
    triples over the cache's keys rounded up to 16 (t0 + 1 valid). rot: the RoPE's rotated width (hd
    when 0); qn_over_v: the q norm writes over V rows."""
    p = Program(seed, image=ATT_IMAGE, qaddr=ATT_QADDR)
    rng = p.rng
    nk, rot = (t0 + 16) // 16 * 16, rot or hd
    kc = p.put(rng.normal(0, 1, (nk, kv_heads * hd)).astype("<f4").tobytes())
    vc = p.put(rng.normal(0, 1, (nk, kv_heads * hd)).astype("<f4").tobytes())
    qx = p.put(rand_rows(p, heads, hd).tobytes())
    kx = p.put(rand_rows(p, kv_heads, hd).tobytes())
    ang = rng.uniform(0, 6.3, rot // 2).astype(np.float32)
    tab = p.put(np.concatenate([np.cos(ang), np.sin(ang)]).astype("<f4").tobytes())
    qn = vc + 4 * kv_heads * hd if qn_over_v else p.alloc(4 * heads * hd)
    qr, kn = p.alloc(4 * heads * hd), p.alloc(4 * kv_heads * hd)
    for x, rows, y in ((qx, heads, qn), (kx, kv_heads, kn)):
        g = p.put(rng.normal(1, 0.2, hd).astype("<f4").tobytes())
        bb = p.put(rng.normal(0, 0.1, hd).astype("<f4").tobytes()) if beta else 0
        p.add(OPCODE=Q.OP_ROW, CTRL=fn, EPI=Q.epi(bias=int(beta)), A_OFF=x, Y_OFF=y, SCALE_OFF=g, BIAS_OFF=bb,
              W_OFF=f32bits(1e-6), M=rows, N=hd)
        ry = qr if y == qn else kc + 4 * (t0 if key_row < 0 else key_row) * kv_heads * hd
        p.add(OPCODE=Q.OP_ROPE, EPI=Q.epi(), A_OFF=y, W_OFF=tab, Y_OFF=ry, M=rows, N=hd, K=rot, GROUP_SIZE=rows)
    sc, pr, att = p.alloc(4 * nk), p.alloc(4 * nk), p.alloc(4 * heads * hd)
    for h in range(heads):
        kv = h // (heads // kv_heads)
        p.add(OPCODE=Q.OP_FDOT, CTRL=0, EPI=Q.epi(), A_OFF=qr + 4 * h * hd, W_OFF=kc + 4 * kv * hd, Y_OFF=sc, M=1,
              N=nk, K=hd, GROUP_SIZE=4 * kv_heads * hd // 16)
        p.add(OPCODE=Q.OP_ROW, CTRL=Q.ROW_SOFTMAX, EPI=Q.epi(), A_OFF=sc, Y_OFF=pr, M=1, N=nk, K=t0 + 1)
        p.add(OPCODE=Q.OP_FDOT, CTRL=1, EPI=Q.epi(), A_OFF=pr, W_OFF=vc + 4 * kv * hd, Y_OFF=att + 4 * h * hd, M=1,
              N=hd, K=nk, GROUP_SIZE=4 * kv_heads * hd // 16)
    return p


@pytest.mark.parametrize("fusion", [True, False])
@pytest.mark.parametrize("heads,kv_heads,hd,t0,fn,beta,rot,key_row,qn_over_v,fused", [
    (16, 8, 128, 250, Q.ROW_RMSNORM, False, 0, -1, False, True),     # Qwen3-0.6B
    (4, 2, 64, 40, Q.ROW_LAYERNORM, True, 0, -1, False, True),       # LayerNorm with beta
    (8, 2, 128, 300, Q.ROW_L2NORM, False, 0, -1, False, True),       # four query heads per K / V head
    (4, 1, 256, 17, Q.ROW_RMSNORM, False, 0, -1, False, True),       # head dim 256, one K / V head
    (4, 2, 128, 60, Q.ROW_RMSNORM, False, 64, -1, False, False),     # partial rotation: apart
    (4, 2, 128, 60, Q.ROW_RMSNORM, False, 0, 59, False, True),       # the k RoPE on another key row
    (4, 2, 128, 64, Q.ROW_RMSNORM, False, 0, -1, False, True),       # the new key in a later key chunk
    (4, 2, 128, 60, Q.ROW_RMSNORM, False, 0, -1, True, False),       # the q norm over V rows: apart
])
def test_rope_pairs_fold_into_the_attention(fusion, heads, kv_heads, hd, t0, fn, beta, rot, key_row, qn_over_v,
                                            fused):
    """A layer's q and k (norm, RoPE) pairs and its attention, which the executor runs as one
    attention launch whose scores kernel forms the query rows and the new key row itself (storing
    the norm and RoPE outputs), when the rotation is full width, the k RoPE writes exactly one key row
    per K / V head and no output of the pairs lands on a K / V row; otherwise the pairs and the
    attention run as their own launches. The images equal the oracle's."""
    p = rope_attention_program(heads * 31 + t0, heads, kv_heads, hd, t0, fn, beta, rot, key_row, qn_over_v)
    prev = NQ.set_fusion(fusion)
    NQ.fusion_counts(reset=True)
    try:
        (o, ost), (g, gst) = both(p.image(), len(p.descs), ATT_QADDR)
    finally:
        NQ.set_fusion(prev)
    assert ost.done and same_status(ost, gst), (ost, gst)
    counts = NQ.fusion_counts()
    assert counts["rope_attention"] == int(fusion and fused), counts
    assert counts["attention"] == int(fusion), counts
    gd = bytes(g.ddr)
    assert gd == bytes(o.ddr), f"first differing byte at {first_diff(gd, bytes(o.ddr)):#x}"


def test_attention_heads_that_depend_on_each_other_run_in_order():
    """The last head reads the first head's output as its q rows: not concurrent, so not fused as
    one group; the image still equals the oracle's in-order run."""
    p = attention_program(7, 4, 2, 64, 1, 30, False, hazard=True)
    (o, ost), (g, gst) = both(p.image(), len(p.descs), ATT_QADDR)
    assert ost.done and same_status(ost, gst), (ost, gst)
    assert bytes(g.ddr) == bytes(o.ddr)


def test_attention_plan_replays_with_new_cache_data():
    """The fused attention inside a launch plan: the same queue run again on changed q / K / V bytes."""
    p = attention_program(11, 16, 8, 128, 1, 60, False)
    img = p.image()
    g = NQ.Machine(img)
    rng = np.random.default_rng(3)
    for rep in range(3):
        if rep:
            new = rng.normal(0, 1, 0x40000).astype("<f4").tobytes()
            img[0x1000:0x1000 + len(new)] = new
            g.write(0x1000, new)
        gst = g.run_queue(ATT_QADDR, len(p.descs))
        o = Q.Machine(img)
        ost = o.run_queue(ATT_QADDR, len(p.descs))
        assert ost.done and gst.done
        assert bytes(g.ddr) == bytes(o.ddr), f"replay {rep}: first differing byte at {first_diff(bytes(g.ddr), bytes(o.ddr)):#x}"


@pytest.mark.parametrize("graphs", [False, True])
def test_attention_queues_on_two_streams_at_once(graphs):
    """Two images' attention queues run on two streams at once, op by op (each stream's own scores
    scratch) or as launch plans (each plan's own): both images end as the oracle's."""
    progs = [attention_program(21 + i, 16, 8, 128, 1, 250 - 80 * i, False) for i in range(2)]
    imgs = [p.image() for p in progs]
    want = []
    for p, img in zip(progs, imgs):
        o = Q.Machine(bytearray(img))
        assert o.run_queue(ATT_QADDR, len(p.descs)).done
        want.append(bytes(o.ddr))
    descs = [bytes(img[ATT_QADDR:ATT_QADDR + 64 * len(p.descs)]) for p, img in zip(progs, imgs)]
    prev = NQ.set_graphs(graphs)
    try:
        ms = [NQ.Machine(img) for img in imgs]
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        torch.cuda.synchronize()
        for rep in range(8):
            for j in (0, 1):
                with torch.cuda.stream(streams[j]):
                    assert ms[j].run_queue(ATT_QADDR, len(progs[j].descs), descs[j]).done
        torch.cuda.synchronize()
        for j in (0, 1):
            got = bytes(ms[j].ddr)
            assert got == want[j], f"image {j}: first differing byte at {first_diff(got, want[j]):#x}"
    finally:
        NQ.set_graphs(prev)


def decode_step_image(seed: int, **shape):
    """A whole decode step of a small Qwen3-style model (bench.DecodeQueue, the reference's lowering
    of one token: tars_mini/llm.py:614-640, 705-767) in a host image with seeded data."""
    from bench import DecodeQueue
    dq = DecodeQueue(**shape)
    rng = np.random.default_rng(seed)
    img = bytearray(dq.size)

    def put(kind, off, n, extra=None):
        if kind == "int8":
            b = rng.integers(-127, 128, n, dtype=np.int8).tobytes()
        elif kind == "scale":
            b = (rng.random(n) * 9e-3 + 1e-3).astype("<f4").tobytes()
        elif kind == "gamma":
            b = (1 + 0.1 * rng.normal(0, 1, n)).astype("<f4").tobytes()
        elif kind == "rope":
            rows, hd = n
            fr = np.arange(rows, dtype=np.float32)[:, None] * (
                1.0 / (1e6 ** (np.arange(0, hd, 2, dtype=np.float32) / hd)))[None, :]
            b = np.concatenate([np.cos(fr), np.sin(fr)], 1).astype("<f4").tobytes()
        else:
            b = (rng.normal(0, 1, n) * extra).astype("<f4").tobytes()
        img[off:off + len(b)] = b

    dq.fill(put)
    q = dq.raw()
    img[dq.qaddr:dq.qaddr + len(q)] = q
    return dq, img


@pytest.mark.parametrize("shape", ["small", "qwen3_width"])
@pytest.mark.parametrize("fusion", [True, False])
def test_whole_decode_step_matches_the_oracle(fusion, shape):
    """Every opcode of a decode step in one queue (RMSNorm, ROW_QUANT + q/k/v GEMMs, q/k norms per
    head, RoPE into the K cache, V straight into the cache, the attention triples, o, residual
    ELT_ADD, SiLU gate * up in place, down, final norm and a 4-block head): the image byte for byte,
    on the first run and on two plan replays. qwen3_width: one layer at Qwen3-0.6B's width (H =
    1024, 16 heads of 128, ff = 3072), where the gate / up GEMMs and their ELT MUL run as one launch."""
    dims = dict(small=dict(layers=2, H=256, heads=4, kv_heads=2, hd=64, ff=512, vocab=1024, t0=40),
                qwen3_width=dict(layers=1, H=1024, heads=16, kv_heads=8, hd=128, ff=3072, vocab=2048, t0=40))[shape]
    dq, img = decode_step_image(5, **dims)
    n = len(dq.descs)
    o = Q.Machine(img)
    ost = o.run_queue(dq.qaddr, n)
    assert ost.done, ost
    prev = NQ.set_fusion(fusion)
    NQ.fusion_counts(reset=True)
    try:
        g = NQ.Machine(img)
        for rep in range(3):
            gst = g.run_queue(dq.qaddr, n)
            assert same_status(ost, gst), (rep, ost, gst)
            gd = bytes(g.ddr)
            assert gd == bytes(o.ddr), f"run {rep}: first differing byte at {first_diff(gd, bytes(o.ddr)):#x}"
    finally:
        NQ.set_fusion(prev)
    counts = NQ.fusion_counts()
    assert counts["gated_mlp"] == (3 * dims["layers"] if fusion and shape == "qwen3_width" else 0), counts
    # each layer's q and k (norm, RoPE) pairs run in its attention launch
    assert counts["rope_attention"] == (3 * dims["layers"] if fusion else 0), counts
    # at Qwen3 width every norm runs in front of its quantizer group: each layer's two and the final one
    assert counts["norm_quant"] == (3 * (2 * dims["layers"] + 1) if fusion and shape == "qwen3_width" else 0), counts
    logits = np.frombuffer(bytes(o.ddr[dq.logits:dq.logits + 4 * dq.vocab]), "<f4")
    assert np.isfinite(logits).all() and np.abs(logits).max() > 0
