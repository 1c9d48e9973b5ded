"""The golden model's matrix ops, restated in numpy -- TEST INFRASTRUCTURE ONLY.

Op-level forms of the descriptor semantics the HIP kernels reproduce bit for bit:
  gemm_rowcol        OP_GEMM with QM_ROWCOL / QM_CHANNEL / QM_TENSOR   golden.py:326-349
  gemm_rowcol_ksplit the K-block split and its in-order fp32 adds      llm.py:303-321, 627-635,
                                                                       golden.py:393-418 (ELT_ADD)
  gemm_w4            OP_GEMM W4A16 (QM_GROUP + INT4 weights)           golden.py:295-324
  convert            output conversion (fp32 / bf16 / int8 / fp16)     golden.py:273-280
plus the host weight quantizers (compiler.py:47-85).
"""
from __future__ import annotations

import numpy as np

from . import numerics as F

OUT_FP32, OUT_BF16, OUT_INT8, OUT_FP16 = 0, 1, 2, 3


def int_dot(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Exact integer products a [M, K] . w [N, K]^T in int64 (golden.py:336)."""
    return np.asarray(a, np.int64) @ np.asarray(w, np.int64).T


def convert(y: np.ndarray, out: int, out_scale: np.float32 | None = None) -> np.ndarray:
    """fp32 results -> stored elements (golden.py:273-280): fp32 flushed; bf16 bits (RNE, NaN
    0x7FC0); int8 q8(y, OUT_SCALE); fp16 bits (RNE with gradual underflow, NaN 0x7E00)."""
    if out == OUT_FP32:
        return F.ftz(y)
    if out == OUT_BF16:
        return F.to_bf16_bits(y)
    if out == OUT_INT8:
        return F.q8(y, np.float32(out_scale))
    if out == OUT_FP16:
        return F.to_fp16_bits(y)
    raise ValueError(f"output format {out}")


def epilogue_rowcol(acc: np.ndarray, srow, scol, bias=None, act: int = F.ACT_NONE) -> np.ndarray:
    """acc int [M, N] -> fp32 [M, N] in the golden order (golden.py:340-348): i2f; times the row
    scale (when given); times the column scale (one value or one per column); plus bias; act.
    Each step one rounded operation, never an FMA."""
    M, N = acc.shape
    y = F.i2f(acc)
    if srow is not None:
        y = F.fmul(y, np.asarray(srow, np.float32).reshape(M, 1))
    y = F.fmul(y, np.broadcast_to(np.asarray(scol, np.float32).reshape(1, -1), (M, N)))
    if bias is not None:
        y = F.fadd(y, np.broadcast_to(np.asarray(bias, np.float32).reshape(1, N), (M, N)))
    return F.act_fn(y, act)


def gemm_rowcol(q, srow, W, scol, bias=None, act: int = F.ACT_NONE, out: int = OUT_FP32,
                out_scale=None) -> np.ndarray:
    """W8A8: q int8 [M, K], srow fp32 [M] (None: QM_CHANNEL / QM_TENSOR, no row scale),
    W int8 [N, K], scol fp32 [N] (or [1]: QM_TENSOR). Returns the stored [M, N] elements."""
    acc = int_dot(q, W)
    if np.abs(acc).max(initial=0) >= 2 ** 31:
        raise OverflowError("accumulator outside int32")
    return convert(epilogue_rowcol(acc, srow, scol, bias, act), out, out_scale)


def gemm_rowcol_ksplit(q, srow, blocks: list, scol) -> np.ndarray:
    """K split into blocks W_i [N, K_i] over consecutive column ranges of the one quantized row
    block q [M, sum K_i], sharing srow and scol: each block is its own W8A8 GEMM with fp32 output,
    then the partials add in block order, y = (((y0 + y1) + y2) + ...) (llm.py:627-635 with
    golden.py:411-412)."""
    c0, y = 0, None
    for W in blocks:
        k = W.shape[1]
        part = gemm_rowcol(q[:, c0:c0 + k], srow, W, scol)
        y = part if y is None else F.ftz(F.fadd(F.ftz(y), part))
        c0 += k
    if c0 != q.shape[1]:
        raise ValueError("blocks do not cover K")
    return y


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """uint8 [N, K/2] -> int [N, K]: the low nibble is the even k, the high nibble the odd k,
    both two's-complement 4-bit (golden.py:308-311)."""
    p = np.asarray(packed, np.uint8)
    lo = (p & 0x0F).astype(np.int16)
    hi = (p >> 4).astype(np.int16)
    lo -= (lo >= 8) * 16
    hi -= (hi >= 8) * 16
    out = np.empty((p.shape[0], 2 * p.shape[1]), np.int16)
    out[:, 0::2] = lo
    out[:, 1::2] = hi
    return out


def w4_group_dots(aq: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Exact per-group dots [M, N, G] of int16 mantissas and int4 weights."""
    M, K = aq.shape
    N = w.shape[0]
    G = K // F.W4_GROUP
    a3 = aq.reshape(M, G, F.W4_GROUP).astype(np.int64)
    w3 = w.reshape(N, G, F.W4_GROUP).astype(np.int64)
    return np.einsum("mgk,ngk->mng", a3, w3)


def gemm_w4(x, Wp, ws_bits, bias=None, act: int = F.ACT_NONE, out: int = OUT_FP32,
            out_scale=None, x_is_bf16: bool = False) -> np.ndarray:
    """W4A16 (golden.py:295-324): x fp32 [M, K] (or bf16 bits), Wp uint8 [N, K/2], ws_bits uint16
    [N, K/128] binary16 group scales. Per group g: term = (i2f(dot) * ws[n, g]) * xs[m, g]; four
    fp32 banks acc[g % 4] each add their terms in g order from +0; y = (b0 + b1) + (b2 + b3);
    then bias, activation, conversion."""
    a = F.bf16_bits_to_f32(x) if x_is_bf16 else np.asarray(x, np.float32)
    aq, xs = F.align_w4_groups(a)
    w = unpack_int4(Wp)
    dots = w4_group_dots(aq, w)
    ws = F.from_fp16_bits(ws_bits)
    M, N, G = dots.shape
    banks = np.zeros((4, M, N), np.float32)
    for g in range(G):
        term = F.fmul(F.fmul(F.i2f(dots[:, :, g]), ws[None, :, g]), xs[:, g, None])
        banks[g % 4] = F.fadd(banks[g % 4], term)
    y = F.fadd(F.fadd(banks[0], banks[1]), F.fadd(banks[2], banks[3]))
    if bias is not None:
        y = F.fadd(y, np.broadcast_to(np.asarray(bias, np.float32).reshape(1, N), (M, N)))
    return convert(F.act_fn(y, act), out, out_scale)


# ---------------------------------------------------------------- host weight formats
def quantize_weight(w: np.ndarray, per_channel: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric INT8 in float64 (compiler.py:51-57), per output channel (QM_ROWCOL / QM_CHANNEL
    scales, int8 [N, K] plus fp32 [N]) or per tensor (QM_TENSOR, fp32 [1]): s = amax / 127 (1.0
    for an all-zero row or tensor), q = rint(w / s) ties to even, clipped to +-127; s stored as
    fp32 after the float64 quotient."""
    w = np.asarray(w, np.float64)
    amax = np.abs(w).max(axis=1) if per_channel else np.array([np.abs(w).max()])
    s = np.where(amax > 0, amax / 127.0, 1.0)
    q = np.clip(np.rint(w / (s[:, None] if per_channel else s[0])), -127, 127).astype(np.int8)
    return q, s.astype(np.float32)


def quantize_weight4(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Group-128 symmetric INT4 (compiler.py:69-85): s = fp16(fp32(amax / 7)) (1.0 for an all-zero
    group), q = rint(w / s) clipped to +-7, packed low nibble = even k. Returns (uint8 [N, K/2],
    uint16 [N, K/128])."""
    w = np.asarray(w, np.float64)
    n, k = w.shape
    if k == 0 or k % F.W4_GROUP:
        raise ValueError("W4A16 weights need [N, K], K a nonzero multiple of 128")
    g = w.reshape(n, k // F.W4_GROUP, F.W4_GROUP)
    amax = np.abs(g).max(axis=2)
    s16 = np.where(amax > 0, amax / 7.0, 1.0).astype(np.float32).astype(np.float16)
    s = s16.astype(np.float64)
    q = np.clip(np.rint(g / s[:, :, None]), -7, 7).astype(np.int16).reshape(n, k)
    packed = ((q[:, 0::2] & 0xF) | ((q[:, 1::2] & 0xF) << 4)).astype(np.uint8)
    return packed, s16.view(np.uint16)


def pack_int4(w: np.ndarray) -> np.ndarray:
    """int [N, K] in [-8, 7] -> uint8 [N, K/2] (low nibble = even k)."""
    w = np.asarray(w, np.int16)
    return ((w[:, 0::2] & 0xF) | ((w[:, 1::2] & 0xF) << 4)).astype(np.uint8)
