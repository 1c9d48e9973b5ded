"""Row, elementwise, rotary and fp32 dot-product steps of the golden model, restated in numpy --
TEST INFRASTRUCTURE ONLY.

The same single-rounding contract as oracle/numerics.py: every fp32 add or multiply is one RNE
step, subnormal inputs and results flush to a zero of the same sign, NaN is canonical. The row
sums follow the contract's 16-lane order: element j of a row goes to lane j mod 16, each lane adds
its elements in order from +0, then the 16 lanes fold pairwise in four levels.

Reference: tars_mini/numerics.py and tars_mini/golden.py (file:line cited per function).
"""
from __future__ import annotations

import numpy as np

from . import numerics as F

f32, u32 = np.float32, np.uint32
LANES = 16
RSQRT_SEED = 0x5F3759DF                    # numerics.py:122


# ---------------------------------------------------------------- order-free max, 16-lane sum
def fmax(a, b) -> np.ndarray:
    """max with one answer for every pair (numerics.py:293-303): NaN (canonical) if either is NaN;
    of two equal values, the one whose sign is the AND of both signs (-0 only if both are -0);
    inputs flushed first."""
    a, b = F.ftz(a), F.ftz(b)
    ab, bb = F.bits(a), F.bits(b)
    with np.errstate(invalid="ignore"):
        big = np.where(a > b, a, b).astype(f32)
        same = a == b
    tie = ((ab & bb & u32(F.SIGN)) | (ab & u32(0x7FFFFFFF))).view(f32)
    out = np.where(same, tie, big).astype(f32)
    return F.canon(np.where(F.isnan(a) | F.isnan(b), f32(np.nan), out).astype(f32))


def sum16(v) -> np.ndarray:
    """Row sums in the contract's lane order (numerics.py:306-316). v: [M, N] -> [M]."""
    v = np.asarray(v, f32)
    lanes = np.zeros((v.shape[0], LANES), f32)
    for j in range(v.shape[1]):
        lanes[:, j % LANES] = F.fadd(lanes[:, j % LANES], v[:, j])
    while lanes.shape[1] > 1:
        lanes = F.fadd(lanes[:, 0::2], lanes[:, 1::2])
    return lanes[:, 0]


def rsqrt_f(x) -> np.ndarray:
    """1/sqrt(x) by the reference's fixed sequence (numerics.py:171-191).

    E = biased exponent - 127 = 2k + j (j in {0, 1}); m = x with exponent field 127 + j, so
    m in [1, 4); seed bits(y0) = SEED - (bits(m) >> 1); three Newton steps
    y <- y + y * (1/2 + -(1/2 * ((m * y) * y))); then -k is added to y's exponent field.
    Specials: +-0 -> +-inf, +inf -> +0, negative or NaN -> canonical NaN."""
    x = F.ftz(x)
    xb = F.bits(x).astype(np.int64)
    E = ((xb >> 23) & 0xFF) - 127
    j, k = E & 1, E >> 1                  # floor halving, so E = 2k + j also for E < 0
    mbits = (xb & F.MANT) | ((127 + j) << 23)
    m = F.from_bits(mbits)
    y = F.from_bits(RSQRT_SEED - (mbits >> 1))
    for _ in range(3):
        t = F.fadd(F.HALF, F.neg(F.fmul(F.HALF, F.fmul(F.fmul(m, y), y))))
        y = F.fadd(y, F.fmul(y, t))
    y = F.add_to_exponent(y, -k)
    mag = xb & 0x7FFFFFFF
    y = np.where(mag == 0, F.from_bits((xb & F.SIGN) | F.EXPO), y)
    y = np.where(xb == F.EXPO, f32(0), y)
    with np.errstate(invalid="ignore"):
        bad = F.isnan(x) | (x < f32(0))
    return F.canon(np.where(bad, f32(np.nan), y).astype(f32))


def inv_n(n: int) -> np.float32:
    """1/N as the contract forms it: recip(i2f(N)) (numerics.py:336-338)."""
    return F.recip_f(F.i2f(np.array([n], np.int64)))[0]


# ---------------------------------------------------------------- row functions (OP_ROW)
def softmax_rows(x) -> np.ndarray:
    """mx = row max; e = exp(x + -mx); y = e * recip(sum16(e)) (numerics.py:328-333)."""
    x = F.ftz(np.asarray(x, f32))
    mx = F.max16(x)[:, None]
    e = F.exp_f(F.fadd(x, F.neg(mx)))
    return F.fmul(e, F.recip_f(sum16(e))[:, None])


def softmax_rows_causal(x, valid) -> np.ndarray:
    """Softmax over the first valid[m] elements of row m; the others are +0 in the sum and in the
    output (numerics.py:362-371)."""
    x = F.ftz(np.asarray(x, f32))
    M, N = x.shape
    valid = np.asarray(valid, np.int64)
    keep = np.arange(N)[None, :] < valid[:, None]
    mx = np.array([F.max16(x[m:m + 1, :valid[m]])[0] for m in range(M)], f32)[:, None]
    e = np.where(keep, F.exp_f(F.fadd(x, F.neg(mx))), f32(0)).astype(f32)
    return F.fmul(e, F.recip_f(sum16(e))[:, None])


def _scale_shift(y, gamma, beta):
    y = F.fmul(y, np.asarray(gamma, f32)[None, :])
    return y if beta is None else F.fadd(y, np.asarray(beta, f32)[None, :])


def layernorm_rows(x, gamma, beta, eps) -> np.ndarray:
    """mean = sum16(x) * 1/N; d = x + -mean; rs = rsqrt(sum16(d * d) * 1/N + eps);
    y = (d * rs) * gamma [+ beta] (numerics.py:341-350)."""
    x = F.ftz(np.asarray(x, f32))
    k = inv_n(x.shape[1])
    d = F.fadd(x, F.neg(F.fmul(sum16(x), k)[:, None]))
    rs = rsqrt_f(F.fadd(F.fmul(sum16(F.fmul(d, d)), k), f32(eps)))[:, None]
    return _scale_shift(F.fmul(d, rs), gamma, beta)


def rmsnorm_rows(x, gamma, beta, eps) -> np.ndarray:
    """rs = rsqrt(sum16(x * x) * 1/N + eps); y = (x * rs) * gamma [+ beta] (numerics.py:353-358)."""
    x = F.ftz(np.asarray(x, f32))
    rs = rsqrt_f(F.fadd(F.fmul(sum16(F.fmul(x, x)), inv_n(x.shape[1])), f32(eps)))[:, None]
    return _scale_shift(F.fmul(x, rs), gamma, beta)


def l2norm_rows(x, gamma, beta, eps) -> np.ndarray:
    """RMSNorm without the 1/N: rs = rsqrt(sum16(x * x) + eps) (numerics.py:374-380)."""
    x = F.ftz(np.asarray(x, f32))
    rs = rsqrt_f(F.fadd(sum16(F.fmul(x, x)), f32(eps)))[:, None]
    return _scale_shift(F.fmul(x, rs), gamma, beta)


# ---------------------------------------------------------------- fp32 dot products (OP_FDOT)
def fdot_nt(a, b) -> np.ndarray:
    """y[m][n] = sum16 over k of a[m][k] * b[n][k] (numerics.py:393-399). a [M, K], b [N, K]."""
    a, b = F.ftz(np.asarray(a, f32)), F.ftz(np.asarray(b, f32))
    M, K = a.shape
    N = b.shape[0]
    return sum16(F.fmul(a[:, None, :], b[None, :, :]).reshape(M * N, K)).reshape(M, N)


def fdot_nn(a, b) -> np.ndarray:
    """y[m][n] = ((+0 + a[m][0] * b[0][n]) + a[m][1] * b[1][n]) + ..., k in order
    (numerics.py:402-409). a [M, K], b [K, N]."""
    a, b = F.ftz(np.asarray(a, f32)), F.ftz(np.asarray(b, f32))
    y = np.zeros((a.shape[0], b.shape[1]), f32)
    for k in range(a.shape[1]):
        y = F.fadd(y, F.fmul(a[:, k:k + 1], b[k:k + 1, :]))
    return y


# ---------------------------------------------------------------- rotary embedding (OP_ROPE)
def rope_rows(x, tab, rows_per_pos: int, rot: int) -> np.ndarray:
    """Rotary embedding of the first rot elements of each row (numerics.py:412-424). Table row
    t = [cos(0..h-1), sin(0..h-1)], h = rot / 2; row m uses table row m // rows_per_pos:
    y[i] = x[i] * c + -(x[i+h] * s), y[i+h] = x[i+h] * c + x[i] * s; later elements unchanged."""
    x = F.ftz(np.asarray(x, f32))
    h = rot // 2
    t = F.ftz(np.asarray(tab, f32))[np.arange(x.shape[0]) // rows_per_pos]
    c, s = t[:, :h], t[:, h:rot]
    y = x.copy()
    y[:, :h] = F.fadd(F.fmul(x[:, :h], c), F.neg(F.fmul(x[:, h:rot], s)))
    y[:, h:rot] = F.fadd(F.fmul(x[:, h:rot], c), F.fmul(x[:, :h], s))
    return y


# ---------------------------------------------------------------- elementwise (OP_ELT)
ELT_MUL, ELT_ADD, ELT_MULADD, ELT_SUB = 0, 1, 2, 3       # contract.py:63-66
BM_DENSE, BM_ROW, BM_COL, BM_SCALAR = 0, 1, 2, 3


def elt(op: int, a, b, c=None, act: int = F.ACT_NONE) -> np.ndarray:
    """y = act(a) * b, act(a) + b, act(a) + -b, or c + act(a) * b, each step rounded once
    (golden.py:393-418). a, b, c are full [M, N] operands (broadcasts already expanded)."""
    a = F.act_fn(np.asarray(a, f32), act)
    b = np.asarray(b, f32)
    if op == ELT_MUL:
        return F.fmul(a, b)
    if op == ELT_ADD:
        return F.fadd(a, b)
    if op == ELT_SUB:
        return F.fadd(a, F.neg(F.ftz(b)))
    if op == ELT_MULADD:
        return F.fadd(np.asarray(c, f32), F.fmul(a, b))
    raise ValueError(f"ELT op {op}")


def broadcast_b(bvals, mode: int, M: int, N: int) -> np.ndarray:
    """B(m, n) for the broadcast modes (contract.py:67-68, golden.py:404-409): DENSE B[m][n],
    ROW B[n], COL B[m], SCALAR B[0]. bvals: [M, N] for DENSE, else the 1-D values read."""
    v = np.asarray(bvals, f32)
    if mode == BM_DENSE:
        return v.reshape(M, N)
    if mode == BM_ROW:
        return np.broadcast_to(v[None, :N], (M, N))
    if mode == BM_COL:
        return np.broadcast_to(v[:M, None], (M, N))
    return np.broadcast_to(v[:1][None, :], (M, N))
