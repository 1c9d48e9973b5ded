"""Pin the CPU oracle before trusting it: the reference's known-answer tests, vectors written by
the reference itself, closed forms and brute force. CPU only."""
from __future__ import annotations

import json
import struct
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import golden as G
from oracle import numerics as F

GOLD = Path(__file__).resolve().parent / "golden"
KAT = json.loads((GOLD / "kats.json").read_text())
VEC = np.load(GOLD / "ref_vectors.npz")
f32 = np.float32


def val(v):
    """A KAT scalar: number, 'nan'/'inf'/'-inf', '0x..' fp32 bits, '2^e' or 'a/b'."""
    if isinstance(v, (int, float)):
        return f32(v)
    if v.startswith("0x"):
        return np.array([int(v, 16)], np.uint32).view(f32)[0]
    if v.startswith("2^"):
        return f32(2.0 ** int(v[2:]))
    if v.startswith("-2^"):
        return f32(-(2.0 ** int(v[3:])))
    if "/" in v:
        a, b = v.split("/")
        return f32(float(a) / float(b))
    return f32(float(v))


def u(x) -> np.ndarray:
    return np.asarray(x, f32).view(np.uint32)


def same_bits(a, b) -> bool:
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and a.dtype == b.dtype and a.tobytes() == b.tobytes()


# ---------------------------------------------------------------- reference KATs
def test_kat_q8():
    k = KAT["q8"]
    x = np.array([val(v) for v in k["x"]], f32)
    assert F.q8(x, f32(k["inv"])).tolist() == k["q"]


def test_kat_bf16():
    k = KAT["bf16"]
    x = np.array([int(b, 16) for b in k["in_bits"]], np.uint32).view(f32)
    assert F.to_bf16_bits(x).tolist() == [int(b, 16) for b in k["out_bits"]]


def test_kat_i2f():
    k = KAT["i2f"]
    assert F.i2f(np.array(k["i"])).tolist() == k["f"]


def test_kat_ftz():
    d = np.array([KAT["ftz"]["denormal"]], f32)
    assert F.ftz(d)[0] == 0 and u(F.ftz(-d))[0] == 0x80000000
    t = np.array([KAT["ftz"]["tiny_product_operand"]], f32)
    assert F.fmul(t, t)[0] == 0


def test_kat_canonical_nan():
    k = KAT["canonical_nan"]
    for op, a, b in k["cases"]:
        fa, fb = np.array([val(a)]), np.array([val(b)])
        r = F.fmul(fa, fb) if op == "mul" else F.fadd(fa, fb)
        assert u(r)[0] == int(k["result_bits"], 16)


def test_kat_relu_relu6():
    k = KAT["relu_signed_zero"]
    x = np.array([val(v) for v in k["x"]], f32)
    assert u(F.act_fn(x, F.ACT_RELU)).tolist() == [int(b, 16) for b in k["out_bits"]]
    k = KAT["relu6"]
    x = np.array([val(v) for v in k["x"]], f32)
    assert F.act_fn(x, F.ACT_RELU6).tolist() == k["y"]


def test_kat_recip():
    k = KAT["recip_specials"]
    x = np.array([val(v) for v in k["x"]], f32)
    assert u(F.recip_f(x)).tolist() == [int(b, 16) for b in k["y_bits"]]
    lo, hi = KAT["recip_powers_of_two"]["exponents"]
    p2 = np.ldexp(1.0, np.arange(lo, hi + 1)).astype(f32)
    assert (F.recip_f(p2) == (1 / p2.astype(np.float64)).astype(f32)).all()
    rng = np.random.default_rng(30)
    x = (np.exp(rng.uniform(-87.3, 87.3, 100000)) * rng.choice([-1, 1], 100000)).astype(f32)
    ref = 1 / x.astype(np.float64)
    err = np.abs(F.recip_f(x).astype(np.float64) - ref) / np.spacing(np.abs(ref).astype(f32))
    assert err.max() <= KAT["recip_ulp_bound"]["max_ulp"]


def test_kat_exp():
    k = KAT["exp_specials"]
    x = np.array([val(v) for v in k["x"]], f32)
    y = F.exp_f(x)
    want = np.array([val(v) for v in k["y"]], f32)
    assert np.array_equal(np.isnan(y), np.isnan(want))
    assert (y[~np.isnan(y)] == want[~np.isnan(want)]).all()
    rng = np.random.default_rng(30)
    x = rng.uniform(-87.3, 88.7, 100000).astype(f32)
    ref = np.exp(x.astype(np.float64))
    err = np.abs(F.exp_f(x).astype(np.float64) - ref) / np.spacing(ref.astype(f32))
    assert err.max() <= KAT["exp_ulp_bound"]["max_ulp"]


def test_kat_quant_rows():
    k = KAT["quant_rows"]
    x = np.array(k["rows"], f32)
    q, s = F.quant_rows(x)
    z = k["zero_row"]
    assert q.dtype == np.int8 and np.abs(q.astype(int)).max() <= 127
    assert (q[z] == 0).all() and s[z] == 0
    assert q[0, 1] == k["q_0_1"] and s[0] == F.fmul(f32(2), F.INV127)
    assert np.abs(q.astype(np.float64) * s[:, None] - x).max() < k["max_abs_dequant_error"]


def test_kat_quantize_weight4():
    k = KAT["quantize_weight4"]
    w = np.zeros(k["shape"], f32)
    w[0, :8] = k["row0_first8"]
    w[1, 128:130] = k["row1_128_130"]
    q, s = G.quantize_weight4(w)
    assert q.shape == (16, 128) and s.shape == (16, 2)
    assert q[0, :4].tolist() == k["q_row0_first4"]
    assert s[0, 0] == np.float16(k["scale00_fp16"]).view(np.uint16)
    assert s[1, 1] == np.float16(val(k["scale11_fp16"])).view(np.uint16)
    assert (q[1, 64] & 15) == k["q_1_64_lo"] and (q[1, 64] >> 4) == k["q_1_64_hi"]


def test_kat_fp16_storage():
    """Every binary16 pattern widens exactly and every finite one narrows back to itself; the
    reference's three narrowing KATs (test_fp16_state.py:28-39)."""
    k = KAT["fp16_storage"]
    h = np.arange(65536, dtype=np.uint16)
    wide = F.from_fp16_bits(h)
    for i in range(0, 65536, 1):
        v = struct.unpack("<e", int(h[i]).to_bytes(2, "little"))[0]
        got = int(wide.view(np.uint32)[i])
        if v != v:
            assert got == int(k["nan_from_bits_result_bits"], 16)
        else:
            assert got == struct.unpack("<I", struct.pack("<f", v))[0], hex(i)
    finite = np.isfinite(wide)
    assert k["every_finite_pattern_round_trips"]
    assert same_bits(F.to_fp16_bits(wide[finite]), h[finite])
    assert wide[1] == val(k["from_bits_0x0001"])
    x = np.array([val(v) for v in k["to_bits_x"]], f32)
    assert F.to_fp16_bits(x).tolist() == [int(b, 16) for b in k["to_bits_h"]]


def fp16_bits_exact(x: np.float32) -> int:
    """binary16 encoding of an fp32 value by exact rational rounding: the nearest multiple of
    the binade's spacing (2^-24 below 2^-14), ties to the even multiple, 65520 and up to
    infinity, NaN to 0x7E00."""
    v = float(x)
    if v != v:
        return 0x7E00
    sign = 0x8000 if np.signbit(x) else 0
    a = Fraction(abs(v)) if abs(v) != float("inf") else None
    if a is None or a >= 65520:
        return sign | 0x7C00
    e = -14
    while e < 15 and a >= Fraction(2) ** (e + 1):
        e += 1
    step = Fraction(2) ** (e - 10)
    n = round(a / step)                      # Fraction rounds half to even
    if a < Fraction(2) ** -14:
        return sign | n                      # subnormal (n = 1024 is the smallest normal)
    if n == 2048:
        e, n = e + 1, 1024
    return sign | ((e + 15) << 10) | (n - 1024)


def test_to_fp16_bits_against_exact_rounding():
    """to_fp16_bits (numerics.py:14-18) against rounding by exact rationals: every half-way
    point between adjacent finite halves and its two fp32 neighbours, both signs, the overflow
    edge, subnormals, and random fp32 encodings."""
    a = np.arange(0x7BFF, dtype=np.uint16).view(np.float16).astype(f32)
    b = np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16).astype(f32)
    mid = (a + b) * f32(0.5)
    pick = np.random.default_rng(5).choice(mid.size, 3000, replace=False)
    m = mid[pick]
    rnd = np.random.default_rng(6).integers(0, 2 ** 32, 3000, dtype=np.uint32).view(f32)
    edge = np.array([65504, 65519.996, 65520, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14,
                     -0.0, 0.0, np.inf, -np.inf, np.nan], f32)
    x = np.concatenate([m, -m, np.nextafter(m, f32(0)), np.nextafter(m, f32(np.inf)), edge, rnd])
    got = F.to_fp16_bits(x)
    want = np.array([fp16_bits_exact(v) for v in x], np.uint16)
    assert same_bits(got, want)


def test_quantize_weight_against_exact_arithmetic():
    """The host INT8 weight quantizer (compiler.py:51-57) against exact rationals: the scale is
    the float64 nearest amax/127 (1.0 for an all-zero row), each q the nearest integer to the
    float64 nearest w/s, ties to even, within +-127; the scale stored as the fp32 nearest it.
    Per channel and per tensor."""
    rng = np.random.default_rng(11)
    w = rng.normal(0, 0.3, (6, 40))
    w[2] = 0.0
    w[3, :6] = [127.0, 2.5, -2.5, 3.5, -0.5, 1.5]
    w[3, 6:] = 0.0
    for per_channel in (True, False):
        q, s = G.quantize_weight(w, per_channel)
        rows = w if per_channel else w.reshape(1, -1)
        assert q.shape == w.shape and q.dtype == np.int8 and s.dtype == f32
        assert s.shape == ((w.shape[0],) if per_channel else (1,))
        for r in range(rows.shape[0]):
            amax = max(abs(Fraction(float(t))) for t in rows[r])
            s64 = float(amax / 127) if amax else 1.0
            assert s[r] == f32(struct.unpack("<f", struct.pack("<f", s64))[0])
            want = [max(-127, min(127, round(Fraction(float(Fraction(float(t)) / Fraction(s64))))))
                    for t in rows[r]]
            got = (q if per_channel else q.reshape(1, -1))[r].tolist()
            assert got == want
    q, s = G.quantize_weight(w)
    assert s[2] == 1.0 and (q[2] == 0).all()
    assert s[3] == 1.0 and q[3, :6].tolist() == [127, 2, -2, 4, 0, 2]


def test_kat_align_extremes():
    k = KAT["align_extremes"]
    x = np.zeros((4, 128), f32)
    for r in range(4):
        vals = [val(v) for v in k[f"row{r}"]]
        x[r, :len(vals)] = vals
    q, s = F.align_w4_groups(x)
    e = k["expect"]
    assert q.shape == x.shape and q.dtype == np.int16 and s.shape == (4, 1)
    assert s[0, 0] == val(e["s00"]) and q[0, 0] == e["q00"] and q[0, 1] == e["q01"]
    assert q[0, 2] == e["q02"] and q[0, 3] == e["q03"] and (q[0, 4:10] == e["q0_4to10"]).all()
    assert s[3, 0] == val(e["s30"]) and q[3, 0] == e["q30"] and q[3, 1] == e["q31"]
    assert s[1, 0] == val(e["s10"]) and q[1, 0] == e["q10"] and q[1, 2] == e["q12"] and q[1, 4] == e["q14"]
    assert s[2, 0] == val(e["s20"]) and q[2, 0] == e["q20"] and q[2, 1] == e["q21"]
    zq, zs = F.align_w4_groups(np.zeros((1, 128), f32))
    assert (zq == 0).all() and zs[0, 0] == 0


def test_kat_align_nan_inf():
    k = KAT["align_nan_inf"]
    x = np.zeros((3, 128), f32)
    for r in range(3):
        for c, v in k[f"row{r}"].items():
            x[r, int(c)] = val(v)
    q, s = F.align_w4_groups(x)
    assert u(s[0, 0]) == 0x7FC00000 and (q[0] == 0).all()
    assert np.isposinf(s[1, 0]) and q[1, 0] == 16384 and q[1, 1] == -16384 and (q[1, 2:] == 0).all()
    assert np.isposinf(s[2, 0]) and q[2, 0] == -16384


def test_kat_worked_example():
    """The contract document's fused GEMM: QM_CHANNEL, bias, RELU, bf16 output."""
    k = KAT["worked_example"]
    rng = np.random.default_rng(k["seed"])
    M, N, K = k["M"], k["N"], k["K"]
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    W = rng.integers(-128, 128, (N, K), dtype=np.int8)
    S = (rng.uniform(0.5, 2.0, N) / 4096).astype(f32)
    B = rng.uniform(-8, 8, N).astype(f32)
    acc = G.int_dot(A, W)
    assert acc[0, 1] == k["acc_0_1"]
    assert u(S[1]) == int(k["scale_1_bits"], 16) and u(B[1]) == int(k["bias_1_bits"], 16)
    v = G.epilogue_rowcol(acc, None, S, B, F.ACT_NONE)
    assert u(v[0, 1]) == int(k["value_0_1_bits"], 16)
    y = G.gemm_rowcol(A, None, W, S, B, act=F.ACT_RELU, out=G.OUT_BF16)
    assert y[0, 1] == int(k["bf16_0_1"], 16)


def test_kat_nan_reaches_output():
    A = np.zeros((1, 16), np.int8)
    W = np.ones((16, 16), np.int8)
    y = G.gemm_rowcol(A, None, W, np.array([np.inf], f32))
    assert (u(y) == 0x7FC00000).all()


def test_kat_w4_inf_everywhere():
    x = np.zeros((1, 512), f32)
    x[0, 0] = np.inf
    wp, ws = G.quantize_weight4(np.ones((16, 512), f32))
    assert np.isposinf(G.gemm_w4(x, wp, ws)).all()


def test_no_fma():
    """Two roundings, not a fused multiply-add: find a distinguishing case and check the oracle."""
    rng = np.random.default_rng(1)
    for _ in range(10000):
        acc = int(rng.integers(-2**20, 2**20))
        s, b = f32(rng.uniform(1e-4, 1e-2)), f32(rng.uniform(-50, 50))
        two = f32(f32(f32(acc) * s) + b)
        fused = f32(np.float64(f32(acc)) * np.float64(s) + np.float64(b))
        if two != fused:
            break
    else:
        pytest.skip("no distinguishing case")
    y = F.fadd(F.fmul(F.i2f(acc), s), b)
    assert y == two and y != fused


# ---------------------------------------------------------------- vectors written by the reference
@pytest.mark.parametrize("name,fn", [("recip", F.recip_f), ("exp", F.exp_f)])
def test_ref_vectors_primitives(name, fn):
    assert same_bits(fn(VEC[name + "_x"]), VEC[name + "_y"])


@pytest.mark.parametrize("code", range(8))
def test_ref_vectors_activations(code):
    assert same_bits(F.act_fn(VEC["act_x"], code), VEC[f"act{code}_y"])


@pytest.mark.parametrize("name", ["qr_1x1024", "qr_4x1024", "qr_4x3072", "qr_1x6912", "qr_3x2048", "qr_edge"])
def test_ref_vectors_quant_rows(name):
    q, s = F.quant_rows(VEC[name + "_x"])
    assert same_bits(q, VEC[name + "_q"]) and same_bits(s, VEC[name + "_s"])


def w4_case(i: int):
    k = f"w4_{i}"
    m, n, K, half, bias, act, fmt, osb = (int(v) for v in VEC[k + "_meta"])
    return dict(x=VEC[k + "_x"], Wp=VEC[k + "_wp"], ws=VEC[k + "_ws"],
                bias=VEC[k + "_bias"] if bias else None, act=act, out=fmt,
                out_scale=np.array([osb], np.uint32).view(f32)[0], half=bool(half), y=VEC[k + "_y"])


@pytest.mark.parametrize("i", range(8))
def test_ref_vectors_w4_gemm(i):
    c = w4_case(i)
    y = G.gemm_w4(c["x"], c["Wp"], c["ws"], bias=c["bias"], act=c["act"], out=c["out"],
                  out_scale=c["out_scale"], x_is_bf16=c["half"])
    assert np.ascontiguousarray(y).tobytes() == c["y"].tobytes()


# ---------------------------------------------------------------- closed forms, brute force
def _round_f32(q: Fraction) -> np.float32:
    """An exact rational rounded once to fp32 (RNE), via float64 when that is exact."""
    d = float(q)
    assert Fraction(d) == q, "needs an exactly representable float64"
    return f32(d)


def test_fmul_fadd_against_exact_arithmetic():
    """fmul/fadd on normal results equal the exact rational result rounded once to fp32."""
    rng = np.random.default_rng(7)
    a = (rng.normal(0, 1, 5000) * np.exp2(rng.integers(-30, 30, 5000))).astype(f32)
    b = (rng.normal(0, 1, 5000) * np.exp2(rng.integers(-30, 30, 5000))).astype(f32)
    pm, pa = F.fmul(a, b), F.fadd(a, b)
    for i in range(0, 5000, 7):
        assert pm[i] == _round_f32(Fraction(float(a[i])) * Fraction(float(b[i])))
        exact = Fraction(float(a[i])) + Fraction(float(b[i]))
        if Fraction(float(exact)) == exact:
            assert pa[i] == _round_f32(exact)


def test_int_dot_brute_force():
    rng = np.random.default_rng(3)
    A = rng.integers(-128, 128, (3, 48), dtype=np.int8)
    W = rng.integers(-128, 128, (5, 48), dtype=np.int8)
    acc = G.int_dot(A, W)
    for m in range(3):
        for n in range(5):
            assert acc[m, n] == sum(int(A[m, k]) * int(W[n, k]) for k in range(48))


def test_epilogue_rowcol_scalar_sequence():
    """Each element is (((i2f(acc) * srow) * scol) + bias), each step rounded once, in that order:
    reversing the two scale products or fusing a step changes some bits."""
    rng = np.random.default_rng(11)
    M, N, K = 4, 64, 1024
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    W = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sr = rng.uniform(1e-3, 1e-1, M).astype(f32)
    sc = rng.uniform(1e-3, 1e-2, N).astype(f32)
    b = rng.normal(0, 1, N).astype(f32)
    y = G.gemm_rowcol(A, sr, W, sc, b)
    acc = G.int_dot(A, W)
    swapped = 0
    for m in range(M):
        for n in range(N):
            a = f32(int(acc[m, n]))                      # int -> float32 conversion rounds once
            t = _round_f32(Fraction(float(a)) * Fraction(float(sr[m])))
            t = _round_f32(Fraction(float(t)) * Fraction(float(sc[n])))
            assert y[m, n] == f32(float(Fraction(float(t)) + Fraction(float(b[n]))))
            r = _round_f32(Fraction(float(a)) * Fraction(float(sc[n])))
            r = _round_f32(Fraction(float(r)) * Fraction(float(sr[m])))
            swapped += int(r != t)
    assert swapped > 0, "the scale order must matter for some element"


def test_w4_group_dots_brute_force():
    rng = np.random.default_rng(5)
    aq = rng.integers(-16384, 16385, (2, 256)).astype(np.int16)
    w = rng.integers(-8, 8, (3, 256)).astype(np.int16)
    d = G.w4_group_dots(aq, w)
    for m in range(2):
        for n in range(3):
            for g in range(2):
                assert d[m, n, g] == sum(int(aq[m, k]) * int(w[n, k]) for k in range(128 * g, 128 * g + 128))
    assert (G.unpack_int4(G.pack_int4(w)) == w).all()


def test_align_independent_scalar():
    """Bit-level scalar restatement of the aligner on random normal bit patterns, RNE ties
    included (the reference checks its own aligner the same way, tests/test_w4a16.py:76-105)."""
    rng = np.random.default_rng(10)
    xb = (rng.integers(1, 254, (3, 256), dtype=np.uint32) << 23) | rng.integers(0, 1 << 23, (3, 256), dtype=np.uint32)
    xb |= rng.integers(0, 2, xb.shape, dtype=np.uint32) << 31
    # plant exact ties: a significand whose dropped bits are exactly one half
    xb[0, 5] = (140 << 23) | 0x00000400
    xb[0, 6] = (140 << 23) | 0x00000C00
    q, s = F.align_w4_groups(xb.view(f32))
    for m in range(3):
        for g in range(2):
            grp = [int(v) for v in xb[m, 128 * g:128 * g + 128]]
            top = max(14, max((v >> 23) & 0xFF for v in grp))
            assert int(s[m, g].view(np.uint32)) == (top - 13) << 23
            for j, v in enumerate(grp):
                e = (v >> 23) & 0xFF
                sig = (1 << 23) | (v & 0x7FFFFF)
                sh = 10 + top - e
                if sh >= 25:
                    want = 0
                else:
                    base, rem = divmod(sig, 1 << sh)
                    half = 1 << (sh - 1) if sh else 0
                    want = base + (sh > 0 and (rem > half or (rem == half and base % 2 == 1)))
                if v >> 31:
                    want = -want
                assert int(q[m, 128 * g + j]) == want


def test_ksplit_order_and_blocks():
    """The K split adds per-block fp32 partials in block order; per-block i2f rounding makes the
    split visible in the bits, and the two splits of K=6912 (3456+3456, 4096+2816) differ."""
    rng = np.random.default_rng(2)
    M, N, K = 1, 256, 6912
    x = rng.normal(0, 1, (M, K)).astype(f32)
    q, sr = F.quant_rows(x)
    W = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sc = rng.uniform(1e-3, 1e-2, N).astype(f32)
    whole = G.gemm_rowcol(q, sr, W, sc)
    ya = G.gemm_rowcol_ksplit(q, sr, [W[:, :3456], W[:, 3456:]], sc)
    yb = G.gemm_rowcol_ksplit(q, sr, [W[:, :4096], W[:, 4096:]], sc)
    p0 = G.gemm_rowcol(q[:, :4096], sr, W[:, :4096], sc)
    p1 = G.gemm_rowcol(q[:, 4096:], sr, W[:, 4096:], sc)
    assert same_bits(yb, F.fadd(p0, p1))
    assert not same_bits(ya, yb) and not same_bits(whole, ya)
    assert same_bits(G.gemm_rowcol_ksplit(q, sr, [W], sc), whole)
    three = G.gemm_rowcol_ksplit(q, sr, [W[:, :2304], W[:, 2304:4608], W[:, 4608:]], sc)
    p = [G.gemm_rowcol(q[:, a:b], sr, W[:, a:b], sc) for a, b in ((0, 2304), (2304, 4608), (4608, 6912))]
    assert same_bits(three, F.fadd(F.fadd(p[0], p[1]), p[2]))


def test_results_independent_of_m_and_n_split():
    """The contract's results cannot depend on tiling (golden.py:3-4)."""
    rng = np.random.default_rng(4)
    A = rng.integers(-127, 128, (6, 96), dtype=np.int8)
    W = rng.integers(-127, 128, (48, 96), dtype=np.int8)
    sr = rng.uniform(1e-2, 1, 6).astype(f32)
    sc = rng.uniform(1e-3, 1e-2, 48).astype(f32)
    full = G.gemm_rowcol(A, sr, W, sc)
    assert same_bits(np.vstack([G.gemm_rowcol(A[i:i + 1], sr[i:i + 1], W, sc) for i in range(6)]), full)
    assert same_bits(np.hstack([G.gemm_rowcol(A, sr, W[j:j + 16], sc[j:j + 16]) for j in range(0, 48, 16)]), full)
