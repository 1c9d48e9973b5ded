"""Pins of the oracle's row, rotary, elementwise and fp32 dot-product functions (oracle/rowops.py):
vectors the reference golden model itself wrote (tests/golden/rowop_vectors.npz), the reference
tests' known answers and independent restatements, exact rational arithmetic, and torch."""
from __future__ import annotations

from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import numerics as F
from oracle import rowops as R

VEC = np.load(Path(__file__).resolve().parent / "golden" / "rowop_vectors.npz")
f32, u32 = np.float32, np.uint32


def same(a, b) -> bool:
    return np.array_equal(np.asarray(a, f32).view(u32), np.asarray(b, f32).view(u32))


def fb(*bits) -> np.ndarray:
    return np.array(bits, u32).view(f32)


# ---------------------------------------------------------------- reference-written vectors
def test_rsqrt_reference_vectors():
    assert same(R.rsqrt_f(VEC["rsqrt_x"]), VEC["rsqrt_y"])


@pytest.mark.parametrize("name", ["sm_4x64", "sm_3x256", "sm_2x1024", "sm_5x16", "sm_edge"])
def test_softmax_reference_vectors(name):
    assert same(R.softmax_rows(VEC[name + "_x"]), VEC[name + "_y"])


@pytest.mark.parametrize("name", ["smc", "smc_edge"])
def test_softmax_causal_reference_vectors(name):
    assert same(R.softmax_rows_causal(VEC[name + "_x"], VEC[name + "_valid"]), VEC[name + "_y"])


@pytest.mark.parametrize("name", ["n_3x1024", "n_2x2048", "n_4x128", "n_2x16", "n_edge"])
@pytest.mark.parametrize("fn", ["ln", "rms", "l2"])
def test_norm_reference_vectors(name, fn):
    f = {"ln": R.layernorm_rows, "rms": R.rmsnorm_rows, "l2": R.l2norm_rows}[fn]
    x, g, b = VEC[name + "_x"], VEC[name + "_g"], VEC[name + "_b"]
    assert same(f(x, g, b, f32(1e-6)), VEC[f"{name}_{fn}_eps6_y"])
    if name == "n_edge":
        assert same(f(x, g, None, f32(0.0)), VEC[f"{name}_{fn}_eps0_y"])
    else:
        assert same(f(x, g, None, f32(1e-5)), VEC[f"{name}_{fn}_eps5_nob_y"])


def test_fdot_and_rope_reference_vectors():
    assert same(R.fdot_nt(VEC["fnt_a"], VEC["fnt_b"]), VEC["fnt_y"])
    assert same(R.fdot_nn(VEC["fnn_a"], VEC["fnn_b"]), VEC["fnn_y"])
    assert same(R.rope_rows(VEC["rope_x"], VEC["rope_tab"], 2, 64), VEC["rope_y"])


# ---------------------------------------------------------------- reference known answers
def test_rsqrt_known_answers():
    """tests/test_golden.py:320 and :323-333: rsqrt(4) = 0.5; +0 -> +inf, -0 -> -inf, +inf -> +0,
    negative values and -inf -> canonical NaN."""
    assert R.rsqrt_f(np.array([4.0], f32))[0] == f32(0.5)
    y = R.rsqrt_f(np.array([0.0, -0.0, np.inf, -1.0, -np.inf], f32)).view(u32)
    assert list(y) == [0x7F800000, 0xFF800000, 0x00000000, 0x7FC00000, 0x7FC00000]


def test_rsqrt_error_bound():
    """tests/test_golden.py:308-317: at most 1.25 ulp from 1/sqrt(x) over normal inputs."""
    rng = np.random.default_rng(4)
    x = np.exp2(rng.uniform(-120, 120, 20000)).astype(f32)
    y = R.rsqrt_f(x).astype(np.float64)
    ref = 1.0 / np.sqrt(x.astype(np.float64))
    ulp = np.spacing(ref.astype(f32)).astype(np.float64)
    assert (np.abs(y - ref) / ulp).max() <= 1.25


def test_rsqrt_exact_at_even_powers_of_two():
    """A closed form: rsqrt(2^(2k)) = 2^-k for every normal even power."""
    k = np.arange(-63, 64)
    assert same(R.rsqrt_f(np.exp2(2.0 * k).astype(f32)), np.exp2(-1.0 * k).astype(f32))


def test_fmax_table():
    """numerics.py:293-303 by cases: ordinary order, +0 against -0 either way gives +0, -0 only
    from two -0, a NaN on either side gives the canonical NaN, subnormals count as zeros."""
    a = fb(0x3F800000, 0x00000000, 0x80000000, 0x80000000, 0x7FC00001, 0x3F800000, 0xFF800000, 0x80000001, 0x00000005)
    b = fb(0x40000000, 0x80000000, 0x00000000, 0x80000000, 0x3F800000, 0xFFC00000, 0xC2C80000, 0x80000000, 0x80000000)
    want = [0x40000000, 0x00000000, 0x00000000, 0x80000000, 0x7FC00000, 0x7FC00000, 0xC2C80000, 0x80000000,
            0x00000000]
    assert list(R.fmax(a, b).view(u32)) == want
    assert list(R.fmax(b, a).view(u32)) == want


def test_causal_softmax_full_rows_equal_plain_softmax():
    """tests/test_v04.py:87-97: valid = N is the plain softmax; the tail of a causal row is +0;
    the valid part is close to the float64 softmax."""
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, (4, 32)).astype(f32)
    assert same(R.softmax_rows_causal(x, [32] * 4), R.softmax_rows(x))
    y = R.softmax_rows_causal(x, [3, 4, 5, 32])
    for m, n in enumerate([3, 4, 5, 32]):
        e = np.exp(x[m, :n].astype(np.float64) - x[m, :n].max())
        assert np.allclose(y[m, :n], e / e.sum(), rtol=1e-5)
        assert (y[m, n:].view(u32) == 0).all()


def test_norms_close_to_float64():
    rng = np.random.default_rng(9)
    x = rng.normal(0, 2, (3, 256)).astype(f32)
    g = rng.normal(1, 0.1, 256).astype(f32)
    b = rng.normal(0, 0.1, 256).astype(f32)
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    ln = (xd - mu) / np.sqrt(((xd - mu) ** 2).mean(1, keepdims=True) + 1e-6) * g + b
    rms = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6) * g + b
    l2 = xd / np.sqrt((xd ** 2).sum(1, keepdims=True) + 1e-6) * g + b
    assert np.allclose(R.layernorm_rows(x, g, b, 1e-6), ln, rtol=1e-5, atol=1e-5)
    assert np.allclose(R.rmsnorm_rows(x, g, b, 1e-6), rms, rtol=1e-5, atol=1e-5)
    assert np.allclose(R.l2norm_rows(x, g, b, 1e-6), l2, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- the 16-lane order
def test_fdot_nt_lane_order_restated_independently():
    """tests/test_v04.py:57-67: the NT dot written out as 16 lane accumulators over k, then the
    pairwise fold; and close to the float64 product."""
    rng = np.random.default_rng(1)
    a = rng.normal(0, 1, (3, 64)).astype(f32)
    b = rng.normal(0, 1, (5, 64)).astype(f32)
    lanes = np.zeros((3, 5, 16), f32)
    for k in range(64):
        lanes[:, :, k % 16] = F.fadd(lanes[:, :, k % 16], F.fmul(a[:, None, k], b[None, :, k]))
    while lanes.shape[2] > 1:
        lanes = F.fadd(lanes[:, :, 0::2], lanes[:, :, 1::2])
    assert same(R.fdot_nt(a, b), lanes[:, :, 0])
    assert np.allclose(R.fdot_nt(a, b), a.astype(np.float64) @ b.T.astype(np.float64), rtol=1e-5, atol=1e-4)


def _rne(q: Fraction) -> np.float32:
    """An exact rational rounded once to fp32 (round to nearest, ties to even), for normal results."""
    if q == 0:
        return f32(0)
    s = -1 if q < 0 else 1
    q = abs(q)
    e = q.numerator.bit_length() - q.denominator.bit_length()
    while Fraction(2) ** e > q:
        e -= 1
    while Fraction(2) ** (e + 1) <= q:
        e += 1
    scaled = q / Fraction(2) ** (e - 23)              # in [2^23, 2^24)
    n, r = divmod(scaled.numerator, scaled.denominator)
    twice = 2 * r
    if twice > scaled.denominator or (twice == scaled.denominator and n % 2):
        n += 1
    return f32(s * n * 2.0 ** (e - 23))


def test_sum16_and_fdot_nn_against_exact_arithmetic():
    """Each step of the 16-lane row sum and of the sequential NN dot is one exactly rounded
    operation: recomputed with exact rationals, rounding after every step. The data mixes
    magnitudes so that a different order (a left fold, or pairwise sums) changes the result."""
    rng = np.random.default_rng(12)
    v = (rng.normal(0, 1, (6, 96)) * np.exp2(rng.integers(-12, 13, (6, 96)))).astype(f32)
    got = R.sum16(v)
    for m in range(6):
        lanes = [Fraction(0)] * 16
        for j in range(96):
            lanes[j % 16] = Fraction(float(_rne(lanes[j % 16] + Fraction(float(v[m, j])))))
        while len(lanes) > 1:
            lanes = [Fraction(float(_rne(lanes[i] + lanes[i + 1]))) for i in range(0, len(lanes), 2)]
        assert got[m] == f32(float(lanes[0]))
    left = np.zeros(6, f32)
    for j in range(96):
        left = F.fadd(left, v[:, j])
    assert not same(left, got), "the data does not separate the lane order from a left fold"

    a = (rng.normal(0, 1, (2, 40)) * np.exp2(rng.integers(-8, 9, (2, 40)))).astype(f32)
    b = (rng.normal(0, 1, (40, 3)) * np.exp2(rng.integers(-8, 9, (40, 3)))).astype(f32)
    y = R.fdot_nn(a, b)
    for m in range(2):
        for n in range(3):
            acc = Fraction(0)
            for k in range(40):
                p = _rne(Fraction(float(a[m, k])) * Fraction(float(b[k, n])))
                acc = Fraction(float(_rne(acc + Fraction(float(p)))))
            assert y[m, n] == f32(float(acc))


# ---------------------------------------------------------------- rotary, elementwise
def test_rope_matches_torch_rotate_half():
    """tests/test_v04.py:69-84: torch's rotate_half RoPE, elementwise fp32 ops, bit for bit."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    x, Rr, G = rng.normal(0, 1, (6, 128)).astype(f32), 64, 2
    pos = np.arange(3, dtype=f32)
    inv = (1.0 / (1e7 ** (np.arange(0, Rr, 2, dtype=f32) / f32(Rr)))).astype(f32)
    fr = (pos[:, None] * inv[None, :]).astype(f32)
    tab = np.concatenate([np.cos(fr), np.sin(fr)], 1).astype(f32)
    tx = torch.from_numpy(x)
    cos = torch.from_numpy(np.repeat(np.cos(fr), G, 0))
    sin = torch.from_numpy(np.repeat(np.sin(fr), G, 0))
    cos, sin = torch.cat([cos, cos], -1), torch.cat([sin, sin], -1)
    xr = tx[:, :Rr]
    rot = torch.cat([-xr[:, Rr // 2:], xr[:, :Rr // 2]], -1)
    ref = torch.cat([xr * cos + rot * sin, tx[:, Rr:]], -1).numpy()
    assert same(R.rope_rows(x, tab, G, Rr), F.ftz(ref))


@pytest.mark.parametrize("op", [R.ELT_MUL, R.ELT_ADD, R.ELT_SUB, R.ELT_MULADD])
@pytest.mark.parametrize("mode", [R.BM_DENSE, R.BM_ROW, R.BM_COL, R.BM_SCALAR])
def test_elt_modes_compose_single_steps(op, mode):
    """tests/test_v04.py:99-121: act(A) op B with B broadcast per mode, each step one fmul/fadd."""
    rng = np.random.default_rng(op * 4 + mode)
    M, N = 5, 32
    a = rng.normal(0, 1, (M, N)).astype(f32)
    bv = rng.normal(0, 1, {R.BM_DENSE: M * N, R.BM_ROW: N, R.BM_COL: M, R.BM_SCALAR: 1}[mode]).astype(f32)
    c = rng.normal(0, 1, (M, N)).astype(f32)
    B = R.broadcast_b(bv, mode, M, N)
    full = {R.BM_DENSE: lambda: bv.reshape(M, N), R.BM_ROW: lambda: np.tile(bv, (M, 1)),
            R.BM_COL: lambda: np.repeat(bv[:, None], N, 1), R.BM_SCALAR: lambda: np.full((M, N), bv[0], f32)}[mode]()
    assert same(B, full)
    A = F.sigmoid_f(a)
    want = {R.ELT_MUL: lambda: F.fmul(A, full), R.ELT_ADD: lambda: F.fadd(A, full),
            R.ELT_SUB: lambda: F.fadd(A, F.neg(full)), R.ELT_MULADD: lambda: F.fadd(c, F.fmul(A, full))}[op]()
    assert same(R.elt(op, a, B, c, act=F.ACT_SIGMOID), want)
