"""CPU proofs for the shortcuts the device code takes inside the contract's fixed sequences.

The HIP kernels drop the flush/canonicalize wrappers where they cannot change a bit. Each claim is
checked here with numpy's float32 (the same IEEE round-to-nearest-even operations the GPU runs),
exhaustively where the input space allows."""
from __future__ import annotations

import numpy as np

from oracle import numerics as F

f32 = np.float32


def test_recip_newton_steps_stay_normal_and_match_the_wrapped_steps():
    """recip_f's Newton loop depends only on the mantissa: for all 2^23 of them, the raw
    operations never produce a subnormal, infinity or NaN and give the wrapped loop's bits."""
    mbits = (np.arange(1 << 23, dtype=np.uint32) | np.uint32(127 << 23))
    m = mbits.view(f32)
    y_raw = (np.uint32(F.RECIP_SEED) - mbits).view(f32)
    y_ref = y_raw.copy()
    tiny = f32(2.0 ** -126)
    for _ in range(3):
        p = m * y_raw
        e = f32(1.0) - p
        t = y_raw * e
        for v in (p, e, t):
            assert np.isfinite(v).all()
            assert ((v == 0) | (np.abs(v) >= tiny)).all()
        y_raw = y_raw + t
        assert (y_raw > f32(0.04)).all() and np.isfinite(y_raw).all()
        y_ref = F.fadd(y_ref, F.fmul(y_ref, F.fadd(F.ONE, F.neg(F.fmul(m, y_ref)))))
    assert (y_raw.view(np.uint32) == y_ref.view(np.uint32)).all()


def test_rsqrt_newton_steps_stay_normal_and_match_the_wrapped_steps():
    """rsqrt_f's Newton loop depends only on m in [1, 4) (exponent field 127 or 128): for all 2^24
    of them, the raw operations never produce a subnormal, infinity or NaN and give the wrapped
    loop's bits."""
    from oracle import rowops as R
    mbits = np.concatenate([np.arange(1 << 23, dtype=np.uint32) | np.uint32(e << 23) for e in (127, 128)])
    m = mbits.view(f32)
    y_raw = (np.uint32(R.RSQRT_SEED) - (mbits >> np.uint32(1))).view(f32)
    y_ref = y_raw.copy()
    tiny, half = f32(2.0 ** -126), f32(0.5)
    for _ in range(3):
        p = m * y_raw
        t = p * y_raw
        h = half * t
        d = half - h
        u = y_raw * d
        for v in (p, t, h, d, u):
            assert np.isfinite(v).all()
            assert ((v == 0) | (np.abs(v) >= tiny)).all()
        y_raw = y_raw + u
        assert (y_raw > f32(0.4)).all() and (y_raw < f32(1.1)).all()
        y_ref = F.fadd(y_ref, F.fmul(y_ref, F.fadd(half, F.neg(F.fmul(half, F.fmul(F.fmul(m, y_ref), y_ref))))))
    assert (y_raw.view(np.uint32) == y_ref.view(np.uint32)).all()


def test_q8_with_flushed_multiplier():
    """q8(x, inv) == clamp(rint(nan->0(ftz(x) * inv))) whenever inv is an fmul output (flushed,
    canonical): random bit patterns for x, and multipliers covering 0, inf, NaN and the range."""
    rng = np.random.default_rng(0)
    xb = rng.integers(0, 1 << 32, 400000, dtype=np.uint64).astype(np.uint32)
    x = xb.view(f32)
    invs = np.concatenate([np.array([0.0, np.inf, 1.0, 127.0, 1e-30, 1e30], f32),
                           (rng.integers(1, 255, 60, dtype=np.uint32) << 23 |
                            rng.integers(0, 1 << 23, 60, dtype=np.uint32)).view(f32),
                           np.array([0x7FC00000], np.uint32).view(f32)])
    for inv in invs:
        inv = F.fmul(np.array([inv], f32), F.ONE)[0]          # an fmul output
        with np.errstate(all="ignore"):
            y = F.ftz(x) * inv
            y = np.where(np.isnan(y), f32(0), np.rint(y))
            lean = np.clip(y, -127, 127).astype(np.int8)
        assert (lean == F.q8(x, inv)).all(), inv


def test_rne_shift_by_add_equals_the_reference_rounding():
    """The aligner's round-to-nearest-even right shift of a 24-bit significand, written as
    (sig + 2^(sh-1) - 1 + ((sig >> sh) & 1)) >> sh, equals the reference's kept/dropped/half rule
    (numerics.py:80-89) for every significand and every shift 10..31 (exhaustive)."""
    sig = (np.arange(1 << 23, dtype=np.int64) | (1 << 23))
    for sh in range(10, 32):
        kept = sig >> sh
        dropped = sig & ((1 << sh) - 1)
        half = 1 << (sh - 1)
        ref = kept + ((dropped > half) | ((dropped == half) & ((kept & 1) == 1)))
        fast = (sig + (half - 1) + ((sig >> sh) & 1)) >> sh
        assert (ref == fast).all(), sh
        assert fast.max() <= (1 << 14) or sh < 10  # mantissas stay within 16384 for sh >= 10


def test_magic_number_rounding_gives_the_int16_mantissa():
    """RN(v + 1.5 * 2^23) for every v = k / 2^j with |v| < 2^14 (k an integer, the exact products
    x * 2^(140 - e_eff) the aligner rounds) has the low 16 bits of rint(v) (ties to even), two's
    complement: checked over every multiple of 1/8 in range (the ties x.5 among them), and on the
    values just above and below each tie."""
    k = np.arange(-(1 << 17), 1 << 17, dtype=np.int64)
    v8 = k.astype(f32) / f32(8)
    ties = np.arange(-(1 << 14), 1 << 14).astype(f32) + f32(0.5)
    for v in (v8, np.nextafter(ties, f32(np.inf)), np.nextafter(ties, f32(-np.inf))):
        v = v[np.abs(v) < 2 ** 14]
        got = (v + f32(12582912.0)).view(np.uint32) & 0xFFFF
        assert (got == (np.rint(v).astype(np.int64) & 0xFFFF)).all()


def test_rne_shift_equals_a_power_of_two_product_rounded_to_even():
    """The aligner's finite-group fast path computes a mantissa as rint(x * 2^(140 - e_eff)) in
    fp32 (one exact power-of-two product, then round-half-even): for a 24-bit significand sig of
    exponent e that is rint(sig * 2^-sh) with sh = 10 + e_eff - e, which equals the reference's
    kept/dropped/half shift for every significand and every shift 10..40 (exhaustive)."""
    sig = (np.arange(1 << 23, dtype=np.int64) | (1 << 23))
    sigf = sig.astype(f32)                                   # exact: sig < 2^24
    for sh in range(10, 41):
        s = min(sh, 31)
        kept = sig >> s
        dropped = sig & ((1 << s) - 1)
        half = 1 << (s - 1)
        ref = np.where(sh >= 25, 0, kept + ((dropped > half) | ((dropped == half) & ((kept & 1) == 1))))
        fast = np.rint(sigf * f32(2.0 ** -sh)).astype(np.int64)
        assert (ref == fast).all(), sh


def test_aligner_fast_path_matches_the_oracle_on_finite_groups():
    """The same formula on real activation rows against the oracle's aligner (numerics.py:55-98):
    groups mixing exponent spreads of 0..250, zeros, signed values, subnormal inputs (flushed),
    products that fall into the subnormal range, exact ties, and the e_eff = 14 floor."""
    rng = np.random.default_rng(3)
    rows = []
    for spread in (0, 3, 12, 24, 25, 40, 120, 250):
        for _ in range(20):
            e = rng.integers(max(1, 200 - spread), 201, 128) if spread < 200 else rng.integers(1, 255, 128)
            b = (rng.integers(0, 2, 128) << 31) | (e.astype(np.int64) << 23) | rng.integers(0, 1 << 23, 128)
            v = b.astype(np.uint32).view(f32).copy()
            v[rng.integers(0, 128, 5)] = 0.0
            v[rng.integers(0, 128, 3)] = np.uint32(rng.integers(1, 1 << 23)).view(f32)   # subnormal input
            rows.append(v)
    small = (rng.integers(0, 1 << 23, (40, 128)) | (rng.integers(1, 20, (40, 128)) << 23)).astype(np.uint32)
    rows.extend(small.view(f32))                                                       # e_eff = 14 floor
    ties = (np.float32(2.0) ** rng.integers(-20, 20, (20, 1))) * (rng.integers(0, 64, (20, 128)) + f32(0.5))
    rows.extend(ties.astype(f32))
    x = np.stack(rows)
    q, scales = F.align_w4_groups(x)
    for flushed in (True, False):
        xf = (F.ftz(x) if flushed else x).reshape(x.shape[0], -1, 128)
        e = (xf.view(np.uint32) >> 23) & 0xFF
        emax = e.max(axis=2)
        e_eff = np.maximum(emax, 14)
        p = ((267 - e_eff).astype(np.uint32) << 23).view(f32)[:, :, None]              # 2^(140 - e_eff)
        with np.errstate(under="ignore"):
            fast = np.rint(xf * p).astype(np.int64)
            # the kernel's form: one fma (x * p is exact), the low 16 bits of RN(x * p + 1.5 * 2^23)
            fma16 = ((xf * p + f32(12582912.0)).view(np.uint32) & 0xFFFF).astype(np.int64)
        want = q.astype(np.int64).reshape(fast.shape)
        # flushed inputs: every finite group; unflushed inputs (the kernel's fast path): groups with
        # emax >= 16, where a subnormal input times 2^(140 - e_eff) <= 2^124 stays below 1/4
        sel = np.ones_like(emax, bool) if flushed else emax >= 16
        assert sel.sum() > 100
        assert (fast[sel] == want[sel]).all()
        assert (fma16[sel] == (want[sel] & 0xFFFF)).all()


def test_q8_fast_path_for_rows_with_a_normal_maximum():
    """A quantizer row whose maximum amax = max |ftz(x)| is finite and at least 2^-118 skips q8's
    input flush and NaN test: with inv = fmul(127, recip_f(amax)), q8(x, inv) equals
    clamp(rint(x * inv), -127, 127) on the unflushed x. Such a row holds no NaN or infinity, a normal
    x is its own flush, and a subnormal x (|x| < 2^-126) gives |x * inv| < 2^-126 * 127 * 2^118 *
    (1 + 2^-22) < 1/2, which rounds to the 0 its flush gives. Exhaustive over every subnormal at the
    smallest maxima; random rows (extremes, exact ties, tiny normals) across the whole range."""
    rng = np.random.default_rng(7)
    edge = np.array([0x04800000, 0x04800001, 0x04800007, 0x04FFFFFF, 0x05000000], np.uint32).view(f32)
    sub = np.arange(1, 1 << 23, dtype=np.uint32)
    sub = np.concatenate([sub, sub | np.uint32(0x80000000)]).view(f32)       # every nonzero subnormal
    for amax in edge:
        inv = F.fmul(F.Q127, F.recip_f(np.array([amax], f32)))[0]
        with np.errstate(all="ignore"):
            fast = np.clip(np.rint(sub * inv), -127, 127)
        assert (fast == 0).all(), amax
        assert (F.q8(sub, inv) == 0).all()
    # random maxima over every exponent from 2^-118 to the largest finite value
    mb = np.concatenate([(rng.integers(9, 255, 400, dtype=np.uint32) << 23) | rng.integers(0, 1 << 23, 400, dtype=np.uint32),
                         np.array([0x04800000, 0x7F7FFFFF, 0x3F800000, 0x42FE0000], np.uint32)])
    for amax in mb.view(f32):
        inv = F.fmul(F.Q127, F.recip_f(np.array([amax], f32)))[0]
        u = rng.uniform(-1, 1, 4000).astype(f32)
        with np.errstate(divide="ignore"):           # inv is 0 for the largest maxima (q8 is then 0)
            ties = ((rng.integers(-127, 127, 200) + f32(0.5)) / inv).astype(f32)
        x = np.concatenate([
            (u * amax).astype(f32),                                          # inside [-amax, amax]
            np.array([amax, -amax, 0.0, -0.0], f32),
            ties,                                                             # near the q8 ties
            sub[rng.integers(0, sub.size, 200)],                              # subnormal inputs
            (np.uint32(0x00800000) + rng.integers(0, 1 << 20, 100, dtype=np.uint32)).view(f32),  # tiny normals
        ])
        x = x[np.abs(F.ftz(x)) <= amax]
        with np.errstate(all="ignore"):
            fast = np.clip(np.rint(x * inv), -127, 127).astype(np.int8)
            byte = rounding_constant_byte(x * inv)        # the kernels' form: no clamp
        assert (fast == F.q8(x, inv)).all(), amax
        assert (byte == F.q8(x, inv)).all(), amax


ROUND_C = f32(1.5 * 2.0 ** 23)


def rounding_constant_byte(t):
    """The fast q8 byte as the kernels form it: the low byte of the encoding of t + 1.5 * 2^23."""
    return ((t.astype(f32) + ROUND_C).view(np.uint32) & np.uint32(0xFF)).astype(np.uint8).view(np.int8)


def test_q8_fast_rows_need_no_clamp():
    """On a row for which the fast path holds, |x * inv| <= amax * inv < 127.5, so clamping
    rint(x * inv) to [-127, 127] never changes it. amax * inv depends only on amax's mantissa m
    (recip_f and the product by 127 scale exactly with a power of two while the results stay normal;
    a flushed subnormal result makes inv 0): exhaustive over all 2^23 mantissas, plus random maxima
    over every fast-path exponent, including those where inv underflows to 0."""
    m = (np.arange(1 << 23, dtype=np.uint32) | np.uint32(127 << 23)).view(f32)
    p = m * F.fmul(F.Q127, F.recip_f(m))
    assert p.max() < f32(127.0001) and p.min() > f32(-127.5)
    rng = np.random.default_rng(11)
    mb = (rng.integers(9, 255, 20000, dtype=np.uint32) << 23) | rng.integers(0, 1 << 23, 20000, dtype=np.uint32)
    amax = np.concatenate([mb, np.array([0x04800000, 0x7F7FFFFF, 0x7F000000, 0x7E800000], np.uint32)]).view(f32)
    inv = F.fmul(F.Q127, F.recip_f(amax))
    with np.errstate(over="ignore"):
        assert (amax * inv < f32(127.5)).all()
    assert (inv == 0).any()                                  # maxima near 2^128 give inv = 0


def test_rounding_constant_gives_the_q8_byte():
    """rint(t) mod 256 as the low byte of RN(t + 1.5 * 2^23): exhaustive over every fp32 t with
    0.5 <= |t| < 128 (the sum lies in [2^23, 2^24), where the spacing is 1 and ties go to even, as
    rint's do), and every |t| < 0.5 gives 0 (random values, every subnormal, +-0)."""
    for e in range(-1, 7):
        t = ((np.uint32(e + 127) << np.uint32(23)) | np.arange(1 << 23, dtype=np.uint32)).view(f32)
        for v in (t, -t):
            want = np.rint(v).astype(np.int64).astype(np.int8)
            assert (rounding_constant_byte(v) == want).all(), e
    rng = np.random.default_rng(5)
    small = np.concatenate([rng.uniform(-0.5, 0.5, 1 << 20).astype(f32),
                            np.arange(1, 1 << 23, 97, dtype=np.uint32).view(f32),
                            np.array([0.0, -0.0, 0.49999997, -0.49999997, 0.5, -0.5], f32)])
    small = small[np.abs(small) <= 0.5]
    assert (rounding_constant_byte(small) == 0).all()


def test_partial_sums_above_2_pow_minus_100_absorb_subnormal_addends():
    """The attention chains skip their products' flushes when every partial sum avoids (0, 2^-100):
    RN(acc + s) == acc for every |acc| >= 2^-100 and every subnormal s (random accumulators over
    every exponent from -100 up, the smallest and largest mantissas at 2^-100, and subnormals at
    both ends of the range and at random), while just below 2^-100 some do not."""
    rng = np.random.default_rng(11)
    sub = np.concatenate([np.array([1, 2, 0x7FFFFF, 0x7FFFFE, 0x400000], np.uint32),
                          rng.integers(1, 1 << 23, 2000, dtype=np.uint32)])
    sub = np.concatenate([sub, sub | np.uint32(0x80000000)]).view(f32)
    accs = np.concatenate([np.array([0x0D800000, 0x0D800001, 0x0DFFFFFF, 0x7F7FFFFF], np.uint32),
                           (rng.integers(27, 255, 3000, dtype=np.uint32) << 23) | rng.integers(0, 1 << 23, 3000, dtype=np.uint32)])
    accs = np.concatenate([accs, accs | np.uint32(0x80000000)]).view(f32)
    assert (np.abs(accs) >= f32(2.0 ** -100)).all()
    for a in accs:
        assert (np.float32(a) + sub == a).all(), a
    below = np.float32(2.0 ** -100) * np.float32(1 - 2.0 ** -24)          # just below 2^-100
    with np.errstate(all="ignore"):
        assert ((np.float32(2.0 ** -110) + sub) != np.float32(2.0 ** -110)).any()
    assert below < np.float32(2.0 ** -100)
    key = lambda x: ((np.asarray(x, f32).view(np.uint32).astype(np.uint64) << 1) + 0xFFFFFFFF) & 0xFFFFFFFF  # (bits << 1) - 1 mod 2^32
    tiny = ((27 << 23) << 1) - 1
    assert key(np.float32(2.0 ** -100)) == tiny and key(below) < tiny and key(np.float32(0)) > tiny
    assert (key(sub) < tiny).all()


def test_plus_zero_steps_leave_unflushed_chains_but_not_flushed_ones():
    """The W4A16 GEMV runs its unflushed bank chains over every register step, the steps past a
    row's last group adding +0, and recomputes a chain with the contract's flushing adds (stopping
    at the last group) when a partial sum is subnormal. Unflushed, a sum that starts at +0 is never
    -0 under round-to-nearest (only -0 + -0 gives -0), so a +0 step changes no bit of it (chains
    of signed zeros, subnormals, normals near the subnormal range, cancelling pairs, infinities);
    flushed, a chain can end at -0 (a negative subnormal partial sum flushed), where a +0 step
    would give +0."""
    rng = np.random.default_rng(23)
    pool = np.array([0.0, -0.0, 2.0 ** -149, -2.0 ** -149, 2.0 ** -126, -2.0 ** -126, 1.5, -1.5,
                     np.inf, -np.inf], f32)
    for _ in range(3000):
        n = int(rng.integers(1, 10))
        t = np.where(rng.random(n) < 0.4, rng.choice(pool, n),
                     (rng.normal(0, 1, n) * np.exp2(rng.integers(-140, -110, n))).astype(f32)).astype(f32)
        for i in range(1, n):
            if rng.random() < 0.3:
                t[i] = -t[i - 1]                                    # exact cancellation
        acc = f32(0.0)
        with np.errstate(all="ignore"):
            for v in t:
                acc = f32(acc + v)
                assert not (acc == 0 and np.signbit(acc))
            padded = f32(acc + f32(0.0))
        assert np.isnan(acc) or padded.view(np.uint32) == acc.view(np.uint32)
    a = f32(2.0 ** -125)
    ends = F.fadd(F.fadd(f32(0.0), a), -f32(a + f32(3 * 2.0 ** -148)))   # a - (a + 3 2^-148), flushed
    assert ends == 0 and np.signbit(ends)
    assert not np.signbit(F.fadd(ends, f32(0.0)))


def test_balanced_hex_digit_planes_reconstruct_every_mantissa():
    """The W4A16 GEMV writes each aligned mantissa a (|a| <= 2^14) as four balanced base-16 digits
    and dots each digit plane with the weight nibbles on v_dot8_i32_i4 (signed 4-bit operands).
    For every a in [-16384, 16384]: nibble i = floor((a + c_i) / 16^i) mod 16 with c = (0, 8, 136,
    2184), read back as a signed 4-bit value d_i, satisfies sum 16^i d_i == a; so for any signed
    4-bit weights w the planes' dots combine to the exact dot, sum_i 16^i sum_e w_e d_ie ==
    sum_e w_e a_e (checked on random 8-element dwords too, with the kernel's packing order)."""
    a = np.arange(-16384, 16385, dtype=np.int64)
    c = (0, 8, 136, 2184)
    nib = [((a + c[i]) >> (4 * i)) & 15 for i in range(4)]
    d = [np.where(n >= 8, n - 16, n) for n in nib]                       # sign-extended 4-bit
    assert all(((di >= -8) & (di <= 7)).all() for di in d)
    assert (d[0] + 16 * d[1] + 256 * d[2] + 4096 * d[3] == a).all()
    assert (np.abs(d[3]) <= 4).all()

    def sext4(v):
        return np.where(v >= 8, v - 16, v)

    def dot8(wd, xd):
        """v_dot8_i32_i4: the sum over the 8 nibble positions of the signed nibble products."""
        s = np.zeros(wd.shape, np.int64)
        for e in range(8):
            s += sext4((wd >> (4 * e)) & 15) * sext4((xd >> (4 * e)) & 15)
        return s

    rng = np.random.default_rng(3)
    w = rng.integers(-8, 8, (4000, 8))
    x = rng.integers(-16384, 16385, (4000, 8))
    x[:8] = [[-16384] * 8, [16384] * 8, [16383] * 8, [-16383] * 8, [8] * 8, [-8] * 8, [7] * 8, [-9] * 8]
    wd = sum((w[:, e] & 15) << (4 * e) for e in range(8))              # low nibble of byte b = k 2b
    total = np.zeros(4000, np.int64)
    for i in range(4):
        xd = sum((((x[:, e] + c[i]) >> (4 * i)) & 15) << (4 * e) for e in range(8))
        total += dot8(wd, xd) << (4 * i)
    assert (total == (w * x).sum(axis=1)).all()
