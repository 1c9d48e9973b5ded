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
