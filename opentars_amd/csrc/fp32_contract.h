// Device-side fp32 steps of the golden model's numeric contract (tars_mini/numerics.py).
//
// Every step rounds once to nearest-even with fp32 subnormals handled in hardware (the kernels'
// fp32 denorm mode is "preserve"), then flushes a subnormal input or result to a zero of the same
// sign with a bit test, and replaces any NaN with 0x7FC00000. That is exactly numpy's float32
// multiply/add followed by the reference's ftz()/canon(). The library is compiled with
// -ffp-contract=off, so no multiply and add pair is ever fused.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tars {

constexpr uint32_t kSign = 0x80000000u;
constexpr uint32_t kExpo = 0x7F800000u;
constexpr uint32_t kMant = 0x007FFFFFu;
constexpr uint32_t kCanonNaN = 0x7FC00000u;

__device__ __forceinline__ uint32_t fbits(float x) { return __float_as_uint(x); }
__device__ __forceinline__ float ffrom(uint32_t b) { return __uint_as_float(b); }

__device__ __forceinline__ bool is_nan(float x) { return (fbits(x) & 0x7FFFFFFFu) > kExpo; }

// numerics.py:26-31. The class test (+-subnormal) and a select: three instructions where the
// exponent-field test took five, which shortens every dependent chain of contract steps (a chain of
// multiply-adds through these wrappers measured 43 instead of 75 cycles per step on MI355X).
__device__ __forceinline__ float ftz(float x) {
  return __builtin_amdgcn_classf(x, 0x90) ? ffrom(fbits(x) & kSign) : x;
}

// numerics.py:34-37 (the class test for signalling and quiet NaN)
__device__ __forceinline__ float canon(float x) { return __builtin_amdgcn_classf(x, 0x3) ? ffrom(kCanonNaN) : x; }

// numerics.py:40-47: one rounded operation, FTZ in and out, canonical NaN
__device__ __forceinline__ float fmul(float a, float b) { return canon(ftz(__fmul_rn(ftz(a), ftz(b)))); }
__device__ __forceinline__ float fadd(float a, float b) { return canon(ftz(__fadd_rn(ftz(a), ftz(b)))); }

// One step of a summation chain over flushed values: the contract's fadd without its input
// flushes (identities here) and without the per-step NaN canonicalization. NaN is absorbing in a
// sum (NaN + x is NaN for every x), so a chain's result is NaN exactly when the contract's
// step-by-step chain's is, and every other step is the same rounded, flushed value; the chain's
// result is canonicalized once at its end (chain_end). The flush tests the value class (+-
// subnormal) in one compare.
__device__ __forceinline__ float fadd_chain(float acc, float p) {
  const float r = __fadd_rn(acc, p);
  return __builtin_amdgcn_classf(r, 0x90) ? ffrom(fbits(r) & kSign) : r;
}
__device__ __forceinline__ float chain_end(float acc) { return canon(acc); }

// A chain run with plain rounded operations (no flushes) equals the contract's chain, up to NaN
// payloads that chain_end canonicalizes, whenever none of its inputs, products and partial sums is
// subnormal: every flush is then an identity. Such a chain keeps the minimum of sub_key over those
// values, off its dependent path in vector registers, and is recomputed with the flushes when the
// minimum is below kSubKeyNormal. sub_key(x) = (bits << 1) - 1 as unsigned drops the sign: +-0 wraps
// to the largest key, a subnormal maps to [0, 2^24 - 2], every normal, infinite or NaN x to at
// least 2^24 - 1 (one shift-add per value, one three-way minimum per two values).
constexpr uint32_t kSubKeyNormal = 0x00FFFFFFu;
__device__ __forceinline__ uint32_t sub_key(float x) { return (fbits(x) << 1) - 1u; }
// A partial sum of magnitude at least 2^-100 absorbs any subnormal addend s: |s| < 2^-126 is below
// half an ulp of it (>= 2^-124), so RN(acc + s) = acc, which is what acc + ftz(s) = acc + 0 gives.
// A chain whose starting value and unflushed partial sums all avoid (0, 2^-100) in magnitude
// therefore matches the contract without testing its products: a subnormal product added to a
// zero shows up as a subnormal partial sum. kSubKeyTiny = sub_key(2^-100); a minimum below it
// (including any subnormal, whose key is smaller still) sends the chain to the flushing recompute.
constexpr uint32_t kSubKeyTiny = ((27u << 23) << 1) - 1u;
__device__ __forceinline__ uint32_t min_key(uint32_t m, float a, float b) {
  return min(m, min(sub_key(a), sub_key(b)));
}
// The same test kept as the minimum magnitude (fminf: NaN ignored, one three-way minimum with
// absolute-value operands per two values): a chain is recomputed when it falls below kTiny. An
// exact zero also sends it there (the same bits, more time), so this form suits chains whose
// partial sums are rarely exactly zero.
constexpr float kTiny = 0x1p-100f;
__device__ __forceinline__ float min_mag(float m, float a, float b) {
  float r;  // one v_min3_f32 with |a| and |b| (fminf would add canonicalizing maxima around it)
  __asm__("v_min3_f32 %0, %1, |%2|, |%3|" : "=v"(r) : "v"(m), "v"(a), "v"(b));
  return r;
}

// numerics.py:50-52: int32 -> fp32 round-to-nearest-even (v_cvt_f32_i32)
__device__ __forceinline__ float i2f(int32_t i) { return static_cast<float>(i); }

// numerics.py:111-113, 265-267
__device__ __forceinline__ float fneg(float x) { return ffrom(fbits(x) ^ kSign); }
__device__ __forceinline__ float fabs_c(float x) { return ffrom(fbits(ftz(x)) & 0x7FFFFFFFu); }

// The constants of the reference's fixed sequences, by encoding (numerics.py:116-123, 234-238).
constexpr uint32_t kOne = 0x3F800000u, kTwo = 0x40000000u, kHalf = 0x3F000000u;
constexpr uint32_t kLog2e = 0x3FB8AA3Bu, kNegLn2Hi = 0xBF317200u, kNegLn2Lo = 0xB5BFBE8Eu;
constexpr uint32_t kExpHi = 0x42B20000u /* 89 */, kExpLo = 0xC2D00000u /* -104 */;
constexpr uint32_t kRecipSeed = 0x7EF311C7u;
constexpr uint32_t kGeluA = 0x3D372713u, kGeluC = 0x3F4C422Au;
constexpr uint32_t kSoftplusHi = 0x41A00000u /* 20 */;
constexpr uint32_t kQ127 = 0x42FE0000u, kInv127 = 0x3C010204u;

// Positive normal y with e added to its biased exponent: >= 255 -> +inf, <= 0 -> +0; the sign bit
// is not carried (numerics.py:126-132).
__device__ __forceinline__ float add_to_exponent(float y, int e) {
  const uint32_t yb = fbits(y);
  const int field = static_cast<int>((yb >> 23) & 0xFFu) + e;
  const uint32_t r = (static_cast<uint32_t>(field) << 23) | (yb & kMant);
  return ffrom(field >= 255 ? kExpo : field <= 0 ? 0u : r);
}

// 1/x: seed from the magic constant, three correction-form Newton steps, exponent surgery
// (numerics.py:153-168).
//
// Inside the Newton steps the contract's flush/canonicalize wrappers are identities, so the raw
// round-to-nearest-even operations give the same bits with a much shorter dependent chain:
// m is in [1, 2) and the seed bits^-1(0x7EF311C7 - bits(m)) is in [0.47, 0.96], so every
// m * y is a positive normal in [0.47, 1.9]; e = 1 - m * y is exactly 0 or a multiple of 2^-25
// (both operands are), hence 0 or normal; y * e is 0 or at least 2^-26 in magnitude; and
// y + y * e = y * (2 - m * y) stays positive and above 0.04. No subnormal, infinity or NaN can
// arise, and each step is still one rounded operation (never fused: -ffp-contract=off).
__device__ __forceinline__ float recip_f(float x) {
  const uint32_t xb = fbits(ftz(x));
  const uint32_t sgn = xb & kSign, mag = xb & 0x7FFFFFFFu;
  const uint32_t mb = (mag & kMant) | (127u << 23);
  const float m = ffrom(mb);
  float y = ffrom(kRecipSeed - mb);
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const float err = __fadd_rn(1.0f, -__fmul_rn(m, y));
    y = __fadd_rn(y, __fmul_rn(y, err));
  }
  const uint32_t r = fbits(add_to_exponent(y, 127 - static_cast<int>(mag >> 23))) | sgn;
  // the special inputs by selects, so the common path runs straight through (no branches)
  const uint32_t special = mag > kExpo ? kCanonNaN : mag == 0 ? (sgn | kExpo) : sgn;
  return ffrom(mag == 0 || mag >= kExpo ? special : r);
}

// e^x (numerics.py:135-150).
//
// After the input flush and the NaN test the contract's flush/canonicalize wrappers change no
// step, so the raw round-to-nearest-even operations give the same bits with a much shorter
// dependent chain. For finite x (zero or normal): x * log2e is 0 or normal (log2e > 1); n is an
// integer in [-200, 200]; n * -ln2_hi is 0 or at least 0.69 in magnitude, and exact (ln2_hi has
// 14 fraction bits); n * -ln2_lo is +-0 or at least 1.4e-6 in magnitude. With n = 0, r = x. Else
// x + n * -ln2_hi is a multiple of 2^-25 (|x| >= 0.34 then, and n * ln2_hi a multiple of 2^-14),
// so 0 or normal, and adding n * -ln2_lo (a multiple of 2^-43 below 2^-11 in magnitude) leaves 0
// or a normal value. For -104 < x < 89 (n unclamped, |r| <= 0.35) every partial value of the
// polynomial lies in [0.0078, 1.5], and a product p * r is normal except when n = 0 and
// |x| < 2^-116, where it may be subnormal: the contract flushes it to 0 and adds a coefficient of
// at least 1/120, whose half ulp (>= 2^-31) the unflushed product cannot reach, so both sums round
// to that coefficient. Other x take their result from the range tests; on the way their steps
// stay free of NaN (r and the coefficients are finite unless x is infinite, and then no product
// pairs an infinity with a zero and no sum pairs opposite infinities). No NaN arises, so the result
// needs no canonicalization. A NaN x runs the same steps (their values are dropped) and returns the
// canonical NaN.
__device__ __forceinline__ float exp_f(float x) {
  x = ftz(x);
  const bool nan = is_nan(x);  // taken by a select at the end: the steps below run branch-free
  float n = rintf(__fmul_rn(x, ffrom(kLog2e)));
  n = fminf(fmaxf(n, -200.0f), 200.0f);
  const float r = __fadd_rn(__fadd_rn(x, __fmul_rn(n, ffrom(kNegLn2Hi))), __fmul_rn(n, ffrom(kNegLn2Lo)));
  const uint32_t coeffs[6] = {0x3C088889u, 0x3D2AAAABu, 0x3E2AAAABu, 0x3F000000u, 0x3F800000u,
                              0x3F800000u};
  float p = ffrom(0x3AB60B61u);
#pragma unroll
  for (int i = 0; i < 6; ++i) p = __fadd_rn(__fmul_rn(p, r), ffrom(coeffs[i]));
  const float y = add_to_exponent(p, static_cast<int>(n));
  return nan ? ffrom(kCanonNaN) : x >= ffrom(kExpHi) ? ffrom(kExpo) : x <= ffrom(kExpLo) ? 0.0f : y;
}

__device__ __forceinline__ float relu_plain(float x) { return x > 0.0f ? x : 0.0f; }

// numerics.py:241-244
__device__ __forceinline__ float sigmoid_f(float x) {
  x = ftz(x);
  return recip_f(fadd(ffrom(kOne), exp_f(fneg(x))));
}

// numerics.py:204-207
__device__ __forceinline__ float silu_f(float x) {
  x = ftz(x);
  return fmul(x, recip_f(fadd(ffrom(kOne), exp_f(fneg(x)))));
}

// numerics.py:194-201
__device__ __forceinline__ float gelu_f(float x) {
  x = ftz(x);
  const float cube = fmul(fmul(x, x), x);
  const float u = fmul(ffrom(kGeluC), fadd(x, fmul(ffrom(kGeluA), cube)));
  const float t = fadd(ffrom(kOne), fneg(fmul(ffrom(kTwo), recip_f(fadd(exp_f(fmul(ffrom(kTwo), u)), ffrom(kOne))))));
  return fmul(fmul(ffrom(kHalf), x), fadd(ffrom(kOne), t));
}

// numerics.py:247-262
__device__ __forceinline__ float softplus_f(float x) {
  x = ftz(x);
  if (is_nan(x)) return ffrom(kCanonNaN);
  const float t = exp_f(fneg(fabs_c(x)));
  const float s = fmul(t, recip_f(fadd(t, ffrom(kTwo))));
  const float z = fmul(s, s);
  const uint32_t coeffs[8] = {0x3D888889u, 0x3D9D89D9u, 0x3DBA2E8Cu, 0x3DE38E39u,
                              0x3E124925u, 0x3E4CCCCDu, 0x3EAAAAABu, 0x3F800000u};
  float p = ffrom(0x3D70F0F1u);
#pragma unroll
  for (int i = 0; i < 8; ++i) p = fadd(fmul(p, z), ffrom(coeffs[i]));
  const float y = fadd(relu_plain(x), fmul(fmul(ffrom(kTwo), s), p));
  return canon(x > ffrom(kSoftplusHi) ? x : y);
}

// The epilogue activation by code (numerics.py:210-230).
__device__ __forceinline__ float act_fn(float x, int act) {
  x = ftz(x);
  switch (act) {
    case 0: return x;
    case 1: return relu_plain(x);
    case 2: { const float r = relu_plain(x); return r > 6.0f ? 6.0f : r; }
    case 3: return gelu_f(x);
    case 4: return silu_f(x);
    case 5: return sigmoid_f(x);
    case 6: return softplus_f(x);
    default: return exp_f(x);
  }
}

// numerics.py:282-286: rint(fmul(x, inv)) ties-to-even, NaN -> 0, clamp to [-127, 127]
__device__ __forceinline__ int8_t q8(float x, float inv) {
  float y = fmul(x, inv);
  if (is_nan(y)) y = 0.0f;
  y = rintf(y);
  y = fminf(fmaxf(y, -127.0f), 127.0f);
  return static_cast<int8_t>(static_cast<int>(y));
}

// q8 with an already flushed multiplier (inv from fmul). The product's output flush only turns a
// subnormal into a zero, whose rint is the same integer 0, and canonicalization only rewrites NaN
// payloads, which map to 0 anyway; so only the input flush of x remains.
__device__ __forceinline__ int q8_flushed_inv(float x, float inv) {
  float y = __fmul_rn(ftz(x), inv);
  y = is_nan(y) ? 0.0f : rintf(y);
  return static_cast<int>(fminf(fmaxf(y, -127.0f), 127.0f));
}

// q8 for a row whose maximum amax = max |ftz(x)| is finite and at least 2^-118 (every row but
// all-tiny, all-zero, infinity and NaN rows): the row holds no NaN or infinity, a normal x is its
// own flush, and a subnormal x gives |x * inv| < 2^-126 * 127 * 2^118 * (1 + 2^-22) < 1/2, which
// rounds to the 0 its flush gives; so q8 is rint(x * inv) clamped, with no flush or NaN test
// (checked on the CPU: every subnormal at the smallest maxima, random rows across the range).
constexpr uint32_t kQ8FastMin = 0x04800000u;  // 2^-118
__device__ __forceinline__ bool q8_fast_row(uint32_t amax_bits) {
  return amax_bits >= kQ8FastMin && amax_bits < kExpo;
}

// numerics.py:270-275: FTZ, round-to-nearest-even to the top 16 bits, NaN -> 0x7FC0
__device__ __forceinline__ uint16_t to_bf16_bits(float x) {
  const uint32_t b = fbits(ftz(x));
  if ((b & 0x7FFFFFFFu) > kExpo) return 0x7FC0u;
  return static_cast<uint16_t>((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

// numerics.py:21-23: binary16 bits -> fp32, exact for subnormals, canonical NaN (branch-free)
__device__ __forceinline__ float from_fp16_bits(uint32_t h) {
  const uint32_t s = (h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, f = h & 0x3FFu;
  // f * 2^-24 is exact (f < 2^10, the product is a normal fp32)
  const uint32_t sub = fbits(static_cast<float>(f) * 5.9604644775390625e-08f) | s;
  const uint32_t normal = s | ((e + 112u) << 23) | (f << 13);
  const uint32_t special = f ? kCanonNaN : (s | kExpo);
  return ffrom(e == 31 ? special : (e == 0 ? sub : normal));
}

// binary16 bits -> fp32 by the conversion instruction (v_cvt_f32_f16): exact for every finite and
// infinite input, subnormals included (binary16 denormals are kept), so equal to from_fp16_bits
// except that a NaN keeps its sign and payload instead of becoming the canonical NaN. For values
// whose NaNs meet a canonicalization before anything is stored: the W4A16 group scales, which only
// feed the bank chains that chain_end canonicalizes.
__device__ __forceinline__ float fp16_to_f32_keep_nan(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// numerics.py:14-18: fp32 -> binary16 bits, round to nearest even with gradual underflow, signed
// zero, NaN -> 0x7E00. Integer rounding of the significand for normal results; for results below
// 2^-14 the exact product x * 2^24 (a power-of-two scaling) rounded to an integer is the subnormal's
// significand (1024 there is the smallest normal, 0x0400).
__device__ __forceinline__ uint16_t to_fp16_bits(float x) {
  const uint32_t b = fbits(x);
  const uint32_t s = (b >> 16) & 0x8000u, a = b & 0x7FFFFFFFu;
  if (a > kExpo) return 0x7E00u;
  if (a >= 0x477FF000u) return static_cast<uint16_t>(s | 0x7C00u);  // 65520 and above round to inf
  if (a >= 0x38800000u) {                                             // 2^-14 and above: normal
    const uint32_t mant = a & kMant, rem = mant & 0x1FFFu;
    uint32_t h = ((((a >> 23) - 112u)) << 10) | (mant >> 13);
    h += (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ? 1u : 0u;
    return static_cast<uint16_t>(s | h);
  }
  return static_cast<uint16_t>(s | static_cast<uint32_t>(rintf(ffrom(a) * 16777216.0f)));
}

// 1/sqrt(x) (numerics.py:171-191): E = biased exponent - 127 = 2k + j; m = x with exponent field
// 127 + j (m in [1, 4)); seed bits(y0) = 0x5F3759DF - (bits(m) >> 1); three correction-form Newton
// steps y <- y + y * (1/2 + -(1/2 * ((m * y) * y))), each op one rounded contract step; then -k is
// added to y's exponent field. +-0 -> +-inf, +inf -> +0, negative or NaN -> canonical NaN.
//
// As in recip_f, the Newton steps run on raw rounded operations: they depend only on m, and for
// every m in [1, 4) each product and sum is a positive normal value or exactly 0 (y stays in
// [0.48, 1.01]; 1/2 - (1/2)(m y^2) is exact by Sterbenz, so 0 or at least 2^-25 in magnitude), so
// the contract's flush and canonicalize wrappers change nothing (checked exhaustively on the CPU).
// The special inputs take their results by selects.
__device__ __forceinline__ float rsqrt_f(float x) {
  const uint32_t xb = fbits(ftz(x));
  const uint32_t mag = xb & 0x7FFFFFFFu;
  const int E = static_cast<int>((xb >> 23) & 0xFFu) - 127;
  const int j = E & 1, k = E >> 1;  // arithmetic shift: floor, so E = 2k + j for E < 0 too
  const uint32_t mb = (xb & kMant) | (static_cast<uint32_t>(127 + j) << 23);
  const float m = ffrom(mb), half = ffrom(kHalf);
  float y = ffrom(0x5F3759DFu - (mb >> 1));
#pragma unroll
  for (int i = 0; i < 3; ++i)
    y = __fadd_rn(y, __fmul_rn(y, __fadd_rn(half, -__fmul_rn(half, __fmul_rn(__fmul_rn(m, y), y)))));
  const float r = add_to_exponent(y, -k);
  const bool nan = mag > kExpo || ((xb & kSign) && mag != 0);
  return nan ? ffrom(kCanonNaN) : mag == 0 ? ffrom((xb & kSign) | kExpo) : xb == kExpo ? 0.0f : r;
}

// Order key of the contract's fmax (numerics.py:293-303) on a flushed, non-NaN value: unsigned
// key order is the fp order with -0 below +0, so the key maximum of a set is its fmax (+0 from
// +0 and -0, -0 only from -0s). NaN is tracked beside the key.
__device__ __forceinline__ uint32_t fmax_key(float x) {
  const uint32_t b = fbits(x);
  return (b & kSign) ? ~b : (b | kSign);
}
__device__ __forceinline__ float fmax_from_key(uint32_t k) { return ffrom((k & kSign) ? (k ^ kSign) : ~k); }

// Stores one epilogue result in the output format (golden.py:273-280).
__device__ __forceinline__ void store_out(void* Y, int64_t byte_row, int n, int out, float y,
                                          float out_scale) {
  char* row = static_cast<char*>(Y) + byte_row;
  if (out == 0) {
    reinterpret_cast<float*>(row)[n] = ftz(y);
  } else if (out == 1) {
    reinterpret_cast<uint16_t*>(row)[n] = to_bf16_bits(y);
  } else if (out == 3) {
    reinterpret_cast<uint16_t*>(row)[n] = to_fp16_bits(y);
  } else {
    reinterpret_cast<int8_t*>(row)[n] = q8(y, out_scale);
  }
}

// store_out for four consecutive columns n .. n + 3 in one vector store (n % 4 == 0; rows and
// the output base are 16-byte aligned, so the 16/8/4-byte store is naturally aligned).
__device__ __forceinline__ void store_out4(void* Y, int64_t byte_row, int n, int out, const float (&y)[4],
                                           float out_scale) {
  char* row = static_cast<char*>(Y) + byte_row;
  if (out == 0) {
    *reinterpret_cast<float4*>(row + 4 * n) = make_float4(ftz(y[0]), ftz(y[1]), ftz(y[2]), ftz(y[3]));
  } else if (out == 1) {
    *reinterpret_cast<uint2*>(row + 2 * n) =
        make_uint2(to_bf16_bits(y[0]) | static_cast<uint32_t>(to_bf16_bits(y[1])) << 16,
                   to_bf16_bits(y[2]) | static_cast<uint32_t>(to_bf16_bits(y[3])) << 16);
  } else {
    uint32_t v = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) v |= static_cast<uint32_t>(static_cast<uint8_t>(q8(y[q], out_scale))) << (8 * q);
    *reinterpret_cast<uint32_t*>(row + n) = v;
  }
}

// The W8A8 epilogue after the exact integer sum (golden.py:340-349).
struct RowColEpilogue {
  const float* srow;   // nullptr: no row scale (QM_CHANNEL / QM_TENSOR)
  const float* scol;
  int scol_per_tensor; // 1: scol[0] for every column (QM_TENSOR)
  const float* bias;   // nullptr: none
  int act;
  int out;
  float out_scale;

  __device__ __forceinline__ float value(int32_t acc, int m, int n) const {
    return value_sr(acc, srow ? srow[m] : 0.0f, srow != nullptr, n);
  }

  // The same with the row scale given by value (a quantizer fused into the GEMV).
  __device__ __forceinline__ float value_sr(int32_t acc, float sr, bool has_sr, int n) const {
    return apply(acc, sr, has_sr, scol[scol_per_tensor ? 0 : n], bias ? bias[n] : 0.0f);
  }

  // The epilogue's operands, fetched early so their latency hides under the weights. Every load
  // is unconditional (an absent operand reads scol[0], a valid address, and is ignored): a load
  // behind a branch would make the compiler drain every outstanding load where the paths join.
  __device__ __forceinline__ float load_scol(int n) const { return scol[scol_per_tensor ? 0 : n]; }
  __device__ __forceinline__ float load_bias(int n) const { return *(bias ? bias + n : scol); }
  __device__ __forceinline__ float load_srow(int m) const { return *(srow ? srow + m : scol); }

  __device__ __forceinline__ float apply(int32_t acc, float sr, bool has_sr, float sc, float b) const {
    float y = i2f(acc);
    if (has_sr) y = fmul(y, sr);
    y = fmul(y, sc);
    if (bias) y = fadd(y, b);
    return act_fn(y, act);
  }
};

// Per-token quantizer pieces shared by the quant_rows kernel and the fused quantize + GEMV
// kernels (numerics.py:383-390).
//
// The row maximum of |ftz(x)| as an unsigned maximum of encodings: the maximum of the unflushed
// |x| encodings, flushed once. A normal, infinite or NaN element dominates every subnormal one, so
// flushing the subnormals first changes the maximum only when every element is zero or subnormal,
// and then both give +0.
__device__ __forceinline__ uint32_t abs_bits(float v) { return fbits(v) & 0x7FFFFFFFu; }
__device__ __forceinline__ uint32_t abs_bits_ftz(float v) {
  const uint32_t b = abs_bits(v);
  return b < 0x00800000u ? 0u : b;  // ftz then |.|: a subnormal counts as +0
}
__device__ __forceinline__ uint32_t max_abs_bits4(uint32_t m, float4 v) {
  return max(max(m, max(abs_bits(v.x), abs_bits(v.y))), max(abs_bits(v.z), abs_bits(v.w)));
}
__device__ __forceinline__ uint32_t flush_max_bits(uint32_t m) { return m < 0x00800000u ? 0u : m; }

// amax encoding (an unsigned max of |x| encodings; any NaN encoding wins) -> (inv, s). inv is the
// contract's fmul(127, recip_f(amax)) written out: recip_f's result is 0, at least 2^-126, infinite
// or the canonical NaN, so 127 times it is never subnormal and needs only the canonicalization.
__device__ __forceinline__ void quant_scales(uint32_t amax_bits, float& inv, float& s) {
  const float amax = ffrom(amax_bits > kExpo ? kCanonNaN : amax_bits);
  inv = canon(__fmul_rn(ffrom(kQ127), recip_f(amax)));
  s = fmul(amax, ffrom(kInv127));
}

// Four q8 bytes packed little-endian; inv must come from fmul (flushed), as quant_scales gives it.
__device__ __forceinline__ uint32_t q8x4(float a, float b, float c, float d, float inv) {
  return (static_cast<uint32_t>(q8_flushed_inv(a, inv)) & 0xFFu) |
         ((static_cast<uint32_t>(q8_flushed_inv(b, inv)) & 0xFFu) << 8) |
         ((static_cast<uint32_t>(q8_flushed_inv(c, inv)) & 0xFFu) << 16) |
         ((static_cast<uint32_t>(q8_flushed_inv(d, inv)) & 0xFFu) << 24);
}

// Four q8 bytes of a row for which q8_fast_row holds, packed little-endian. q8 is then
// clamp(rint(x * inv), -127, 127) on the unflushed x (above), and the clamp is the identity:
// |x * inv| <= amax * inv < 127.5 for every such amax (checked on the CPU for every mantissa of amax;
// the exponent cancels). t = x * inv is rounded once; adding 1.5 * 2^23 rounds it to an integer in
// the sum's last mantissa bits (the sum lies in [2^23, 2^24), where the spacing is 1, and ties go
// to even as rint's do, 1.5 * 2^23 being even), so the low byte of the sum's encoding is
// rint(t) mod 256, the two's-complement q8 byte; three byte permutes gather the four bytes.
// A subnormal x gives |t| < 1/2 and the byte 0, as its flush does.
__device__ __forceinline__ uint32_t q8x4_fast(float a, float b, float c, float d, float inv) {
  const float kRound = 12582912.0f;  // 1.5 * 2^23
  const uint32_t ea = fbits(__fadd_rn(__fmul_rn(a, inv), kRound));
  const uint32_t eb = fbits(__fadd_rn(__fmul_rn(b, inv), kRound));
  const uint32_t ec = fbits(__fadd_rn(__fmul_rn(c, inv), kRound));
  const uint32_t ed = fbits(__fadd_rn(__fmul_rn(d, inv), kRound));
  // v_perm_b32 (hi, lo, sel): selector byte k picks byte k of lo (0-3) or byte k-4 of hi (4-7); 0x0C is 0
  const uint32_t ab = __builtin_amdgcn_perm(eb, ea, 0x0C0C0400u);  // [a, b, 0, 0]
  const uint32_t cd = __builtin_amdgcn_perm(ed, ec, 0x0C0C0400u);  // [c, d, 0, 0]
  return __builtin_amdgcn_perm(cd, ab, 0x05040100u);                 // [a, b, c, d]
}

}  // namespace tars
