// W4A16: block-FP activation alignment (tars_mini/numerics.py:55-98) and the group-128 GEMV
// (tars_mini/golden.py:295-324).
//
// Work unit: a 16-byte chunk of a packed weight row = 32 int4 weights = a quarter of a 128-wide
// group. A wave owns whole rows; lane l streams chunks l, l + 64, ... of each, so a group's four
// chunks sit on four consecutive lanes (a quad).
//
// Alignment is fused into the GEMV prologue: the workgroup aligns each activation row once,
// cooperatively (16 lanes per 128-wide group, 8 elements each; the group's exponent maximum meets
// through DPP lane permutes). Each mantissa (an int16 in [-16384, 16384]) is rounded to
// nearest-even exactly as the reference does: for finite groups as rint(x * 2^(140 - e_eff)),
// otherwise by the integer shift rule with the NaN / infinity cases.
//
// Exact int16 x int4 dots on v_dot8_i32_i4: each mantissa is written in balanced base 16 (four
// signed digits in [-8, 7]); LDS holds one "digit plane" per digit, 8 elements per dword in the
// packed weights' nibble order, so a weight dword dotted with plane i gives sum w d_i exactly and
// the chunk's dot is P0 + 16 P1 + 256 P2 + 4096 P3 (16 dot instructions per chunk and row; the
// former byte split needed 28 instructions).
//
// The per-group fp32 terms (i2f(dot) * ws) * xs meet in four bank chains per output (group g goes
// to bank g % 4, added in g order from +0), combined as (b0 + b1) + (b2 + b3) before bias,
// activation and conversion: with one activation row the terms stay in registers and the chain
// lanes gather them by permlane swaps; otherwise they go through the wave's own LDS rows (the
// quad's four lanes form the terms of four different rows in one instruction stream). The only
// workgroup barrier is the one after the alignment. Two more forms follow the GEMV: one
// activation row with K split over the waves of a workgroup, and the INT8 MFMA form for prefill
// chunks.
//
// Roofline: HBM. Algorithmic bytes per row: K/2 (weights) + K/64 (fp16 scales) + 4 (output). The
// kernels also carry VALU work per weight byte (dots, terms, chains) that measured as the larger
// share of a call at these sizes; see the launcher's notes.
#include "kernels.h"

namespace tars {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kGroup = 128;

// The 32 fp32 encodings of this thread's chunk of activation row `m`, flushed.
__device__ __forceinline__ void load_chunk_bits(const void* x, int64_t lda, int bf16, int m, int c,
                                                uint32_t xb[32]) {
  const char* row = static_cast<const char*>(x) + m * lda;
  if (bf16) {
    const v4u* p = reinterpret_cast<const v4u*>(row + c * 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const v4u v = p[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xb[8 * i + 2 * j] = v[j] << 16;
        xb[8 * i + 2 * j + 1] = v[j] & 0xFFFF0000u;
      }
    }
  } else {
    const v4u* p = reinterpret_cast<const v4u*>(row + c * 128);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const v4u v = p[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) xb[4 * i + j] = v[j];
    }
  }
#pragma unroll
  for (int i = 0; i < 32; ++i) xb[i] = (xb[i] & kExpo) ? xb[i] : (xb[i] & kSign);  // ftz
}

// Aligns NE elements held by each of GL consecutive lanes that together form one 128-wide group
// (NE * GL == 128; every lane of the wave must call it, dead lanes on shadow data). Inputs are raw
// fp32 encodings (not flushed). Outputs the signed mantissas (their low 16 bits: int16 values) and
// the group's fp32 scale encoding.
template <int NE, int GL>
__device__ __forceinline__ void align_elems(const uint32_t* xraw, int* mant, uint32_t& scale_bits) {
  static_assert(NE * GL == kGroup, "a group is 128 elements");
  // A subnormal's exponent field is 0 whether or not it is flushed, so emax needs no flush.
  int emax = 0;
#pragma unroll
  for (int i = 0; i < NE; ++i) emax = max(emax, static_cast<int>((xraw[i] >> 23) & 0xFF));
  emax = group_reduce<GL>(emax, OpMaxU{});
  const int e_eff = max(emax, 14);
  if (__builtin_amdgcn_ballot_w64(emax < 16 || emax == 255) == 0) {
    // Every group of the wave is finite with emax >= 16 (the usual case). For a finite x of
    // exponent e the reference's mantissa is its significand shifted right by sh = 10 + e_eff - e
    // with round-to-nearest-even, i.e. rint(sig * 2^-sh) = rint(x * 2^(140 - e_eff)): one exact
    // power-of-two product (|result| <= 2^14) and v_rndne_f32 (round half to even), the sign
    // carried through. A product small enough to be subnormal is far below 1/2 and rounds to 0,
    // and so does an unflushed subnormal input (|x * 2^(140 - e_eff)| < 2^-126 * 2^124), so no
    // flush is needed. Equal to the shift rule for every significand and shift (exhaustive CPU
    // check) and on real rows, flushed or not (CPU check against the aligner's restatement).
    // One fma per element: x * p is exact and |x * p| < 2^14, so RN(x * p + 1.5 * 2^23) is
    // 1.5 * 2^23 + rint(x * p) (ties to even; its ulp is 1) and the encoding's low 16 bits are the
    // mantissa as an int16, the only bits the digit planes and the aligned rows take.
    const float p = __uint_as_float(static_cast<uint32_t>(267 - e_eff) << 23);
#pragma unroll
    for (int i = 0; i < NE; ++i)
      mant[i] = static_cast<int>(__float_as_uint(__builtin_fmaf(__uint_as_float(xraw[i]), p, 12582912.0f)));
    scale_bits = static_cast<uint32_t>(e_eff - 13) << 23;
    return;
  }
  // Some group of the wave holds a NaN or an infinity, or is all zeros / tiny (emax < 16).
  uint32_t xb[NE];
  int flags = 0;
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    xb[i] = (xraw[i] & kExpo) ? xraw[i] : (xraw[i] & kSign);  // ftz
    const int e = (xb[i] >> 23) & 0xFF;
    flags |= e == 255 ? ((xb[i] & kMant) ? 1 : 2) : 0;
  }
  flags = group_reduce<GL>(flags, OpOr{});
  const bool grp_nan = flags & 1;
  const bool grp_inf = ((flags & 2) != 0) & !grp_nan;
  // Round-to-nearest-even right shift as (sig + 2^(sh-1) - 1 + lsb) >> sh (equal to the
  // reference's kept/dropped/half rule for every 24-bit significand and shift; checked
  // exhaustively on the CPU); exponent 0 (a flushed zero) has significand 0.
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    const uint32_t b = xb[i];
    const int e = (b >> 23) & 0xFF;
    const uint32_t frac = b & kMant;
    const uint32_t sig = ((e != 0) & (e != 255)) ? (frac | (1u << 23)) : 0u;
    const uint32_t sh = static_cast<uint32_t>(min(10 + e_eff - e, 31));
    int mag = static_cast<int>((sig + ((1u << (sh - 1u)) - 1u) + ((sig >> sh) & 1u)) >> sh);
    mag = (grp_inf & (e == 255) & (frac == 0)) ? 16384 : mag;
    mag = grp_nan ? 0 : mag;
    mant[i] = (b & kSign) ? -mag : mag;
  }
  uint32_t sb = emax == 0 ? 0u : static_cast<uint32_t>(e_eff - 13) << 23;
  sb = grp_inf ? kExpo : sb;
  scale_bits = grp_nan ? kCanonNaN : sb;
}

__device__ __forceinline__ void align_chunk(const uint32_t xb[32], int mant[32], uint32_t& scale_bits) {
  align_elems<32, 4>(xb, mant, scale_bits);
}

// ---------------------------------------------------------------------------- align (standalone)
__global__ __launch_bounds__(kThreads) void align_w4_kernel(AlignArgs a) {
  const int C = a.K / 32;
  const int t = blockIdx.x * kThreads + threadIdx.x;
  const int m = blockIdx.y;
  const bool live = t < C;
  const int c = live ? t : C - 1;  // dead lanes shadow a live chunk so group shuffles stay defined
  uint32_t xb[32];
  load_chunk_bits(a.x, a.lda, a.bf16, m, c, xb);
  int mant[32];
  uint32_t sb;
  align_chunk(xb, mant, sb);
  if (!live) return;
  int16_t* qrow = reinterpret_cast<int16_t*>(reinterpret_cast<char*>(a.q) + m * a.ldq);
  v4i* dst = reinterpret_cast<v4i*>(qrow + 32 * c);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v4i v;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      v[j] = static_cast<int>((static_cast<uint32_t>(mant[8 * i + 2 * j]) & 0xFFFFu) |
                              (static_cast<uint32_t>(mant[8 * i + 2 * j + 1]) << 16));
    dst[i] = v;
  }
  if ((c & 3) == 0) {
    float* srow = reinterpret_cast<float*>(reinterpret_cast<char*>(a.scales) + m * a.lds);
    srow[c >> 2] = ffrom(sb);
  }
}

// ---------------------------------------------------------------------------- GEMV
// Digit planes. An aligned mantissa a (|a| <= 2^14) is written in balanced base 16,
// a = d0 + 16 d1 + 256 d2 + 4096 d3 with every digit in [-8, 7]; digit i's nibble (d_i mod 16) is
// floor((a + c_i) / 16^i) mod 16 with c = {0, 8, 136, 2184}, and the top digit is in [-4, 4]. A
// plane dword holds one digit of 8 consecutive elements, element e in nibble e: the same nibble
// order as a packed weight dword (low nibble of byte b = k 2b, high nibble = k 2b + 1). Then
// v_dot8_i32_i4 of a weight dword with plane i is sum_e w_e d_{i,e} exactly, and the chunk's dot is
// P0 + 16 P1 + 256 P2 + 4096 P3 (|dot| <= 2^24 per group: exact in int32).
__device__ __forceinline__ void digit_planes(const int mant[8], uint32_t pl[4]) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  constexpr unsigned kC[4] = {0, 8, 136, 2184};
  // elements e and e + 4 as the two 16-bit halves of one register (|a| <= 2^14 and a + c_i fit
  // in 16 bits, so 16-bit adds give the low 16 bits of a + c_i), then per plane and pair: one
  // packed add, one packed shift moving nibble i of both halves to nibble positions e and e + 4
  // of their halves, one masked or into the plane
  u16x2 pr[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    pr[e] = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(static_cast<uint32_t>(mant[e + 4]),
                                                           static_cast<uint32_t>(mant[e]), 0x05040100u));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t v = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      u16x2 q = pr[e] + u16x2{static_cast<unsigned short>(kC[i]), static_cast<unsigned short>(kC[i])};
      if (e > i) q = q << static_cast<unsigned short>(4 * (e - i));
      if (e < i) q = q >> static_cast<unsigned short>(4 * (i - e));
      v |= __builtin_bit_cast(uint32_t, q) & (0x000F000Fu << (4 * e));
    }
    pl[i] = v;
  }
}

// exact dot of a chunk's 32 weights (4 dwords) with its 32 elements' digit planes
__device__ __forceinline__ int chunk_dot_digits(v4u w, const v4u x[4]) {
  int p[4] = {0, 0, 0, 0};
#pragma unroll
  for (int d = 0; d < 4; ++d)
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_sdot8(static_cast<int>(w[d]), static_cast<int>(x[i][d]), p[i], false);
  return p[0] + (p[1] << 4) + (p[2] << 8) + (p[3] << 12);
}

// A wave owns U consecutive weight rows; lane l streams chunks l, l + 64, ... (CPL per lane) of
// each, so a 128-wide group's four chunks sit on four consecutive lanes (a quad). A workgroup of
// NW waves shares one alignment of each of its MR activation rows.
//
// 1. One batch of loads: the activation rows (only the waves that align them), the wave's fp16
//    group scales (U * G halves, contiguous: one dword per lane), then the U * CPL weight chunks.
//    A lane past the row's last chunk re-reads that chunk, a row past N re-reads row N - 1 (the
//    values are never used): addresses stay inside rows the wave streams anyway (a fixed fallback
//    address shared by every wave measured as a hot spot).
// 2. Aligner thread t (t < K / 8) owns elements 8 t .. 8 t + 7 of a row; 16 threads form a
//    128-wide group (exponent maximum and flags by DPP). Digit planes and the group scale go to LDS.
//    The only workgroup barrier follows.
// 3. Per chunk, row and activation row: 16 v_dot8 and the digit combination; the quad adds its
//    four chunks (DPP). Lane q of the quad forms the terms (i2f(dot) * ws) * xs of the rows
//    u = q, q + 4, ... into the wave's LDS terms.
// 4. Lane 4 (m U + u) + b runs bank b's chain of row u, activation row m: groups b, b + 4, ... in
//    order from +0 (every term read first, the adds unflushed with the subnormal check and redone
//    with the flushes when a partial sum is subnormal), and the quad folds (b0 + b1) + (b2 + b3).
constexpr int kTermStride = 65;  // LDS floats per term row (G <= 64), padded against bank conflicts

template <int NW, int U, int MR, int CPL>
struct W4Smem {
  float terms[NW][MR * U][kTermStride];
  uint32_t ws[NW][U * 32];                             // U rows x G <= 64 halves per wave
  float xs[MR][64];
  // then the digit planes: MR rows x 4 planes x 4C dwords (dynamic)
};

// What the first loads need (x, lda, the weight and scale pointers, M, N, K) leads the kernel
// arguments as scalars, preloaded into SGPRs at wave launch; the epilogue's fields follow in `a`
// and are read through the kernel-argument segment once the streams are in flight.
struct W4Kernargs {
  const void* x;
  int64_t lda;
  const uint8_t* Wp;
  const uint16_t* ws;
  int M, N, K;
  W4Args a;
};
constexpr size_t kW4ArgsOffset = offsetof(W4Kernargs, a);
static_assert(kW4ArgsOffset == 48, "the preloaded scalars take 48 bytes before the argument block");

// The MFMA form's leading scalars: x, the weight and scale pointers, lda, M, N, K.
struct W4MfmaKernargs {
  const void* x;
  const uint8_t* Wp;
  const uint16_t* ws;
  int lda, M, N, K;
  W4Args a;
};
constexpr size_t kW4MfmaArgsOffset = offsetof(W4MfmaKernargs, a);
static_assert(kW4MfmaArgsOffset == 40, "the preloaded scalars take 40 bytes before the argument block");

template <int NW, int U, int MR, int CPL, bool BF16, bool SIMPLE>
__global__ __launch_bounds__(NW * 64) void gemv_w4a16_kernel(const void* x, int64_t lda, const uint8_t* Wp,
                                                             const uint16_t* ws, int M, int N, int K, W4Args a) {
  static_assert(CPL >= 1 && CPL <= 4 && MR * U * 4 <= 64, "K <= 8192; one chain lane per bank");
  constexpr int NT = NW * 64;
  constexpr int AP = (CPL * 256 + NT - 1) / NT;       // aligner passes (K / 8 <= 256 CPL threads)
  using Smem = W4Smem<NW, U, MR, CPL>;
  __shared__ Smem sm;
  extern __shared__ __align__(16) uint32_t planes[];    // [MR][4][4C]
  const int C = K >> 5;
  const int G = K >> 7;
  const int A = K >> 3;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m0 = blockIdx.y * MR;
  const int n0 = (blockIdx.x * NW + wave) * U;
  const int64_t row_bytes = K >> 1;

  // 1. activations (per pass: whole waves only; dead lanes of a live wave shadow group 0)
  uint32_t xb[MR][AP][8];
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    const char* xrow = static_cast<const char*>(x) + min(m0 + r, M - 1) * lda;
#pragma unroll
    for (int p = 0; p < AP; ++p) {
      const int t = p * NT + tid;
      if (p * NT + wave * 64 >= A) continue;                   // wave-uniform
      const int tt = t < A ? t : (t & 15);
      if constexpr (BF16) {
        const v4u v = *reinterpret_cast<const v4u*>(xrow + 16 * tt);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          xb[r][p][2 * j] = v[j] << 16;
          xb[r][p][2 * j + 1] = v[j] & 0xFFFF0000u;
        }
      } else {
        const v4u* src = reinterpret_cast<const v4u*>(xrow + 32 * tt);
        const v4u v0 = src[0], v1 = src[1];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          xb[r][p][j] = v0[j];
          xb[r][p][4 + j] = v1[j];
        }
      }
    }
  }
  issue_fence();
  // the wave's group scales: halves [n0 G, (n0 + U) G) as dwords (G is even), clamped at the end
  const int ws_dw = (U * G) >> 1;
  const uint32_t* ws32 = reinterpret_cast<const uint32_t*>(ws);
  const int64_t ws_last = (static_cast<int64_t>(N) * G >> 1) - 1;
  constexpr int kWsPer = (U * 32 + 63) / 64;          // dwords per lane: U rows x G <= 64 halves
  uint32_t wsv[kWsPer];
#pragma unroll
  for (int i = 0; i < kWsPer; ++i)
    wsv[i] = ws32[min(static_cast<int64_t>(n0) * G / 2 + min(lane + 64 * i, ws_dw - 1), ws_last)];
  issue_fence();
  v4u wv[U][CPL];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const v4u* wrow = reinterpret_cast<const v4u*>(Wp + min(n0 + u, N - 1) * row_bytes);
#pragma unroll
    for (int j = 0; j < CPL; ++j) wv[u][j] = __builtin_nontemporal_load(wrow + min(lane + 64 * j, C - 1));
  }
  issue_fence();
  // the epilogue's fields, their loads issued now and waited for at their first use
  const KArg ka = kernarg_at(kW4ArgsOffset);
  void* const Y = kload<void*>(ka + offsetof(W4Args, Y));
  const int64_t ldy = kload<int64_t>(ka + offsetof(W4Args, ldy));
  const float* const bias = SIMPLE ? nullptr : kload<const float*>(ka + offsetof(W4Args, bias));
  const int act = SIMPLE ? 0 : kload<int>(ka + offsetof(W4Args, act));
  const int out = SIMPLE ? 0 : kload<int>(ka + offsetof(W4Args, out));
  const float out_scale = SIMPLE ? 0.0f : kload<float>(ka + offsetof(W4Args, out_scale));
  // chain lanes. One activation row and at most four rows per wave: lane 4 b + u (b, u < 4) runs
  // bank b of row u, its terms gathered from the four 16-lane rows by permlane swaps (kRegChain);
  // otherwise lane 4 (m U + u) + b, its terms through LDS.
  constexpr bool kRegChain = MR == 1 && U <= 4;
  const int ce = kRegChain ? (lane & 3) : lane >> 2, bank = kRegChain ? (lane >> 2) & 3 : lane & 3;
  const int ue = ce % U, me = ce / U;
  const bool chain_lane = kRegChain ? lane < 16 && (lane & 3) < U : ce < MR * U;
  float bias_v = 0.0f;

  // 2. alignment into LDS digit planes
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    uint32_t* pl = planes + r * 16 * C;
#pragma unroll
    for (int p = 0; p < AP; ++p) {
      if (p * NT + wave * 64 >= A) continue;                   // wave-uniform
      const int t = p * NT + tid;
      int mant[8];
      uint32_t sb;
      align_elems<8, 16>(xb[r][p], mant, sb);
      if (t < A) {
        uint32_t d[4];
        digit_planes(mant, d);
#pragma unroll
        for (int i = 0; i < 4; ++i) pl[i * 4 * C + t] = d[i];
        if ((t & 15) == 0) sm.xs[r][t >> 4] = ffrom(sb);
      }
    }
  }
  if constexpr (!SIMPLE) bias_v = *(bias ? bias + min(n0 + ue, N - 1) : reinterpret_cast<const float*>(ws));
  // the wave's scales into its LDS slot (read back by other lanes of the wave after the barrier)
#pragma unroll
  for (int i = 0; i < kWsPer; ++i)
    if (lane + 64 * i < ws_dw) sm.ws[wave][lane + 64 * i] = wsv[i];
  __syncthreads();

  // 3. dots and terms
  const uint16_t* wsh = reinterpret_cast<const uint16_t*>(sm.ws[wave]);
  const int q = lane & 3;
  float T[CPL];  // kRegChain: this lane's term of chunk j (row q, group (lane >> 2) + 16 j)
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    const int cc = c < C ? c : 0;
    const int g = cc >> 2;
#pragma unroll
    for (int r = 0; r < MR; ++r) {
      v4u x[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = *reinterpret_cast<const v4u*>(planes + r * 16 * C + i * 4 * C + 4 * cc);
      const float xs = sm.xs[r][g];
      int dots[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int d = chunk_dot_digits(wv[u][j], x);
        d += lane_xor1(d);
        d += lane_xor2(d);
        dots[u] = d;
      }
      // lane q of the quad forms the terms of rows q, q + 4, ... in one instruction stream
#pragma unroll
      for (int k = 0; k < (U + 3) / 4; ++k) {
        const int u = q + 4 * k;
        int d = dots[4 * k];
#pragma unroll
        for (int v = 1; v < 4; ++v)
          if (4 * k + v < U) d = q == v ? dots[4 * k + v] : d;
        // the contract's fmul(fmul(i2f(d), ws), xs) with its wrappers where they act: i2f(d) is exact
        // (|d| <= 2^24) and the fp16 scale is an fp32 normal, infinity or NaN, so the first product
        // is 0, at least 2^-24 in magnitude, infinite or NaN (no flush); the second is flushed; a NaN
        // payload only feeds the chains, whose results are canonicalized
        const float term = ftz(__fmul_rn(__fmul_rn(i2f(d), fp16_to_f32_keep_nan(wsh[min(u, U - 1) * G + g])), xs));
        // a chunk past the row (its group past the last) gives the term +0, which the chains add
        // as a no-op (below)
        if constexpr (kRegChain) T[j] = c < C ? term : 0.0f;
        else if (u < U && n0 + u < N) sm.terms[wave][r * U + u][c >> 2] = c < C ? term : 0.0f;
      }
    }
  }
  // 4. bank chains (at most G / 4 <= 4 CPL steps): step i adds group g = bank + 4 i
  constexpr int kSteps = 4 * CPL;
  float tv[kSteps];
  if constexpr (kRegChain) {
    // group g = bank + 4 i is on lane 4 b + u + 16 (i & 3), chunk i >> 2: for a lane of row 0,
    // the lanes 16, 32 and 48 above it, gathered with permlane swaps (no LDS, no barrier)
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint32_t t0 = __float_as_uint(T[j]);
      const uint32_t t1 = __builtin_amdgcn_permlane16_swap(t0, t0, false, false)[1];  // lane + 16 (row 2: + 48)
      const uint32_t t2 = __builtin_amdgcn_permlane32_swap(t0, t0, false, false)[1];  // lane + 32
      const uint32_t t3 = __builtin_amdgcn_permlane32_swap(t1, t1, false, false)[1];  // lane + 48
      tv[4 * j] = T[j];
      tv[4 * j + 1] = __uint_as_float(t1);
      tv[4 * j + 2] = __uint_as_float(t2);
      tv[4 * j + 3] = __uint_as_float(t3);
    }
  } else {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float* trow = sm.terms[wave][ce < MR * U ? ce : 0];
#pragma unroll
    for (int i = 0; i < kSteps; ++i) tv[i] = trow[bank + 4 * i];  // index <= 16 CPL - 1 < kTermStride
  }
  // the unflushed chain runs all 4 CPL steps: the steps past the row's last group add +0, and a
  // sum that starts from +0 never becomes -0 under round-to-nearest (x + y is -0 only when both are
  // -0), so adding +0 leaves it and its subnormal key unchanged. The flushed recompute stops at the
  // last group: a negative subnormal partial sum flushes to -0, which a +0 step would turn into +0
  float acc = 0.0f;
  uint32_t mk = ~0u;
#pragma unroll
  for (int i = 0; i < kSteps; ++i) {
    acc = __fadd_rn(acc, tv[i]);
    mk = min(mk, sub_key(acc));
  }
  if (__builtin_expect(mk < kSubKeyNormal, 0)) {
    acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kSteps; ++i)
      if (bank + 4 * i < G) acc = fadd_chain(acc, tv[i]);
  }
  acc = chain_end(acc);
  // bank 0: b0 + b1, bank 2: b2 + b3 (the next bank's lane: 1 above, or 4 above by a row rotation)
  const float pair = fadd(acc, kRegChain ? __int_as_float(dpp<kDppRowRor12>(__float_as_int(acc))) : lane_xor1(acc));
  const float other = kRegChain ? __int_as_float(dpp<kDppRowRor8>(__float_as_int(pair))) : lane_xor2(pair);
  if (bank == 0 && chain_lane && n0 + ue < N && m0 + me < M) {
    float y = fadd(pair, other);
    const int64_t yrow = static_cast<int64_t>(m0 + me) * ldy;
    if constexpr (SIMPLE) {
      reinterpret_cast<float*>(static_cast<char*>(Y) + yrow)[n0 + ue] = ftz(y);
    } else {
      if (bias) y = fadd(y, bias_v);
      y = act_fn(y, act);
      store_out(Y, yrow, n0 + ue, out, y, out_scale);
    }
  }
}

// One activation row with K split over the waves of a workgroup. Wave w owns groups 4 w .. 4 w + 3
// (one per bank; the last wave two when G % 4 == 2) of the workgroup's 4 RS weight rows, and
// aligns just those groups of the activation itself (lane l: group 4 w + l / 16, elements
// 8 (l % 16) .. + 7), so no alignment waits behind a workgroup barrier and each wave's work does
// not grow with K. Lane 16 u + 4 g + q streams quarter q of group 4 w + g of row 4 s + u for each
// row set s; the four aligner lanes 16 g + 4 q .. + 3 hold that quarter's 32 elements, so the
// chunk's four digit planes are one 16-byte read each from the wave's own LDS slot (a wave
// barrier, no workgroup one). The quad adds its four chunk dots and lane q = 0 stores the group's
// term (i2f(dot) * ws) * xs in the workgroup's term rows; after the one workgroup barrier, wave
// 0's lane 4 r + b runs bank b's chain of row r over groups b, b + 4, ... in order from +0
// (golden.py:315-319) and each quad folds (b0 + b1) + (b2 + b3).
// Roofline: HBM, K / 2 + K / 64 bytes per weight row; the activation (2 or 4 bytes per element)
// is read once per workgroup, from L2.
template <int RS, bool BF16, bool SIMPLE>
__global__ __launch_bounds__(1024) void gemv_w4a16_kslice_kernel(const void* x, int64_t lda, const uint8_t* Wp,
                                                                 const uint16_t* ws, int M, int N, int K, W4Args a) {
  constexpr int R = 4 * RS;
  __shared__ __align__(16) uint32_t planes[16][4][64];   // [wave][digit plane][aligner lane]
  __shared__ float xs_t[16][4];                          // [wave][group of the wave]
  __shared__ float terms[R][kTermStride];                // [row][group]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = K >> 7;
  const int g0 = 4 * wave, ng = min(4, G - g0);  // 2 or 4 (G is even)
  const int n0 = blockIdx.x * R;

  // 1. the wave's groups of the activation (lanes of a group past the wave's last shadow its
  //    first), then the weight chunks and their fp16 scales (rows past N read row N - 1)
  const int gl = lane >> 4;
  const int xg = g0 + (gl < ng ? gl : 0);
  uint32_t xb[8];
  if constexpr (BF16) {
    const v4u v = *reinterpret_cast<const v4u*>(static_cast<const char*>(x) + 2 * (xg * kGroup + 8 * (lane & 15)));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xb[2 * j] = v[j] << 16;
      xb[2 * j + 1] = v[j] & 0xFFFF0000u;
    }
  } else {
    const v4u* src = reinterpret_cast<const v4u*>(static_cast<const char*>(x) + 4 * (xg * kGroup + 8 * (lane & 15)));
    const v4u v0 = src[0], v1 = src[1];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xb[j] = v0[j];
      xb[4 + j] = v1[j];
    }
  }
  issue_fence();
  const int u = lane >> 4, gq = (lane >> 2) & 3, q = lane & 3;
  const int wg = g0 + (gq < ng ? gq : 0);
  v4u wv[RS];
  uint32_t wsv[RS];
#pragma unroll
  for (int s = 0; s < RS; ++s) {
    const int64_t row = min(n0 + 4 * s + u, N - 1);
    wv[s] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(Wp + row * (K >> 1) + 64 * wg + 16 * q));
    wsv[s] = ws[row * G + wg];
  }
  issue_fence();
  const KArg ka = kernarg_at(kW4ArgsOffset);
  void* const Y = kload<void*>(ka + offsetof(W4Args, Y));
  const float* const bias = SIMPLE ? nullptr : kload<const float*>(ka + offsetof(W4Args, bias));
  const int act = SIMPLE ? 0 : kload<int>(ka + offsetof(W4Args, act));
  const int out = SIMPLE ? 0 : kload<int>(ka + offsetof(W4Args, out));
  const float out_scale = SIMPLE ? 0.0f : kload<float>(ka + offsetof(W4Args, out_scale));

  // 2. alignment into the wave's digit planes and group scales
  {
    int mant[8];
    uint32_t sb;
    align_elems<8, 16>(xb, mant, sb);
    uint32_t d[4];
    digit_planes(mant, d);
#pragma unroll
    for (int i = 0; i < 4; ++i) planes[wave][i][lane] = d[i];
    if ((lane & 15) == 0) xs_t[wave][gl] = ffrom(sb);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // 3. dots and terms
  v4u xp[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xp[i] = *reinterpret_cast<const v4u*>(&planes[wave][i][16 * gq + 4 * q]);
  const float xs = xs_t[wave][gq];
#pragma unroll
  for (int s = 0; s < RS; ++s) {
    int d = chunk_dot_digits(wv[s], xp);
    d += lane_xor1(d);
    d += lane_xor2(d);
    // the contract's fmul(fmul(i2f(d), ws), xs) with its wrappers where they act (see the GEMV)
    const float term = ftz(__fmul_rn(__fmul_rn(i2f(d), fp16_to_f32_keep_nan(wsv[s])), xs));
    if (q == 0 && gq < ng) terms[4 * s + u][g0 + gq] = term;
  }
  __syncthreads();
  if (wave != 0) return;

  // 4. chains: lane 4 r + b runs bank b of row r (lanes past the last row read row 0)
  const int r = lane >> 2, bank = lane & 3;
  const float* trow = terms[r < R ? r : 0];
  float tv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) tv[i] = bank + 4 * i < G ? trow[bank + 4 * i] : 0.0f;
  float acc = 0.0f;
  uint32_t mk = ~0u;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (bank + 4 * i < G) {
      acc = __fadd_rn(acc, tv[i]);
      mk = min(mk, sub_key(acc));
    }
  if (__builtin_expect(mk < kSubKeyNormal, 0)) {
    acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (bank + 4 * i < G) acc = fadd_chain(acc, tv[i]);
  }
  acc = chain_end(acc);
  const float pair = fadd(acc, lane_xor1(acc));
  const float other = lane_xor2(pair);
  const int n = n0 + r;
  if (bank == 0 && r < R && n < N) {
    float y = fadd(pair, other);
    if constexpr (SIMPLE) {
      static_cast<float*>(Y)[n] = ftz(y);
    } else {
      if (bias) y = fadd(y, bias[n]);
      y = act_fn(y, act);
      store_out(Y, 0, n, out, y, out_scale);
    }
  }
}

template <int RS>
hipError_t go_w4_kslice(const W4Args& a, hipStream_t s) {
  const dim3 grid((a.N + 4 * RS - 1) / (4 * RS)), block(64 * ((a.K / 128 + 3) / 4));
  const bool simple = !a.bias && a.act == 0 && a.out == 0;
#define TARS_W4K(BF, SI)                                                                                      \
  hipLaunchKernelGGL((gemv_w4a16_kslice_kernel<RS, BF, SI>), grid, block, 0, s, a.x, a.lda, a.Wp, a.ws, a.M, \
                     a.N, a.K, a)
  if (a.bf16) {
    if (simple) TARS_W4K(true, true);
    else TARS_W4K(true, false);
  } else {
    if (simple) TARS_W4K(false, true);
    else TARS_W4K(false, false);
  }
#undef TARS_W4K
  return hipGetLastError();
}

template <int NW, int U, int MR, int CPL>
hipError_t go_w4(const W4Args& a, hipStream_t s) {
  const dim3 grid((a.N + NW * U - 1) / (NW * U), (a.M + MR - 1) / MR);
  const size_t lds = static_cast<size_t>(MR) * (a.K / 32) * 64;
  const bool simple = !a.bias && a.act == 0 && a.out == 0;
  if (a.bf16) {
    if (simple) hipLaunchKernelGGL((gemv_w4a16_kernel<NW, U, MR, CPL, true, true>), grid, dim3(NW * 64), lds, s, a.x, a.lda, a.Wp, a.ws, a.M, a.N, a.K, a);
    else hipLaunchKernelGGL((gemv_w4a16_kernel<NW, U, MR, CPL, true, false>), grid, dim3(NW * 64), lds, s, a.x, a.lda, a.Wp, a.ws, a.M, a.N, a.K, a);
  } else {
    if (simple) hipLaunchKernelGGL((gemv_w4a16_kernel<NW, U, MR, CPL, false, true>), grid, dim3(NW * 64), lds, s, a.x, a.lda, a.Wp, a.ws, a.M, a.N, a.K, a);
    else hipLaunchKernelGGL((gemv_w4a16_kernel<NW, U, MR, CPL, false, false>), grid, dim3(NW * 64), lds, s, a.x, a.lda, a.Wp, a.ws, a.M, a.N, a.K, a);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------- GEMM on INT8 MFMA
// Prefill chunks (M >= 2): the group dots on v_mfma_i32_16x16x64_i8. An aligned mantissa a
// (|a| <= 2^14) is split as a = 256 h + l with l its low byte sign-extended (in [-128, 127]) and
// h = (a - l) / 256 = (a + 128) >> 8 (in [-64, 64]); a weight w in [-8, 7] is taken as u = w + 8
// in [0, 15] (its nibble with the top bit flipped, no sign extension). Then over a 128-wide group
//   dot = sum a w = 256 sum h u + sum l u - 8 sum a,
// every sum exact in int32 (|sum h u| <= 2^17, |sum a| <= 2^21, |dot| <= 2^24), so the group's
// dot is the reference's exactly. The MFMA sums over 64 k: lane l supplies 16 bytes of operand
// row l % 16 and of weight row l % 16; with the weights' packed nibble order (byte b of the
// group's 64 bytes holds k = 2 b and 2 b + 1), one instruction takes the group's even k (the low
// nibbles) and a second its odd k (the high nibbles).
//
// The operand's 16 rows hold both halves: row i < MT is h of activation row i, row MT + i its l
// (MT = 8 fills the 16 rows; with MT = 4, rows 8-15 repeat rows 0-7). LDS holds them in the
// MFMA's order, [group][parity][lane quarter][row][16 bytes], so each operand is one ds_read_b128
// per lane. A group's two MFMAs leave sum h u and sum l u of every activation row in one
// accumulator (lane l: operand rows 4 (l / 16) .. + 3 against weight row l % 16); a permlane swap
// across the lane halves (MT = 8) or the 16-lane rows (MT = 4) brings each row's two sums to one
// lane, so every lane forms MT / 4 of the tile's MT x 16 terms and none idles.
//
// A workgroup owns MT activation rows (rows past M repeat row M - 1 and are never stored) and TT
// tiles of 16 weight rows; NW waves, NW / TT per tile, split the tile's groups. Phases:
//   1. the MT rows are loaded as MT * K / 8 tasks of 8 elements spread over every thread (a
//      16-lane unit is one group of one row);
//   2. they are aligned once (the group's exponent maximum by DPP; align_elems) into the LDS
//      operands: the int16 mantissas paired by byte permutes, h as byte 1 of each pair plus 128
//      (one packed 16-bit add), l as byte 0; each group's scale and 8 sum a beside them;
//   3. only then does each wave issue its weight loads (issued before, they held up the
//      alignment's instructions behind them);
//   4. after a barrier each wave runs its groups' MFMAs and forms the fp32 terms
//      (i2f(dot) * ws) * xs into LDS;
//   5. after a second barrier a lane per (row, weight row, bank) runs bank b's chain over groups
//      b, b + 4, ... in order from +0 (golden.py:315-319), and each quad folds
//      (b0 + b1) + (b2 + b3) before bias, activation and conversion.
//
// Roofline: HBM for the weights (K / 2 + K / 64 bytes per weight row), read once per MT rows; the
// alignment, the per-(row, group) fp32 terms and the chains are VALU work.
template <int MT, int TT, int NW, int GMAX, bool BF16, bool SIMPLE>
__global__ __launch_bounds__(NW * 64) void gemm_w4a16_mfma_kernel(const void* x, const uint8_t* Wp, const uint16_t* ws,
                                                                  int lda, int M, int N, int K, W4Args a) {
  constexpr int NT = NW * 64, WPT = NW / TT, GW = (GMAX + WPT - 1) / WPT;
  constexpr int R16 = 2 * MT, LGM = MT == 8 ? 3 : 2;
  constexpr int TR = (MT * GMAX * 16 + NT - 1) / NT;  // alignment rounds over MT * K / 8 tasks
  constexpr int TPL = MT / 4;                          // terms per lane and group
  static_assert(NW % TT == 0 && (MT == 4 || MT == 8), "waves split evenly over tiles");
  __shared__ __align__(16) int8_t aop[GMAX * 128 * R16];  // [g][parity][quarter][h rows, l rows][16 B]
  __shared__ __align__(16) int2 xs8[GMAX][MT];             // (scale encoding, 8 sum a)
  __shared__ float terms[TT][16][MT][GMAX + 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lq = lane >> 4;
  const int G = K >> 7, units = MT * G;
  const int m0 = blockIdx.y * MT;
  const int tile = wave % TT, part = wave / TT;
  const int nt0 = (blockIdx.x * TT + tile) * 16;
  const int gpw = (G + WPT - 1) / WPT, ga = part * gpw, gb = min(G, ga + gpw);

  // 1. the activation rows: thread t takes element block t % 16 of row (t / 16) % MT in every
  //    round, of group (t / 16) / MT + rd * GPR in round rd (each wave one group per round); a task
  //    past the last group reads it again (never stored); rows past M read the last row
  constexpr int GPR = NT / 16 / MT;  // groups per alignment round
  static_assert(GPR * 16 * MT == NT, "a thread keeps its row and block in every round");
  const int tq = tid & 15, r = (tid >> 4) & (MT - 1), g0 = tid >> (4 + LGM);
  const char* xrow = static_cast<const char*>(x) + static_cast<int64_t>(min(m0 + r, M - 1)) * lda;
  uint32_t xb[TR][8];
#pragma unroll
  for (int rd = 0; rd < TR; ++rd) {
    if (rd * NT >= units * 16) continue;  // uniform
    const int t = (min(g0 + rd * GPR, G - 1) << 4) | tq;
    if constexpr (BF16) {
      const v4u v = *reinterpret_cast<const v4u*>(xrow + 16 * t);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xb[rd][2 * j] = v[j] << 16;
        xb[rd][2 * j + 1] = v[j] & 0xFFFF0000u;
      }
    } else {
      const v4u* src = reinterpret_cast<const v4u*>(xrow + 32 * t);
      const v4u v0 = src[0], v1 = src[1];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xb[rd][j] = v0[j];
        xb[rd][4 + j] = v1[j];
      }
    }
  }
  issue_fence();

  // 2. alignment into the LDS operands: task (row r, group g, block tq) holds k = 8 tq .. 8 tq + 7:
  //    quarter q = tq / 4, even k at bytes 4 (tq % 4) .. + 3 of the even parity's 16, odd k likewise
  typedef uint16_t v2h __attribute__((ext_vector_type(2)));
  typedef short v2s __attribute__((ext_vector_type(2)));
  const auto add128 = [](uint32_t p) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2h, p) + (v2h){128, 128});
  };
  int8_t* const abase = aop + ((tq >> 2) * R16 + r) * 16 + 4 * (tq & 3);  // group 0, even parity, h
#pragma unroll
  for (int rd = 0; rd < TR; ++rd) {
    if (rd * NT + wave * 64 >= units * 16) continue;  // wave-uniform: a wave with no live task
    const int g = g0 + rd * GPR;
    int mant[8];
    uint32_t sb;
    align_elems<8, 16>(xb[rd], mant, sb);
    // int16 pairs: p[0] = (k0, k2), p[1] = (k4, k6), p[2] = (k1, k3), p[3] = (k5, k7)
    uint32_t p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = (j & 1) * 4 + (j >> 1);
      p[j] = __builtin_amdgcn_perm(static_cast<uint32_t>(mant[e + 2]), static_cast<uint32_t>(mant[e]), 0x05040100u);
    }
    int sum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) sum = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, p[j]), (v2s){1, 1}, sum, false);
    sum = group_sum<16>(sum);
    if (g < G) {
#pragma unroll
      for (int par = 0; par < 2; ++par) {
        const uint32_t lo = __builtin_amdgcn_perm(p[2 * par + 1], p[2 * par], 0x06040200u);
        const uint32_t hi = __builtin_amdgcn_perm(add128(p[2 * par + 1]), add128(p[2 * par]), 0x07050301u);
        int8_t* base = abase + (g * 2 + par) * 4 * R16 * 16;
        *reinterpret_cast<uint32_t*>(base) = hi;                // h: row r
        *reinterpret_cast<uint32_t*>(base + MT * 16) = lo;      // l: row MT + r
      }
      if (tq == 0) xs8[g][r] = make_int2(static_cast<int>(sb), 8 * sum);
    }
  }
  // 3. this wave's weights (row nt0 + l % 16, the 16 bytes of quarter l / 16 of each of its groups)
  //    and their fp16 scales; rows past N read the last row, groups past the wave's range group ga
  const int nr = min(nt0 + li, N - 1);
  const uint8_t* wrow = Wp + static_cast<int64_t>(nr) * (K >> 1) + 16 * lq;
  v4u wv[GW];
  uint32_t wsv[GW];
#pragma unroll
  for (int i = 0; i < GW; ++i) {
    const int g = min(ga + i < gb ? ga + i : ga, G - 1);
    wv[i] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(wrow + 64 * g));
    wsv[i] = ws[static_cast<int64_t>(nr) * G + g];
  }
  issue_fence();
  const KArg ka = kernarg_at(kW4MfmaArgsOffset);
  void* const Y = kload<void*>(ka + offsetof(W4Args, Y));
  const int64_t ldy = kload<int64_t>(ka + offsetof(W4Args, ldy));
  const float* const bias = SIMPLE ? nullptr : kload<const float*>(ka + offsetof(W4Args, bias));
  const int act = SIMPLE ? 0 : kload<int>(ka + offsetof(W4Args, act));
  const int out = SIMPLE ? 0 : kload<int>(ka + offsetof(W4Args, out));
  const float out_scale = SIMPLE ? 0.0f : kload<float>(ka + offsetof(W4Args, out_scale));

  __syncthreads();

  // 4. per group two MFMAs: accumulator row 4 (l / 16) + v of lane l is h (rows < MT) or l (rows
  //    MT ..) of an activation row, against weight row l % 16. After the swaps lane l holds the pair
  //    of activation row rows[j] in (hv[j], lv[j]): MT = 8: 4 (lq % 2) + lq / 2 + 2 j; MT = 4: lq.
  int rows[TPL];
  if constexpr (MT == 8) {
    rows[0] = 4 * (lq & 1) + (lq >> 1);
    rows[1] = rows[0] + 2;
  } else {
    rows[0] = lq;
  }
  const v4i zero = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < GW; ++i) {
    if (ga + i >= gb) break;  // uniform
    const int g = ga + i;
    const int8_t* base = aop + (((g * 2) * 4 + lq) * R16 + (li & (R16 - 1))) * 16;
    const v4i a0 = *reinterpret_cast<const v4i*>(base);
    const v4i a1 = *reinterpret_cast<const v4i*>(base + 4 * R16 * 16);
    v4i blo, bhi;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      blo[d] = static_cast<int>((wv[i][d] & 0x0F0F0F0Fu) ^ 0x08080808u);
      bhi[d] = static_cast<int>(((wv[i][d] >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u);
    }
    v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, blo, zero, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bhi, acc, 0, 0, 0);
    int dot[TPL];
    if constexpr (MT == 8) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const auto sw = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(acc[2 * j]),
                                                         static_cast<uint32_t>(acc[2 * j + 1]), false, false);
        dot[j] = static_cast<int>(sw[0]) * 256 + static_cast<int>(sw[1]);
      }
    } else {
      const auto s01 = __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(acc[0]), static_cast<uint32_t>(acc[1]),
                                                        false, false);
      const auto s23 = __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(acc[2]), static_cast<uint32_t>(acc[3]),
                                                        false, false);
      dot[0] = lq < 2 ? static_cast<int>(s01[0]) * 256 + static_cast<int>(s01[1])
                      : static_cast<int>(s23[0]) * 256 + static_cast<int>(s23[1]);
    }
    const float wsf = fp16_to_f32_keep_nan(wsv[i]);
#pragma unroll
    for (int j = 0; j < TPL; ++j) {
      const int2 e = xs8[g][rows[j]];
      // the contract's fmul(fmul(i2f(d), ws), xs) with its wrappers where they act (see the GEMV)
      terms[tile][li][rows[j]][g] = ftz(__fmul_rn(__fmul_rn(i2f(dot[j] - e.y), wsf), ffrom(static_cast<uint32_t>(e.x))));
    }
  }
  __syncthreads();

  // 5. chains: chain c = (tile, weight row, row, bank); the quad's four banks fold into bank 0
  constexpr int NCH = TT * 16 * MT * 4, CP = (NCH + NT - 1) / NT;
#pragma unroll
  for (int pc = 0; pc < CP; ++pc) {
    const int c = pc * NT + tid;
    if (pc * NT >= NCH) break;  // uniform
    const int cc = c < NCH ? c : 0;
    const int bank = cc & 3, o = cc >> 2;
    const int m = o % MT, n = (o / MT) % 16, tl = o / (MT * 16);
    float acc = 0.0f;
    for (int g = bank; g < G; g += 4) acc = fadd_chain(acc, terms[tl][n][m][g]);
    acc = chain_end(acc);
    const float pair = fadd(acc, lane_xor1(acc));
    const float other = lane_xor2(pair);
    const int ng = (blockIdx.x * TT + tl) * 16 + n, mg = m0 + m;
    if (c < NCH && bank == 0 && ng < N && mg < M) {
      float y = fadd(pair, other);
      const int64_t yrow = static_cast<int64_t>(mg) * ldy;
      if constexpr (SIMPLE) {
        reinterpret_cast<float*>(static_cast<char*>(Y) + yrow)[ng] = ftz(y);
      } else {
        if (bias) y = fadd(y, bias[ng]);
        y = act_fn(y, act);
        store_out(Y, yrow, ng, out, y, out_scale);
      }
    }
  }
}

template <int MT, int TT, int NW, int GMAX>
hipError_t go_w4_mfma(const W4Args& a, hipStream_t s) {
  const dim3 grid((a.N + 16 * TT - 1) / (16 * TT), (a.M + MT - 1) / MT), block(NW * 64);
  const bool simple = !a.bias && a.act == 0 && a.out == 0;
  const int lda = static_cast<int>(a.lda);
#define TARS_W4M(BF, SI)                                                                                          \
  hipLaunchKernelGGL((gemm_w4a16_mfma_kernel<MT, TT, NW, GMAX, BF, SI>), grid, block, 0, s, a.x, a.Wp, a.ws, lda, \
                     a.M, a.N, a.K, a)
  if (a.bf16) {
    if (simple) TARS_W4M(true, true);
    else TARS_W4M(true, false);
  } else {
    if (simple) TARS_W4M(false, true);
    else TARS_W4M(false, false);
  }
#undef TARS_W4M
  return hipGetLastError();
}

}  // namespace

hipError_t launch_align_w4(const AlignArgs& a, hipStream_t s) {
  const int C = a.K / 32;
  const dim3 grid((C + kThreads - 1) / kThreads, a.M);
  hipLaunchKernelGGL(align_w4_kernel, grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

template <int NW, int U, int MR>
hipError_t go_cpl(const W4Args& a, int cpl, hipStream_t s) {
  switch (cpl) {
    case 1: return go_w4<NW, U, MR, 1>(a, s);
    case 2: return go_w4<NW, U, MR, 2>(a, s);
    case 3: return go_w4<NW, U, MR, 3>(a, s);
    default: return go_w4<NW, U, MR, 4>(a, s);
  }
}

// Shapes by measurement on MI355X (weights cold, graph replays). One activation row: rows of at
// most 2048 k (one chunk per lane) 4 rows per wave in 4-wave workgroups (K = 1536, N = 12288:
// 4.0 us; 2-, 3-, 6- and 8-wave workgroups and 1 to 3 rows per wave 0.1 - 3 us slower). Longer
// rows (swept over K = 2304 - 8192 and N = 512 - 12288): the fewest weight rows per workgroup (4,
// 8, 12, 16 in 4-wave workgroups; 24, 32 in 8-wave ones) that keep the grid at most 256
// workgroups, 4 only up to 3072 k, and 24 rows past N = 8192; at N <= 1024 past 6144 k the
// K-split form below. Against one row per wave in 8-wave workgroups and the K-split form from
// N = 4096: K = 6144: N = 1536 / 2048 / 3072 / 4096 / 6144 / 8192 / 12288: 3.44 / 3.67 / 5.00 /
// 4.97 / 6.59 / 7.38 / 10.53 -> 3.25 / 3.38 / 4.00 / 4.50 / 5.71 / 6.64 / 8.79 us; K = 2304,
// N = 3072: 3.82 -> 2.96 us; K = 8192, N = 2048 / 4096: 4.33 / 6.37 -> 3.97 / 6.01 us (K = 8192,
// N = 1024: K split 3.75 us, 8 rows per workgroup 3.84 us).
// Several rows (swept over M = 2 - 32 and 15 (K, N) pairs from 512 x 4096 to 8192 x 4096; every
// form bit-exact):
//   * the per-lane form, two activation rows per workgroup in 8-wave workgroups, with the fewest
//     rows per wave (1, 2; 3 from 1536 to 6144 k; 4 from 1536 to 4096 k; 3 and 4 at any K at
//     M = 2) that keep the grid at most 256 workgroups, up to 8 rows: K = 6144, N = 1536: M = 2 /
//     4 / 8: 4.4 / 5.3 / 6.2 us; K = 3072, N = 1024: M = 2 - 8: 3.3 - 4.0 us; K = 2048, N = 2048:
//     M = 2 - 8: 2.8 - 3.6 us (three rows per wave: K = 6144, N = 3072, M = 4: 7.1 -> 6.5 us;
//     K = 4096, N = 1536, M = 7: 5.2 -> 4.7 us; past 6144 k it lost to the MFMA form: K = 8192,
//     N = 1536, M = 8: 8.2 against 7.9 us); at M = 2 it is always the per-lane form (the 4-row
//     waves of 4-wave workgroups past those grids: K = 1536, N = 12288: 5.1 us);
//   * otherwise the MFMA form. Up to 2048 k: M <= 4 on 4-row tiles, 4 waves above N = 8192 (K =
//     1536, N = 12288: 5.7 us) and 8 below (K = 1024, N = 3072: 3.3 us; K = 2048, N = 8192: 5.2
//     us); more rows on 8-row tiles, 8 waves per weight tile while the grid stays at most 256
//     workgroups (K = 1536, N = 3072: M = 8 4.3 us), else two weight tiles of 16 waves while that
//     holds (M = 16: 4.4 us; K = 2048, N = 8192, M = 8: 5.6 us), else 8 waves per tile with one,
//     two or four tiles per workgroup, the fewest that keep the grid at most 768 workgroups (K =
//     1536, N = 12288: M = 8 / 16 / 32: 6.7 / 9.9 / 16.6 us); with at most 128 workgroups of 8-row
//     tiles, 4-row tiles (twice the workgroups; K = 1024, N = 1024, M = 16: 3.2 against 3.7 us).
//     Past 2048 k, 16 waves per workgroup and the tile shape (4 rows; 8 rows; 8 rows and two
//     weight tiles) with the largest grid of at most 256 workgroups: K = 6144, N = 1536: M = 8 /
//     16 / 32: 6.6 / 7.8 / 11.6 us; K = 3072, N = 4096: M = 8 / 16: 6.0 / 8.5 us.
// The 8-row tiles with the two halves of the mantissa in the operand rows replaced tiles that
// took them in separate MFMAs (4 rows per tile and masked operand rows): K = 1536, N = 12288:
// M = 4 / 8 / 16 / 32: 6.3 / 9.1 / 12.5 / 22.1 -> 5.7 / 6.7 / 9.9 / 16.6 us.
hipError_t launch_gemv_w4a16(const W4Args& a, hipStream_t s) {
  const int cpl = (a.K / 32 + 63) / 64;  // chunks per lane
  const int G = a.K / 128;
  const int64_t n16 = (a.N + 15) / 16;
  if (a.M >= 2 && a.M <= 8) {
    const int64_t mb = (a.M + 1) / 2;
    auto wgs = [&](int u) { return static_cast<int64_t>((a.N + 8 * u - 1) / (8 * u)) * mb; };
    if (wgs(1) <= 256) return go_cpl<8, 1, 2>(a, cpl, s);
    if (wgs(2) <= 256) return go_cpl<8, 2, 2>(a, cpl, s);
    if ((a.M == 2 || a.K >= 1536) && a.K <= 6144 && wgs(3) <= 256) return go_cpl<8, 3, 2>(a, cpl, s);
    if ((a.M == 2 || (a.K >= 1536 && a.K <= 4096)) && wgs(4) <= 256) return go_cpl<8, 4, 2>(a, cpl, s);
  }
  if (a.M >= 3 && a.lda <= INT32_MAX) {
    const int64_t mb4 = (a.M + 3) / 4, mb8 = (a.M + 7) / 8;
    if (G <= 16) {
      if (a.M <= 4) return a.N > 8192 ? go_w4_mfma<4, 1, 4, 16>(a, s) : go_w4_mfma<4, 1, 8, 16>(a, s);
      if (n16 * mb8 <= 128) return go_w4_mfma<4, 1, 8, 16>(a, s);
      if (n16 * mb8 <= 256) return go_w4_mfma<8, 1, 8, 16>(a, s);
      if ((n16 + 1) / 2 * mb8 <= 256) return go_w4_mfma<8, 2, 16, 16>(a, s);
      if (n16 * mb8 <= 768) return go_w4_mfma<8, 1, 8, 16>(a, s);
      if ((n16 + 1) / 2 * mb8 <= 768) return go_w4_mfma<8, 2, 8, 16>(a, s);
      return go_w4_mfma<8, 4, 8, 16>(a, s);
    }
    if (G <= 48) {
      if (n16 * mb4 <= 256) return go_w4_mfma<4, 1, 16, 48>(a, s);
      if (n16 * mb8 <= 256) return go_w4_mfma<8, 1, 16, 48>(a, s);
      return go_w4_mfma<8, 2, 16, 48>(a, s);
    }
    return go_w4_mfma<4, 1, 16, 64>(a, s);
  }
  if (a.M >= 2) return go_cpl<4, 4, 2>(a, cpl, s);
  if (cpl == 1) return go_cpl<4, 4, 1>(a, cpl, s);
  if (a.N <= 1024) {
    if (a.K > 6144) return go_w4_kslice<1>(a, s);
    if (a.K <= 3072) return go_cpl<4, 1, 1>(a, cpl, s);
  }
  if (a.N <= 2048) return go_cpl<4, 2, 1>(a, cpl, s);
  if (a.N <= 3072) return go_cpl<4, 3, 1>(a, cpl, s);
  if (a.N <= 4096) return go_cpl<4, 4, 1>(a, cpl, s);
  if (a.N <= 8192 && a.N > 6144) return go_cpl<8, 4, 1>(a, cpl, s);
  return go_cpl<8, 3, 1>(a, cpl, s);
}

}  // namespace tars
