// W4A16: block-FP activation alignment (tars_mini/numerics.py:55-98) and the group-128 GEMV
// (tars_mini/golden.py:295-324).
//
// Work unit: a 16-byte chunk of a packed weight row = 32 int4 weights = a quarter of a 128-wide
// group. A wave owns whole rows; lane l streams chunks l, l + 64, ... of each (every load
// instruction reads 1 KiB of a row, fully coalesced), so a group's four chunks sit on four
// consecutive lanes.
//
// Alignment is fused into the GEMV prologue: the workgroup aligns its activation row once,
// cooperatively (16 lanes per 128-wide group, 8 elements each; the group's exponent maximum meets
// through DPP lane permutes), into LDS byte planes that every weight row of the workgroup reads.
// Each mantissa (an int16 in [-16384, 16384]) is rounded to nearest-even exactly as the reference
// does: for finite groups as rint(x * 2^(140 - e_eff)), otherwise by the integer shift rule with
// the NaN / infinity cases.
//
// Exact int16 x int4 dots on v_dot4 (signed 8-bit): a mantissa a is split as a = 256 * ah + al with
// al, ah signed bytes (al = the low byte read as signed, ah in [-64, 64]); a weight nibble w is
// used as the byte w * 16 (the nibble moved to the byte's top, which sign-extends it). Then
// 16 * sum(w * a) = 256 * dot4(w16, ah) + dot4(w16, al), exact in int32 (|.| <= 2^28), and the
// final arithmetic shift by 4 is exact. The packed byte holds the even k in its low nibble and the
// odd k in its high nibble, so the activations are kept as even/odd byte lanes.
//
// The per-group fp32 terms (i2f(dot) * ws) * xs go to the wave's own LDS rows; four lanes per
// row then run the four bank chains (group g goes to bank g % 4, added in g order from +0) and
// combine (b0 + b1) + (b2 + b3) before bias, activation and conversion. The only workgroup
// barrier is the one after the alignment.
//
// Roofline: HBM. Algorithmic bytes per row: K/2 (weights) + K/64 (fp16 scales) + 4 (output).
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
// fp32 encodings (not flushed). Outputs the signed mantissas and the group's fp32 scale encoding.
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
    const float p = __uint_as_float(static_cast<uint32_t>(267 - e_eff) << 23);
#pragma unroll
    for (int i = 0; i < NE; ++i) mant[i] = static_cast<int>(__builtin_rintf(__uint_as_float(xraw[i]) * p));
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

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
  return (static_cast<uint32_t>(a) & 0xFFu) | ((static_cast<uint32_t>(b) & 0xFFu) << 8) |
         ((static_cast<uint32_t>(c) & 0xFFu) << 16) | ((static_cast<uint32_t>(d) & 0xFFu) << 24);
}

// Splits 32 mantissas into the byte lanes the nibble layout needs: for weight dword d (k = 8d..8d+7
// of the chunk), even k pair with the low nibbles and odd k with the high nibbles.
struct ActBytes {
  uint32_t lo_even[4], lo_odd[4], hi_even[4], hi_odd[4];
};

__device__ __forceinline__ ActBytes split_bytes(const int mant[32]) {
  ActBytes r;
  int lo[32], hi[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    lo[i] = static_cast<int8_t>(mant[i] & 0xFF);
    hi[i] = (mant[i] - lo[i]) >> 8;
  }
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    r.lo_even[d] = pack4(lo[8 * d], lo[8 * d + 2], lo[8 * d + 4], lo[8 * d + 6]);
    r.lo_odd[d] = pack4(lo[8 * d + 1], lo[8 * d + 3], lo[8 * d + 5], lo[8 * d + 7]);
    r.hi_even[d] = pack4(hi[8 * d], hi[8 * d + 2], hi[8 * d + 4], hi[8 * d + 6]);
    r.hi_odd[d] = pack4(hi[8 * d + 1], hi[8 * d + 3], hi[8 * d + 5], hi[8 * d + 7]);
  }
  return r;
}

// 16 * (exact dot of the chunk's 32 weights with its 32 mantissas)
__device__ __forceinline__ int chunk_dot16(v4u w, const ActBytes& x) {
  int lo = 0, hi = 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const int we = static_cast<int>((w[d] << 4) & 0xF0F0F0F0u);
    const int wo = static_cast<int>(w[d] & 0xF0F0F0F0u);
    lo = __builtin_amdgcn_sdot4(we, static_cast<int>(x.lo_even[d]), lo, false);
    lo = __builtin_amdgcn_sdot4(wo, static_cast<int>(x.lo_odd[d]), lo, false);
    hi = __builtin_amdgcn_sdot4(we, static_cast<int>(x.hi_even[d]), hi, false);
    hi = __builtin_amdgcn_sdot4(wo, static_cast<int>(x.hi_odd[d]), hi, false);
  }
  return hi * 256 + lo;
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
// One wave owns U whole weight rows: lane l streams chunks l, l + 64, ... (CPL per lane) of each
// row, so a group's four chunks sit on four consecutive lanes and everything after the activation
// alignment (the group sums, the terms and the four bank chains) stays inside the wave.
//
// 1. Loads are issued activations first (the aligner waits on them alone), then the U * CPL weight
//    chunks, then the group scales and the bias.
// 2. The workgroup aligns activation row m once: aligner thread t (t < K / 8, CPL passes of 256)
//    owns elements [8 t, 8 t + 8), 16 consecutive threads form one 128-wide group and meet their
//    exponent maximum and flags by DPP. The split signed bytes go to LDS plane-major (plane q =
//    lo_even, lo_odd, hi_even, hi_odd; dword t of each plane), the group scale beside them.
// 3. After the one workgroup barrier each lane reads its chunks' 64 bytes, forms the exact dots,
//    adds its group's four lanes (quad permutes), and the group's first lane writes the fp32 term
//    (i2f(dot) * ws) * xs into the wave's own LDS rows.
// 4. Lane 4 u + b runs bank b's chain of row u (groups b, b + 4, ... in order from +0, every term
//    read up front so only the fadds are sequential), and the quad folds (b0 + b1) + (b2 + b3).
constexpr int kWaves = kThreads / 64;
constexpr int kTermStride = 65;  // LDS floats per term row (G <= 64), padded against bank conflicts

template <int CPL, int U, bool BF16, bool SIMPLE>
__global__ __launch_bounds__(kThreads) void gemv_w4a16_kernel(W4Args a) {
  static_assert(CPL >= 1 && CPL <= 4 && U >= 1 && 4 * U <= 64, "K <= 8192; one chain quad per row");
  extern __shared__ __align__(16) uint32_t planes[];  // 4 planes of 4C dwords, then G scale encodings
  __shared__ float terms[kWaves][U][kTermStride];
  const int C = a.K >> 5;
  const int G = a.K >> 7;
  const int A = a.K >> 3;  // aligner threads (8 elements each)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int m = blockIdx.y;
  const int n0 = (blockIdx.x * kWaves + wave) * U;
  const int64_t row_bytes = a.K >> 1;
  const char* xrow = static_cast<const char*>(a.x) + m * a.lda;

  // 1. activations (dead aligner threads shadow the first group's lanes: whole 16-lane groups)
  uint32_t xb[CPL][8];
#pragma unroll
  for (int p = 0; p < CPL; ++p) {
    const int t = p * kThreads + tid;
    const int tt = t < A ? t : (t & 15);
    if constexpr (BF16) {
      const v4u v = *reinterpret_cast<const v4u*>(xrow + 16 * tt);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xb[p][2 * j] = v[j] << 16;
        xb[p][2 * j + 1] = v[j] & 0xFFFF0000u;
      }
    } else {
      const v4u* src = reinterpret_cast<const v4u*>(xrow + 32 * tt);
      const v4u v0 = src[0], v1 = src[1];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xb[p][j] = v0[j];
        xb[p][4 + j] = v1[j];
      }
    }
  }
  issue_fence();
  v4u wv[U][CPL];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int n = n0 + u;
    const v4u* wrow = reinterpret_cast<const v4u*>(a.Wp + n * row_bytes);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      wv[u][j] = load_stream_pred(wrow + c, reinterpret_cast<const v4u*>(a.Wp), n < a.N && c < C,
                                  v4u{0u, 0u, 0u, 0u});
    }
  }
  issue_fence();
  uint32_t wsb[U][CPL];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int n = min(n0 + u, a.N - 1);
#pragma unroll
    for (int j = 0; j < CPL; ++j) wsb[u][j] = a.ws[static_cast<int64_t>(n) * G + min((lane + 64 * j) >> 2, G - 1)];
  }
  const int ue = lane >> 2, bank = lane & 3;  // this lane's chain: bank `bank` of row n0 + ue
  const int ne = n0 + (ue < U ? ue : 0);
  const float bias_v = *(a.bias ? a.bias + min(ne, a.N - 1) : reinterpret_cast<const float*>(a.ws));
  issue_fence();

  // 2. cooperative alignment into the LDS planes
  float* xs_lds = reinterpret_cast<float*>(planes + 16 * C);
#pragma unroll
  for (int p = 0; p < CPL; ++p) {
    const int t = p * kThreads + tid;
    int mant[8];
    uint32_t sb;
    align_elems<8, 16>(xb[p], mant, sb);
    if (t < A) {
      int lo[8], hi[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        lo[j] = static_cast<int8_t>(mant[j] & 0xFF);
        hi[j] = (mant[j] - lo[j]) >> 8;
      }
      planes[t] = pack4(lo[0], lo[2], lo[4], lo[6]);
      planes[4 * C + t] = pack4(lo[1], lo[3], lo[5], lo[7]);
      planes[8 * C + t] = pack4(hi[0], hi[2], hi[4], hi[6]);
      planes[12 * C + t] = pack4(hi[1], hi[3], hi[5], hi[7]);
      if ((t & 15) == 0) xs_lds[t >> 4] = ffrom(sb);
    }
  }
  __syncthreads();

  // 3. dots and group terms
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    const int cc = c < C ? c : 0;
    ActBytes act;
    const v4u le = *reinterpret_cast<const v4u*>(planes + 4 * cc);
    const v4u lo = *reinterpret_cast<const v4u*>(planes + 4 * C + 4 * cc);
    const v4u he = *reinterpret_cast<const v4u*>(planes + 8 * C + 4 * cc);
    const v4u ho = *reinterpret_cast<const v4u*>(planes + 12 * C + 4 * cc);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      act.lo_even[d] = le[d];
      act.lo_odd[d] = lo[d];
      act.hi_even[d] = he[d];
      act.hi_odd[d] = ho[d];
    }
    const float xs = xs_lds[cc >> 2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int d16 = chunk_dot16(wv[u][j], act);
      d16 += lane_xor1(d16);
      d16 += lane_xor2(d16);
      if ((lane & 3) == 0 && c < C && n0 + u < a.N)
        terms[wave][u][c >> 2] = fmul(fmul(i2f(d16 >> 4), from_fp16_bits(wsb[u][j])), xs);
    }
  }
  // the terms were written by other lanes of this wave: order the LDS accesses (no block barrier)
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // 4. four bank chains per row (at most G / 4 <= K / 512 <= 4 CPL steps; the terms are flushed
  //    fmul results, so the steps are fadd_chain's, run unflushed and checked: recomputed with the
  //    flushes when a partial sum is subnormal), then (b0 + b1) + (b2 + b3)
  constexpr int kSteps = 4 * CPL;
  const float* trow = terms[wave][ue < U ? ue : 0];
  float tv[kSteps];
#pragma unroll
  for (int i = 0; i < kSteps; ++i) tv[i] = trow[bank + 4 * i];  // index <= 16 CPL - 1 < kTermStride
  float acc = 0.0f;
  uint32_t mk = ~0u;
#pragma unroll
  for (int i = 0; i < kSteps; ++i)
    if (bank + 4 * i < G) {
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
  const float pair = fadd(acc, lane_xor1(acc));  // bank 0: b0 + b1, bank 2: b2 + b3
  const float other = lane_xor2(pair);
  if (bank == 0 && ue < U && n0 + ue < a.N) {
    float y = fadd(pair, other);
    if constexpr (SIMPLE) {
      reinterpret_cast<float*>(static_cast<char*>(a.Y) + m * a.ldy)[n0 + ue] = ftz(y);
    } else {
      if (a.bias) y = fadd(y, bias_v);
      y = act_fn(y, a.act);
      store_out(a.Y, m * a.ldy, n0 + ue, a.out, y, a.out_scale);
    }
  }
}

template <int CPL, int U>
hipError_t go_w4(const W4Args& a, hipStream_t s) {
  const dim3 grid((a.N + kWaves * U - 1) / (kWaves * U), a.M);
  const size_t lds = static_cast<size_t>(a.K / 32) * 64 + static_cast<size_t>(a.K / kGroup) * 4;
  // fp32 output with neither bias nor activation: the epilogue's general code compiled out
  const bool simple = !a.bias && a.act == 0 && a.out == 0;
  if (a.bf16) {
    if (simple) hipLaunchKernelGGL((gemv_w4a16_kernel<CPL, U, true, true>), grid, dim3(kThreads), lds, s, a);
    else hipLaunchKernelGGL((gemv_w4a16_kernel<CPL, U, true, false>), grid, dim3(kThreads), lds, s, a);
  } else {
    if (simple) hipLaunchKernelGGL((gemv_w4a16_kernel<CPL, U, false, true>), grid, dim3(kThreads), lds, s, a);
    else hipLaunchKernelGGL((gemv_w4a16_kernel<CPL, U, false, false>), grid, dim3(kThreads), lds, s, a);
  }
  return hipGetLastError();
}

template <int CPL>
hipError_t go_w4_rows(const W4Args& a, int u, hipStream_t s) {
  switch (u) {
    case 1: return go_w4<CPL, 1>(a, s);
    case 2: return go_w4<CPL, 2>(a, s);
    case 4: return go_w4<CPL, 4>(a, s);
    default: return go_w4<CPL, 8>(a, s);
  }
}

}  // namespace

hipError_t launch_align_w4(const AlignArgs& a, hipStream_t s) {
  const int C = a.K / 32;
  const dim3 grid((C + kThreads - 1) / kThreads, a.M);
  hipLaunchKernelGGL(align_w4_kernel, grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

// Rows per wave: every workgroup aligns the whole activation row, so U trades that repeated work
// (workgroups x K elements) against workgroups in flight: the smallest U in {1, 2, 4, 8} that keeps
// the repeated alignment within 1.5M elements. Measured on MI355X: K = 1536, N = 12288 6.59 us at
// U = 4 (7.01 at U = 2, 7.55 at U = 8); K = 6144, N = 1536 5.53 us at U = 2 (5.81 at U = 1, 7.51
// at U = 4).
static int w4_rows_per_wave(int64_t N, int K) {
  int u = 1;
  while (u < 8 && (N + kWaves * u - 1) / (kWaves * u) * K > 3 * (1 << 19)) u *= 2;
  return u;
}

hipError_t launch_gemv_w4a16(const W4Args& a, hipStream_t s) {
  const int u = w4_rows_per_wave(a.N, a.K);
  switch ((a.K / 32 + 63) / 64) {  // chunks per lane
    case 1: return go_w4_rows<1>(a, u, s);
    case 2: return go_w4_rows<2>(a, u, s);
    case 3: return go_w4_rows<3>(a, u, s);
    default: return go_w4_rows<4>(a, u, s);
  }
}

}  // namespace tars
