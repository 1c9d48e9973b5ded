// W4A16: block-FP activation alignment (tars_mini/numerics.py:55-98) and the group-128 GEMV
// (tars_mini/golden.py:295-324).
//
// Work unit: a 16-byte chunk of a packed weight row = 32 int4 weights = a quarter of a 128-wide
// group. Thread c of a row owns chunk c (so a row of K/2 bytes is read by K/32 consecutive
// threads, fully coalesced), and the four threads of a group are four consecutive lanes.
//
// Alignment is fused into the GEMV prologue: the workgroup aligns its activation row once,
// cooperatively (8 lanes per 128-wide group, 16 elements each; the group's exponent maximum meets
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
// The per-group fp32 terms (i2f(dot) * ws) * xs go to LDS; four threads per row then run the four
// bank chains (group g goes to bank g % 4, added in g order from +0) and combine
// (b0 + b1) + (b2 + b3) before bias, activation and conversion.
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
// U: rows each thread streams. R = 256 / C rows share a workgroup pass (C = K / 32 chunks per row).
//
// 1. Each thread issues its weight loads (U rows x 16 bytes) first.
// 2. The workgroup aligns activation row m once, cooperatively: 8 consecutive lanes own one
//    128-wide group (16 elements each), meet their exponent maximum and NaN/inf flags in an 8-lane
//    DPP reduction, and write the split signed byte planes of their mantissas to LDS in the layout
//    the dot product reads (per 32-element chunk: lo_even, lo_odd, hi_even, hi_odd, 4 dwords each),
//    plus the group scale.
// 3. Each thread reads its chunk's 64 bytes, forms the exact dots, the four lanes of a group add
//    theirs (quad permutes), the group leader writes the fp32 term to LDS, and four threads per row
//    run the bank chains.
template <int U, bool BF16>
__global__ __launch_bounds__(kThreads) void gemv_w4a16_kernel(W4Args a) {
  extern __shared__ __align__(16) uint32_t act_lds[];  // C * 16 dwords of byte planes, then G scales
  __shared__ float terms[64][65];
  const int C = a.K / 32;
  const int G = a.K / kGroup;
  const int R = kThreads / C;
  const int rows_per_block = R * U;
  const int m = blockIdx.y;
  const int tid = threadIdx.x;
  const int r = tid / C;
  const int c = tid - r * C;
  const bool live = r < R;
  const int cc = live ? c : 0;
  const int g = cc >> 2;

  const int nbase = blockIdx.x * rows_per_block;
  const size_t row_bytes = static_cast<size_t>(a.K / 2);

  // Issue order matters: vmcnt counts loads in order, so the activation loads go first (the
  // alignment waits on them alone), then the weights, then the group scales the epilogue needs.
  // Lane i of the 8 * G alignment lanes owns elements [16 i, 16 i + 16) of row m; K <= 8192 means
  // at most two passes of 256 lanes.
  const char* xrow = static_cast<const char*>(a.x) + m * a.lda;
  const int npass = (8 * G + kThreads - 1) / kThreads;
  uint32_t xb[2][16];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    // pass 1 exists only for K > 4096; when it does not, its loads read shadow data (always
    // issued, never branched around: see load_pred) and the results are never used
    const int i = p * kThreads + tid;
    const int ii = i < 8 * G ? i : (i & 7);  // dead lanes shadow group 0 (whole 8-lane groups)
    if constexpr (BF16) {
      const v4u* src = reinterpret_cast<const v4u*>(xrow + 32 * ii);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const v4u v = src[q];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          xb[p][8 * q + 2 * j] = v[j] << 16;
          xb[p][8 * q + 2 * j + 1] = v[j] & 0xFFFF0000u;
        }
      }
    } else {
      const v4u* src = reinterpret_cast<const v4u*>(xrow + 64 * ii);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const v4u v = src[q];
#pragma unroll
        for (int j = 0; j < 4; ++j) xb[p][4 * q + j] = v[j];
      }
    }
  }
  issue_fence();
  v4u wv[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int n = nbase + u * R + r;
    wv[u] = load_stream_pred(reinterpret_cast<const v4u*>(a.Wp + n * row_bytes) + cc,
                             reinterpret_cast<const v4u*>(a.Wp), live && n < a.N, v4u{0u, 0u, 0u, 0u});
  }
  issue_fence();
  uint32_t wsb[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int n = min(nbase + u * R + r, a.N - 1);
    wsb[u] = a.ws[static_cast<size_t>(n) * G + g];
  }
  // this thread's epilogue row (four threads per row run the bank chains) and its bias, fetched
  // unconditionally from a valid address
  const int slot = tid >> 2;
  const int bank = tid & 3;
  const bool has_row = slot < rows_per_block;
  const int slot_c = has_row ? slot : 0;
  const int ue = slot_c / R, re = slot_c - ue * R;
  const int ne = nbase + ue * R + re;
  const float bias_v = *(a.bias ? a.bias + min(ne, a.N - 1) : reinterpret_cast<const float*>(a.ws));
  issue_fence();

  // cooperative alignment of row m into LDS byte planes
  float* xs_lds = reinterpret_cast<float*>(act_lds + C * 16);
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    if (p < npass) {
      const int i = p * kThreads + tid;
      const bool valid = i < 8 * G;
      const int ii = valid ? i : (i & 7);
      int mant[16];
      uint32_t sb;
      align_elems<16, 8>(xb[p], mant, sb);
      if (valid) {
        int lo[16], hi[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          lo[j] = static_cast<int8_t>(mant[j] & 0xFF);
          hi[j] = (mant[j] - lo[j]) >> 8;
        }
        const int chunk = ii >> 1, half = ii & 1;
        uint32_t* dst = act_lds + chunk * 16 + 2 * half;
#pragma unroll
        for (int d = 0; d < 2; ++d) {
          dst[0 + d] = pack4(lo[8 * d], lo[8 * d + 2], lo[8 * d + 4], lo[8 * d + 6]);
          dst[4 + d] = pack4(lo[8 * d + 1], lo[8 * d + 3], lo[8 * d + 5], lo[8 * d + 7]);
          dst[8 + d] = pack4(hi[8 * d], hi[8 * d + 2], hi[8 * d + 4], hi[8 * d + 6]);
          dst[12 + d] = pack4(hi[8 * d + 1], hi[8 * d + 3], hi[8 * d + 5], hi[8 * d + 7]);
        }
        if ((ii & 7) == 0) xs_lds[ii >> 3] = ffrom(sb);
      }
    }
  }
  __syncthreads();

  ActBytes act;
  {
    const v4u* src = reinterpret_cast<const v4u*>(act_lds + cc * 16);
    const v4u le = src[0], lo = src[1], he = src[2], ho = src[3];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      act.lo_even[d] = le[d];
      act.lo_odd[d] = lo[d];
      act.hi_even[d] = he[d];
      act.hi_odd[d] = ho[d];
    }
  }
  const float xs = xs_lds[g];

#pragma unroll
  for (int u = 0; u < U; ++u) {
    int d16 = chunk_dot16(wv[u], act);
    d16 += lane_xor1(d16);
    d16 += lane_xor2(d16);
    const int n = nbase + u * R + r;
    if (live && (cc & 3) == 0 && n < a.N) {
      terms[u * R + r][g] = fmul(fmul(i2f(d16 >> 4), from_fp16_bits(wsb[u])), xs);
    }
  }
  __syncthreads();

  // four bank chains per row, then (b0 + b1) + (b2 + b3)
  float acc = 0.0f;
  for (int gg = bank; gg < G; gg += 4) acc = fadd(acc, terms[slot_c][gg]);
  const float pair = fadd(acc, lane_xor1(acc));  // bank 0: b0 + b1, bank 2: b2 + b3
  const float other = lane_xor2(pair);
  if (has_row && bank == 0 && ne < a.N) {
    float y = fadd(pair, other);
    if (a.bias) y = fadd(y, bias_v);
    y = act_fn(y, a.act);
    store_out(a.Y, m * a.ldy, ne, a.out, y, a.out_scale);
  }
}

template <int U>
hipError_t go_w4(const W4Args& a, hipStream_t s) {
  const int C = a.K / 32;
  const int R = kThreads / C;
  const int rows = R * U;
  const dim3 grid((a.N + rows - 1) / rows, a.M);
  const size_t lds = static_cast<size_t>(C) * 64 + static_cast<size_t>(a.K / kGroup) * 4;
  if (a.bf16) {
    hipLaunchKernelGGL((gemv_w4a16_kernel<U, true>), grid, dim3(kThreads), lds, s, a);
  } else {
    hipLaunchKernelGGL((gemv_w4a16_kernel<U, false>), grid, dim3(kThreads), lds, s, a);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_align_w4(const AlignArgs& a, hipStream_t s) {
  const int C = a.K / 32;
  const dim3 grid((C + kThreads - 1) / kThreads, a.M);
  hipLaunchKernelGGL(align_w4_kernel, grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_gemv_w4a16(const W4Args& a, hipStream_t s) {
  // Rows per block R * U must not exceed the 64 LDS term rows. Long rows (R <= 2, K >= 4096)
  // take 8 rows per thread so the activation row is read and aligned once per 8 * R weight rows;
  // shorter rows take 4, which keeps >= 600 workgroups at N = 12288 (measured on MI355X:
  // K=6144 N=1536 8.0 us at U=8 vs 10.2 at U=4; K=1536 N=12288 8.7 us at U=4 vs 9.3 at U=8).
  const int R = kThreads / (a.K / 32);
  if (R <= 2) return go_w4<8>(a, s);
  if (R * 4 <= 64) return go_w4<4>(a, s);
  if (R * 2 <= 64) return go_w4<2>(a, s);
  return go_w4<1>(a, s);
}

}  // namespace tars
