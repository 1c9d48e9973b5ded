// W4A16: block-FP activation alignment (tars_mini/numerics.py:55-98) and the group-128 GEMV
// (tars_mini/golden.py:295-324).
//
// Work unit: a 16-byte chunk of a packed weight row = 32 int4 weights = a quarter of a 128-wide
// group. Thread c of a row owns chunk c (so a row of K/2 bytes is read by K/32 consecutive
// threads, fully coalesced), and the four threads of a group are four consecutive lanes.
//
// Alignment is fused into the GEMV prologue: each thread aligns the 32 activations of its chunk;
// the group's exponent maximum and NaN/inf flags meet through two quad lane permutes; each mantissa
// (an int16 in [-16384, 16384]) is rounded to nearest-even exactly as the reference does.
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
  for (int i = 0; i < 32; ++i)
    if ((xb[i] & kExpo) == 0) xb[i] &= kSign;  // ftz
}

// Aligns one chunk within its group of 4 consecutive lanes (every lane of the wave must call it).
// Outputs the signed mantissas and the group's fp32 scale encoding.
__device__ __forceinline__ void align_chunk(const uint32_t xb[32], int mant[32], uint32_t& scale_bits) {
  int emax = 0, flags = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const int e = (xb[i] >> 23) & 0xFF;
    emax = max(emax, e);
    if (e == 255) flags |= (xb[i] & kMant) ? 1 : 2;
  }
  emax = max(emax, lane_xor1(emax));
  emax = max(emax, lane_xor2(emax));
  flags |= lane_xor1(flags);
  flags |= lane_xor2(flags);
  const bool grp_nan = flags & 1;
  const bool grp_inf = (flags & 2) && !grp_nan;
  const int e_eff = max(emax, 14);
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const uint32_t b = xb[i];
    const int e = (b >> 23) & 0xFF;
    const uint32_t frac = b & kMant;
    const int sh = 10 + e_eff - e;  // >= 10
    int mag = 0;
    if (e != 0 && e != 255 && sh < 25) {
      const uint32_t sig = frac | (1u << 23);
      const uint32_t kept = sig >> sh;
      const uint32_t dropped = sig & ((1u << sh) - 1u);
      const uint32_t half = 1u << (sh - 1);
      mag = static_cast<int>(kept + ((dropped > half || (dropped == half && (kept & 1u))) ? 1u : 0u));
    }
    if (grp_inf && e == 255 && frac == 0) mag = 16384;
    if (grp_nan) mag = 0;
    mant[i] = (b & kSign) ? -mag : mag;
  }
  uint32_t sb = emax == 0 ? 0u : static_cast<uint32_t>(e_eff - 13) << 23;
  if (grp_inf) sb = kExpo;
  if (grp_nan) sb = kCanonNaN;
  scale_bits = sb;
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
// U: rows each thread streams per pass. R = 256 / C rows share a workgroup pass (C = K / 32).
template <int U>
__global__ __launch_bounds__(kThreads) void gemv_w4a16_kernel(W4Args a) {
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

  uint32_t xb[32];
  load_chunk_bits(a.x, a.lda, a.bf16, m, cc, xb);
  int mant[32];
  uint32_t xs_bits;
  align_chunk(xb, mant, xs_bits);
  const ActBytes act = split_bytes(mant);
  const float xs = ffrom(xs_bits);

  const int nbase = blockIdx.x * rows_per_block;
  const size_t row_bytes = static_cast<size_t>(a.K / 2);
  v4u wv[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int n = nbase + u * R + r;
    wv[u] = (live && n < a.N)
                ? __builtin_nontemporal_load(reinterpret_cast<const v4u*>(a.Wp + n * row_bytes) + cc)
                : v4u{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    int d16 = chunk_dot16(wv[u], act);
    d16 += lane_xor1(d16);
    d16 += lane_xor2(d16);
    const int n = nbase + u * R + r;
    if (live && (cc & 3) == 0 && n < a.N) {
      const float ws = from_fp16_bits(a.ws[static_cast<size_t>(n) * G + g]);
      terms[u * R + r][g] = fmul(fmul(i2f(d16 >> 4), ws), xs);
    }
  }
  __syncthreads();

  // four bank chains per row, then (b0 + b1) + (b2 + b3)
  const int slot = tid >> 2;
  const int bank = tid & 3;
  const bool has_row = slot < rows_per_block;
  const int slot_c = has_row ? slot : 0;
  float acc = 0.0f;
  for (int gg = bank; gg < G; gg += 4) acc = fadd(acc, terms[slot_c][gg]);
  const float pair = fadd(acc, lane_xor1(acc));  // bank 0: b0 + b1, bank 2: b2 + b3
  const float other = lane_xor2(pair);
  const int u = slot_c / R, rr = slot_c - u * R;
  const int n = nbase + u * R + rr;
  if (has_row && bank == 0 && n < a.N) {
    float y = fadd(pair, other);
    if (a.bias) y = fadd(y, a.bias[n]);
    y = act_fn(y, a.act);
    store_out(a.Y, m * a.ldy, n, a.out, y, a.out_scale);
  }
}

template <int U>
hipError_t go_w4(const W4Args& a, hipStream_t s) {
  const int C = a.K / 32;
  const int R = kThreads / C;
  const int rows = R * U;
  const dim3 grid((a.N + rows - 1) / rows, a.M);
  hipLaunchKernelGGL(gemv_w4a16_kernel<U>, grid, dim3(kThreads), 0, s, a);
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
  // rows per block R * U must not exceed the 64 LDS term rows
  const int R = kThreads / (a.K / 32);
  if (R * 8 <= 64 && R > 1) return go_w4<8>(a, s);
  if (R * 4 <= 64) return go_w4<4>(a, s);
  if (R * 2 <= 64) return go_w4<2>(a, s);
  return go_w4<1>(a, s);
}

}  // namespace tars
