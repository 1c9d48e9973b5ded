// sum16 (tars_mini/numerics.py:306-316) over rows held in LDS: element j of a row goes to lane
// j mod 16, each lane adds its elements in order from +0, then the 16 lanes fold pairwise (0+1,
// 2+3, ...) in four levels. A row is a group of 16 consecutive lanes: lane l runs the chain of
// elements l, l+16, ... and the fold is four DPP steps (lane xor 1, xor 2, the other half of each
// 8, the other 8 of each 16). fadd is commutative bit for bit, and after each level every lane of a
// group of 2^i holds the same partial, so the mirrored partners deliver exactly the reference's
// pairs. Shared by the row kernels and the fused norm + quantizer + GEMV kernel.
#pragma once

#include <type_traits>

#include "kernels.h"

namespace tars {
namespace {

__device__ __forceinline__ float fdpp_xor1(float v) { return __int_as_float(dpp<kDppQuadXor1>(__float_as_int(v))); }
__device__ __forceinline__ float fdpp_xor2(float v) { return __int_as_float(dpp<kDppQuadXor2>(__float_as_int(v))); }
__device__ __forceinline__ float fdpp_half(float v) { return __int_as_float(dpp<kDppRowHalfMirror>(__float_as_int(v))); }
__device__ __forceinline__ float fdpp_mirror(float v) { return __int_as_float(dpp<kDppRowMirror>(__float_as_int(v))); }

// The pairwise fold of a 16-lane group's partial chain sums (every lane receives the row sum,
// canonicalized).
__device__ __forceinline__ float fold16(float v) {
  v = fadd_chain(v, fdpp_xor1(v));
  v = fadd_chain(v, fdpp_xor2(v));
  v = fadd_chain(v, fdpp_half(v));
  return chain_end(fadd_chain(v, fdpp_mirror(v)));
}

// The 16-lane chains of sum16 over rows of n values in LDS (row i at v + i * ld), of the values
// (SQUARE: of fmul(v, v)): lane l of threads 16 i .. 16 i + 15 adds element l, l + 16, ... of row i
// in order from +0, then the pairwise fold; row i's sum lands in bcast[i] for every thread of the
// workgroup. v must hold contract results.
// NONNEG: every term is +0, at least 2^-126, +inf or NaN (a square of a contract result, or the
// terms of such a sum). Every partial sum is then +0, normal, +inf or NaN (a rounded sum of two
// non-negative values is at least the larger one), so the contract's flushes never fire and the
// plain chain, canonicalized at its end, is the contract's chain: no check, one add per step.
template <bool SQUARE, bool NONNEG = false>
__device__ __forceinline__ void lds_sum16_rows(const float* v, int ld, int rows, int n, float* bcast) {
  __syncthreads();  // v complete
  if (static_cast<int>(threadIdx.x) < 16 * rows) {
    const int l = threadIdx.x & 15, i = threadIdx.x >> 4;
    v += i * ld;
    // the chain unflushed with its partial sums checked (its terms are flushed contract results),
    // then with the flushes when one was subnormal
    auto chain = [&](auto flushed) {
      float acc = 0.0f;
      uint32_t mk = ~0u;
      auto step = [&](float t) {
        if constexpr (decltype(flushed)::value) {
          acc = fadd_chain(acc, t);
        } else {
          acc = __fadd_rn(acc, t);
          if constexpr (!SQUARE && !NONNEG) mk = min(mk, sub_key(acc));
        }
      };
      // blocks of a lane's terms read from LDS together, then added: one LDS round trip per block
      auto block = [&](int j0, auto size) {
        constexpr int B = decltype(size)::value;
        float t[B];
#pragma unroll
        for (int u = 0; u < B; ++u) t[u] = SQUARE ? fmul(v[j0 + l + 16 * u], v[j0 + l + 16 * u]) : v[j0 + l + 16 * u];
#pragma unroll
        for (int u = 0; u < B; ++u) step(t[u]);
      };
      int j0 = 0;
      for (; j0 + 16 * 32 <= n; j0 += 16 * 32) block(j0, std::integral_constant<int, 32>{});
      for (; j0 + 16 * 8 <= n; j0 += 16 * 8) block(j0, std::integral_constant<int, 8>{});
      for (int j = j0 + l; j < n; j += 16) step(SQUARE ? fmul(v[j], v[j]) : v[j]);
      return mk < kSubKeyNormal ? ffrom(kCanonNaN) : acc;  // NaN marks "recompute" (a NaN sum recomputes too)
    };
    float acc = chain(std::false_type{});
    if constexpr (!SQUARE && !NONNEG)
      if (__builtin_expect(is_nan(acc), 0)) acc = chain(std::true_type{});
    acc = fold16(acc);
    if (l == 0) bcast[i] = acc;
  }
  __syncthreads();
}

// The sum16 of v[0..n) in LDS (as lds_sum16_rows for one row), returned to every thread.
template <bool SQUARE, bool NONNEG = false>
__device__ __forceinline__ float lds_sum16(const float* v, int n, float* bcast) {
  lds_sum16_rows<SQUARE, NONNEG>(v, 0, 1, n, bcast);
  return *bcast;
}

// The sum16 of a row of n values (n % 64 == 0) held in LDS transposed for the chains: element e at
// v[(e % 16) * S + e / 16] (S = n / 16 + 4: chain lane l's terms are contiguous, read 16 bytes at a
// time). Run by every wave on its own: all four 16-lane rows of the wave run the same chains (the
// reads broadcast), so after the fold every lane holds the sum and no barrier or broadcast through
// LDS follows. The caller orders v's writes before the call. NONNEG as for lds_sum16_rows.
template <bool NONNEG>
__device__ __forceinline__ float wave_sum16_t(const float* v, int n, int S) {
  const float4* row = reinterpret_cast<const float4*>(v + (threadIdx.x & 15) * S);
  const int n4 = n >> 6;  // float4s of each lane's terms
  auto chain = [&](auto flushed) {
    float acc = 0.0f;
    uint32_t mk = ~0u;
    auto step = [&](float t) {
      if constexpr (decltype(flushed)::value) {
        acc = fadd_chain(acc, t);
      } else {
        acc = __fadd_rn(acc, t);
        if constexpr (!NONNEG) mk = min(mk, sub_key(acc));
      }
    };
    int k = 0;
    for (; k + 8 <= n4; k += 8) {
      float4 t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = row[k + u];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        step(t[u].x);
        step(t[u].y);
        step(t[u].z);
        step(t[u].w);
      }
    }
    for (; k < n4; ++k) {
      const float4 t = row[k];
      step(t.x);
      step(t.y);
      step(t.z);
      step(t.w);
    }
    return mk < kSubKeyNormal ? ffrom(kCanonNaN) : acc;  // NaN marks "recompute" (a NaN sum recomputes too)
  };
  float acc = chain(std::false_type{});
  if constexpr (!NONNEG)
    if (__builtin_expect(is_nan(acc), 0)) acc = chain(std::true_type{});
  return fold16(acc);
}

// The norm (LayerNorm / RMSNorm / L2Norm, golden.py:358-380) of one row of N values (N % 64 == 0)
// held as float4s by the 256 threads of a workgroup: thread t holds elements 4 (t + 256 j) ..
// 4 (t + 256 j) + 3 in x[j] (float4 index t + 256 j < N / 4; others ignored), flushed (NaN payloads
// are free: every NaN result is canonicalized); g and b hold gamma and beta there. v: LDS for
// 2 (N + 64) floats. On return x holds the norm's output values as an fp32 output stores them: the
// values and sums of the row kernels' norm, in the same order. Every wave runs the sums itself
// (wave_sum16_t), so the norm takes one workgroup barrier (two for LayerNorm, whose squared
// differences go to a second buffer).
//
// The contract's operations are written out where their wrappers are identities: a square of a
// flushed value is the raw product flushed (its NaN payload only feeds a sum that is canonicalized
// at its end), and the output chain fmul(fmul(x, rs), g) (+ beta) takes its inputs flushed once and
// canonicalizes once at the end (an intermediate NaN stays NaN to the end).
template <int XV>
__device__ __forceinline__ void norm_row_f4(int fn, int N, float eps, float4 (&x)[XV], const float4 (&g)[XV],
                                            const float4 (&b)[XV], bool beta, float* v) {
  const int t = threadIdx.x, N4 = N >> 2, S = (N >> 4) + 4;
  const float kinv = recip_f(i2f(N));
  auto sq = [](float a) { return ftz(__fmul_rn(a, a)); };
  // element e of float4 index i (e = 4 i + c) to its transposed place
  auto put = [&](float* w, int i, float4 a) {
    const int r = (i & 3) * 4, col = i >> 2;
    w[r * S + col] = a.x;
    w[(r + 1) * S + col] = a.y;
    w[(r + 2) * S + col] = a.z;
    w[(r + 3) * S + col] = a.w;
  };
  float rs;
  if (fn == ROWFN_LAYERNORM) {
#pragma unroll
    for (int j = 0; j < XV; ++j)
      if (t + 256 * j < N4) put(v, t + 256 * j, x[j]);
    __syncthreads();
    const float nmean = fneg(fmul(wave_sum16_t<false>(v, N, S), kinv));
    float* v2 = v + 16 * S;
#pragma unroll
    for (int j = 0; j < XV; ++j) {
      x[j] = make_float4(fadd(x[j].x, nmean), fadd(x[j].y, nmean), fadd(x[j].z, nmean), fadd(x[j].w, nmean));
      if (t + 256 * j < N4) put(v2, t + 256 * j, make_float4(sq(x[j].x), sq(x[j].y), sq(x[j].z), sq(x[j].w)));
    }
    __syncthreads();
    rs = rsqrt_f(fadd(fmul(wave_sum16_t<true>(v2, N, S), kinv), eps));
  } else {
#pragma unroll
    for (int j = 0; j < XV; ++j)
      if (t + 256 * j < N4) put(v, t + 256 * j, make_float4(sq(x[j].x), sq(x[j].y), sq(x[j].z), sq(x[j].w)));
    __syncthreads();
    const float ss = wave_sum16_t<true>(v, N, S);
    rs = rsqrt_f(fadd(fn == ROWFN_RMSNORM ? fmul(ss, kinv) : ss, eps));
  }
  // rs is canonical and never subnormal (rsqrt_f's results are 0, normal, infinite or the NaN)
  auto out = [&](float xe, float ge, float be) {
    float y = ftz(__fmul_rn(ftz(__fmul_rn(xe, rs)), ftz(ge)));
    if (beta) y = ftz(__fadd_rn(y, ftz(be)));
    return canon(y);
  };
#pragma unroll
  for (int j = 0; j < XV; ++j)
    x[j] = make_float4(out(x[j].x, g[j].x, b[j].x), out(x[j].y, g[j].y, b[j].y), out(x[j].z, g[j].z, b[j].z),
                       out(x[j].w, g[j].w, b[j].w));
}

}  // namespace
}  // namespace tars
