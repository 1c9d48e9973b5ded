// W8A8 GEMV (tars_mini/golden.py:326-349 at small M; the decode-step linears and the lm_head).
//
// Weight-streaming kernel: every weight byte is read from HBM exactly once. A row of W is cut into
// 16-byte chunks; a group of L lanes (L = 64 for K >= 1024) owns one row, lane `sub` taking chunks
// sub, sub + L, ... so each wave-wide load instruction reads L * 16 contiguous bytes of a row.
// Each lane keeps its activation chunks in registers (the activation row is tiny and shared by
// all rows), issues the loads of U rows back to back so U * CPL 16-byte loads are in flight, and
// accumulates with the packed signed 8-bit dot product (v_dot4, 4 MACs per instruction) into
// exact int32 sums. The L partial sums of a row are combined with cross-lane xor shuffles (exact
// integer adds, so the order is free), and lane `u` of the group runs the fp32 epilogue for row u.
//
// Roofline: HBM. Algorithmic bytes per row: K (weights) + 4 (scale) + 4 (output) (+4 bias).
#include "kernels.h"

namespace tars {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ v4i load_stream(const v4i* p) { return __builtin_nontemporal_load(p); }

__device__ __forceinline__ int dot16(v4i w, v4i x, int acc) {
  acc = __builtin_amdgcn_sdot4(w.x, x.x, acc, false);
  acc = __builtin_amdgcn_sdot4(w.y, x.y, acc, false);
  acc = __builtin_amdgcn_sdot4(w.z, x.z, acc, false);
  acc = __builtin_amdgcn_sdot4(w.w, x.w, acc, false);
  return acc;
}

template <int L>
__device__ __forceinline__ int group_sum(int v) {
#pragma unroll
  for (int off = L / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// CPL > 0: exactly CPL chunks per lane with the activations held in registers (K <= 128 * L).
// CPL == 0: any K, chunks walked in a loop with the activation chunk re-read from cache.
template <int L, int CPL, int U>
__global__ __launch_bounds__(kThreads) void gemv_w8a8_kernel(W8A8Args a) {
  constexpr int kSlots = 64 / L;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int slot = lane / L;
  const int sub = lane % L;
  const int m = blockIdx.y;
  const int C = a.K >> 4;
  const int n0 = (blockIdx.x * (kWaves * kSlots) + wave * kSlots + slot) * U;
  const v4i* xrow = reinterpret_cast<const v4i*>(a.A + m * a.lda);
  const v4i zero = {0, 0, 0, 0};

  int acc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) acc[u] = 0;

  if constexpr (CPL > 0) {
    v4i xv[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = sub + j * L;
      xv[j] = c < C ? xrow[c] : zero;
    }
    v4i wv[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int n = n0 + u;
      const v4i* wrow = reinterpret_cast<const v4i*>(a.W + static_cast<int64_t>(n) * a.K);
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = sub + j * L;
        wv[u][j] = (n < a.N && c < C) ? load_stream(wrow + c) : zero;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < CPL; ++j) acc[u] = dot16(wv[u][j], xv[j], acc[u]);
  } else {
    for (int c = sub; c < C; c += L) {
      const v4i xv = xrow[c];
      v4i wv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int n = n0 + u;
        wv[u] = n < a.N ? load_stream(reinterpret_cast<const v4i*>(a.W + static_cast<int64_t>(n) * a.K) + c) : zero;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) acc[u] = dot16(wv[u], xv, acc[u]);
    }
  }

#pragma unroll
  for (int u = 0; u < U; ++u) acc[u] = group_sum<L>(acc[u]);

  // lane `sub` of the group finishes row n0 + sub (U <= L)
  int mine = 0;
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (sub == u) mine = acc[u];
  const int n = n0 + sub;
  if (sub < U && n < a.N) {
    const float y = a.epi.value(mine, m, n);
    store_out(a.Y, m * a.ldy, n, a.epi.out, y, a.epi.out_scale);
  }
}

// ---- K split: blocks over consecutive column ranges of A, partials added in block order ----
template <int U>
__global__ __launch_bounds__(kThreads) void gemv_w8a8_ksplit_kernel(KSplitArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m = blockIdx.y;
  const int n0 = (blockIdx.x * kWaves + wave) * U;
  const float sr = a.srow ? a.srow[m] : 1.0f;
  const v4i zero = {0, 0, 0, 0};
  float y[U];
  for (int b = 0; b < a.nblocks; ++b) {
    const int C = a.K[b] >> 4;
    const v4i* xrow = reinterpret_cast<const v4i*>(a.A + m * a.lda + a.koff[b]);
    int acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] = 0;
    for (int c = lane; c < C; c += 64) {
      const v4i xv = xrow[c];
      v4i wv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int n = n0 + u;
        wv[u] = n < a.N ? load_stream(reinterpret_cast<const v4i*>(a.W[b] + static_cast<int64_t>(n) * a.K[b]) + c) : zero;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) acc[u] = dot16(wv[u], xv, acc[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = group_sum<64>(acc[u]);
      // the block's partial: the full W8A8 epilogue without bias or activation
      float part = i2f(s);
      if (a.srow) part = fmul(part, sr);
      const int n = min(n0 + u, a.N - 1);
      part = fmul(part, a.scol[n]);
      y[u] = b == 0 ? part : fadd(y[u], part);
    }
  }
  float mine = 0.0f;
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (lane == u) mine = y[u];
  const int n = n0 + lane;
  if (lane < U && n < a.N) {
    reinterpret_cast<float*>(reinterpret_cast<char*>(a.Y) + m * a.ldy)[n] = ftz(mine);
  }
}

template <int L, int CPL, int U>
hipError_t go(const W8A8Args& a, hipStream_t s) {
  constexpr int rows_per_block = kWaves * (64 / L) * U;
  const dim3 grid((a.N + rows_per_block - 1) / rows_per_block, a.M);
  hipLaunchKernelGGL((gemv_w8a8_kernel<L, CPL, U>), grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv_w8a8(const W8A8Args& a, hipStream_t s) {
  const int C = a.K / 16;
  if (C <= 8) return go<8, 1, 8>(a, s);
  if (C <= 16) return go<16, 1, 8>(a, s);
  if (C <= 32) return go<32, 1, 8>(a, s);
  switch ((C + 63) / 64) {
    case 1: return go<64, 1, 8>(a, s);
    case 2: return go<64, 2, 4>(a, s);
    case 3: return go<64, 3, 2>(a, s);
    case 4: return go<64, 4, 2>(a, s);
    case 5: return go<64, 5, 1>(a, s);
    case 6: return go<64, 6, 1>(a, s);
    case 7: return go<64, 7, 1>(a, s);
    case 8: return go<64, 8, 1>(a, s);
    default: return go<64, 0, 4>(a, s);
  }
}

hipError_t launch_gemv_w8a8_ksplit(const KSplitArgs& a, hipStream_t s) {
  constexpr int U = 4;
  constexpr int rows_per_block = kWaves * U;
  const dim3 grid((a.N + rows_per_block - 1) / rows_per_block, a.M);
  hipLaunchKernelGGL((gemv_w8a8_ksplit_kernel<U>), grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace tars
