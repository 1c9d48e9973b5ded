// Cross-lane reductions inside a 64-wide wavefront using DPP lane permutes (no LDS round trip).
//
// A group is L consecutive lanes (L = 4, 8, 16, 32 or 64, aligned to L). After the call every
// lane of a group holds the group's reduction. Within a 16-lane row the steps are quad_perm xor 1,
// quad_perm xor 2, row_half_mirror (the other quad of each 8) and row_mirror (the other 8 of the
// row); rows are combined with v_readlane. Only order-free operations are reduced here (exact
// int32 sums, unsigned maxima), so the combination order does not affect any result.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tars {

constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1, 0, 3, 2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2, 3, 0, 1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

struct OpAdd {
  __device__ __forceinline__ int operator()(int a, int b) const { return a + b; }
};
struct OpMaxU {
  __device__ __forceinline__ int operator()(int a, int b) const {
    return static_cast<int>(max(static_cast<uint32_t>(a), static_cast<uint32_t>(b)));
  }
};

struct OpOr {
  __device__ __forceinline__ int operator()(int a, int b) const { return a | b; }
};

template <int L, class Op>
__device__ __forceinline__ int group_reduce(int v, Op op) {
  static_assert(L == 4 || L == 8 || L == 16 || L == 32 || L == 64, "group of 4..64 lanes");
  v = op(v, dpp<kDppQuadXor1>(v));
  v = op(v, dpp<kDppQuadXor2>(v));
  if constexpr (L >= 8) v = op(v, dpp<kDppRowHalfMirror>(v));
  if constexpr (L >= 16) v = op(v, dpp<kDppRowMirror>(v));
  if constexpr (L == 32) {
    const int lo = op(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16));
    const int hi = op(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48));
    v = (threadIdx.x & 32) ? hi : lo;
  } else if constexpr (L == 64) {
    v = op(op(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
           op(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
  }
  return v;
}

template <int L>
__device__ __forceinline__ int group_sum(int v) { return group_reduce<L>(v, OpAdd{}); }

template <int L>
__device__ __forceinline__ uint32_t group_max(uint32_t v) {
  return static_cast<uint32_t>(group_reduce<L>(static_cast<int>(v), OpMaxU{}));
}

// ---- wave-wide sums of U values per lane, scattered over the lanes ----
// v_permlane32_swap(A, B) exchanges lanes 32-63 of A with lanes 0-31 of B, so afterwards A + B holds
// in lanes 0-31 the sum of A's lanes l and l ^ 32 and in lanes 32-63 the same sum of B's:
// one instruction and one add halve the number of values per lane (a reduce-scatter step, no
// selects). v_permlane16_swap does the same across the 16-lane rows (lane bit 4).
__device__ __forceinline__ int swap32_sum(int a, int b) {
  const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  return static_cast<int>(r[0]) + static_cast<int>(r[1]);
}
__device__ __forceinline__ int swap16_sum(int a, int b) {
  const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
  return static_cast<int>(r[0]) + static_cast<int>(r[1]);
}
constexpr int kDppRowRor4 = 0x124, kDppRowRor8 = 0x128, kDppRowRor12 = 0x12C;  // lane i <- lane (i - n) mod 16 of its row

// Every lane ends with the total over the wave's 64 lanes of one of its U (1, 2, 4 or 8) values,
// value scatter_row<U>(lane); exact int32 sums, so the order of the adds does not matter.
// U = 8: the pairs (v0, v1), (v2, v3), ... are halved across lane bit 5, the results across bit 4,
// then once more between lanes l and l ^ 1 (DPP with selects); the lane bits left are summed in full.
template <int U>
__device__ __forceinline__ int wave_sum_scatter(const int (&v)[U]) {
  static_assert(U == 1 || U == 2 || U == 4 || U == 8, "1, 2, 4 or 8 values per lane");
  if constexpr (U == 1) {
    const int t = group_sum<16>(v[0]);
    const int h = swap16_sum(t, t);
    return swap32_sum(h, h);
  } else if constexpr (U == 2) {
    const int t = group_sum<16>(swap32_sum(v[0], v[1]));
    return swap16_sum(t, t);
  } else if constexpr (U == 4) {
    return group_sum<16>(swap16_sum(swap32_sum(v[0], v[1]), swap32_sum(v[2], v[3])));
  } else {
    const int t0 = swap16_sum(swap32_sum(v[0], v[1]), swap32_sum(v[2], v[3]));
    const int t1 = swap16_sum(swap32_sum(v[4], v[5]), swap32_sum(v[6], v[7]));
    const bool odd = threadIdx.x & 1;
    int u = (odd ? t1 : t0) + dpp<kDppQuadXor1>(odd ? t0 : t1);
    u += dpp<kDppQuadXor2>(u);
    u += dpp<kDppRowRor4>(u);
    return u + dpp<kDppRowRor8>(u);
  }
}
// The value whose total lane `lane` holds after wave_sum_scatter<U>, and whether the lane is the
// first (lowest) lane holding that value's total.
template <int U>
__device__ __forceinline__ int scatter_row(int lane) {
  const int b5 = (lane >> 5) & 1, b4 = (lane >> 4) & 1;
  if constexpr (U == 1) return 0;
  else if constexpr (U == 2) return b5;
  else if constexpr (U == 4) return 2 * b4 + b5;
  else return 4 * (lane & 1) + 2 * b4 + b5;
}
template <int U>
__device__ __forceinline__ bool scatter_owner(int lane) {
  if constexpr (U == 1) return lane == 0;
  else if constexpr (U == 2) return (lane & 31) == 0;
  else if constexpr (U == 4) return (lane & 15) == 0;
  else return (lane & 14) == 0;
}

// The unsigned maximum over the wave's 64 lanes, in every lane (DPP within the 16-lane rows, then
// the rows' exchanges by permlane swaps: no v_readlane round trip through scalar registers).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  const int m = group_reduce<16>(static_cast<int>(v), OpMaxU{});
  const auto a = __builtin_amdgcn_permlane16_swap(m, m, false, false);
  const uint32_t h = max(static_cast<uint32_t>(a[0]), static_cast<uint32_t>(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(h, h, false, false);
  return max(static_cast<uint32_t>(b[0]), static_cast<uint32_t>(b[1]));
}

// Lane i receives lane (i ^ 1) / (i ^ 2)'s value (within its quad).
__device__ __forceinline__ int lane_xor1(int v) { return dpp<kDppQuadXor1>(v); }
__device__ __forceinline__ int lane_xor2(int v) { return dpp<kDppQuadXor2>(v); }
__device__ __forceinline__ float lane_xor1(float v) { return __int_as_float(dpp<kDppQuadXor1>(__float_as_int(v))); }
__device__ __forceinline__ float lane_xor2(float v) { return __int_as_float(dpp<kDppQuadXor2>(__float_as_int(v))); }

}  // namespace tars
