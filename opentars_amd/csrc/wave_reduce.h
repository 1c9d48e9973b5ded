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

// Lane i receives lane (i ^ 1) / (i ^ 2)'s value (within its quad).
__device__ __forceinline__ int lane_xor1(int v) { return dpp<kDppQuadXor1>(v); }
__device__ __forceinline__ int lane_xor2(int v) { return dpp<kDppQuadXor2>(v); }
__device__ __forceinline__ float lane_xor1(float v) { return __int_as_float(dpp<kDppQuadXor1>(__float_as_int(v))); }
__device__ __forceinline__ float lane_xor2(float v) { return __int_as_float(dpp<kDppQuadXor2>(__float_as_int(v))); }

}  // namespace tars
