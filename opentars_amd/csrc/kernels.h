// Internal launcher interface between the C ABI (abi.hip) and the kernel translation units.
// Launchers assume validated arguments; they only pick a kernel instance and enqueue it.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fp32_contract.h"
#include "wave_reduce.h"

namespace tars {

// Predicated loads without branches. A load behind a branch makes the compiler's wait-counter
// bookkeeping assume either path where they join, so waiting for one early load (the activations)
// would also wait for every later one (the weight stream). These helpers always issue the load, on
// a valid fallback address when the predicate is false, and select the value afterwards.
template <class T>
__device__ __forceinline__ T load_pred(const T* p, const T* safe, bool pred, T zero) {
  const T v = *(pred ? p : safe);
  return pred ? v : zero;
}
template <class T>
__device__ __forceinline__ T load_stream_pred(const T* p, const T* safe, bool pred, T zero) {
  const T v = __builtin_nontemporal_load(pred ? p : safe);
  return pred ? v : zero;
}

// Keeps the machine scheduler from moving instructions across this point. Used between groups of
// loads whose issue order matters for the wait counters (activations before weights before
// epilogue operands).
__device__ __forceinline__ void issue_fence() { __builtin_amdgcn_sched_barrier(0); }

struct W8A8Args {
  const int8_t* A;  // [M, K] rows at stride lda bytes
  int64_t lda;
  const int8_t* W;  // [N, K] dense
  RowColEpilogue epi;
  void* Y;          // [M, N] rows at stride ldy bytes
  int64_t ldy;
  int M, N, K;
};

// Up to kMaxBlocks K blocks sharing A, srow and scol; partials add in block order.
constexpr int kMaxBlocks = 8;
struct KSplitArgs {
  const int8_t* A;
  int64_t lda;
  const float* srow;
  const float* scol;
  const int8_t* W[kMaxBlocks];
  int K[kMaxBlocks];
  int koff[kMaxBlocks];
  int nblocks;
  float* Y;
  int64_t ldy;
  int M, N;
};

struct QuantArgs {
  const float* x;
  int64_t lda;
  int8_t* q;
  int64_t ldq;
  float* s;
  int M, K;
};

struct AlignArgs {
  const void* x;
  int64_t lda;
  int bf16;          // 1: x holds bf16 bits
  int16_t* q;
  int64_t ldq;
  float* scales;
  int64_t lds;
  int M, K;
};

struct W4Args {
  const void* x;
  int64_t lda;
  int bf16;
  const uint8_t* Wp;   // [N, K/2]
  const uint16_t* ws;  // [N, K/128]
  const float* bias;
  int act, out;
  float out_scale;
  void* Y;
  int64_t ldy;
  int M, N, K;
};

// Fused per-token quantizer + grouped W8A8 GEMV: the activation rows are quantized in registers by
// every wave and feed up to kMaxGroups weight matrices (q/k/v, gate/up) in one launch.
constexpr int kMaxGroups = 4;
struct GemvGroup {
  const int8_t* W;       // [N, K] dense
  RowColEpilogue epi;    // srow unused: the row scale comes from the fused quantizer
  void* Y;
  int64_t ldy;
  int N;
};

struct QuantGemvArgs {
  const float* x;        // [M, K] fp32 rows at stride lda bytes
  int64_t lda;
  int8_t* q;             // optional: the quantized rows (stride ldq) and row scales, as quant_rows
  int64_t ldq;
  float* s;
  int M, K;
  GemvGroup g[kMaxGroups];
  int ngroups;
  int block_start[kMaxGroups + 1];  // first workgroup of each group along grid x
};

hipError_t launch_quant_rows(const QuantArgs& a, hipStream_t s);
hipError_t launch_gemv_w8a8(const W8A8Args& a, hipStream_t s);
hipError_t launch_quant_gemv_w8a8(QuantGemvArgs& a, hipStream_t s);
hipError_t launch_gemm_w8a8_mfma(const W8A8Args& a, hipStream_t s);
hipError_t launch_gemv_w8a8_ksplit(const KSplitArgs& a, hipStream_t s);
hipError_t launch_gemm_w8a8_ksplit_mfma(const KSplitArgs& a, hipStream_t s);
hipError_t launch_align_w4(const AlignArgs& a, hipStream_t s);
hipError_t launch_gemv_w4a16(const W4Args& a, hipStream_t s);

}  // namespace tars
