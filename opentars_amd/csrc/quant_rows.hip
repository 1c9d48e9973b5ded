// Per-token INT8 quantizer (tars_mini/numerics.py:383-390, ROW_QUANT at tars_mini/golden.py:369-372).
//
// One workgroup per row. Pass 1 takes the row maximum of |ftz(x)|: the maximum of the |x|
// encodings, flushed once. The reference's fmax is order-free (numerics.py:293-303), and on
// non-negative encodings it is exactly an unsigned integer max in which every NaN encoding
// (> 0x7F800000) wins, so the reduction is a plain wave/LDS max over bit patterns. Lane 0 then runs
// the fixed recip_f sequence once; pass 2 quantizes with q8 and writes 16 bytes per lane.
// HBM-bound: 4 bytes read and 1 written per element.
#include "kernels.h"

namespace tars {
namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void quant_rows_kernel(QuantArgs a) {
  const int m = blockIdx.x;
  const float4* row = reinterpret_cast<const float4*>(reinterpret_cast<const char*>(a.x) + m * a.lda);
  const int chunks = a.K / 16;  // 16 elements = 4 float4 per chunk
  uint32_t mx = 0;
  for (int c = threadIdx.x; c < chunks; c += kThreads) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      mx = max_abs_bits4(mx, row[4 * c + j]);
    }
  }
  mx = wave_max_u32(mx);  // DPP within rows, then permlane swaps (no lane reads)
  __shared__ uint32_t wave_max[kThreads / 64];
  __shared__ float inv_shared;
  if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = wave_max[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) t = max(t, wave_max[w]);
    t = flush_max_bits(t);
    float inv, sr;
    quant_scales(t, inv, sr);
    inv_shared = inv;
    a.s[m] = sr;
  }
  __syncthreads();
  const float inv = inv_shared;
  int4* qrow = reinterpret_cast<int4*>(a.q + m * a.ldq);
  for (int c = threadIdx.x; c < chunks; c += kThreads) {
    uint32_t packed[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 v = row[4 * c + j];
      packed[j] = q8x4(v.x, v.y, v.z, v.w, inv);
    }
    qrow[c] = make_int4(static_cast<int>(packed[0]), static_cast<int>(packed[1]),
                        static_cast<int>(packed[2]), static_cast<int>(packed[3]));
  }
}

}  // namespace

hipError_t launch_quant_rows(const QuantArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(quant_rows_kernel, dim3(a.M), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace tars
