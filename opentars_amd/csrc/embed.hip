// Token rows of an export's bf16 embedding tables, written on the device.
//
// The board runtime looks the rows up on the host (deploy/kv260/sw/tars_board.py:298-316, _put):
// bf16 -> fp32 by moving the 16 bits to the top half (exact), then, for Gemma, one fp32 multiply
// by the manifest's scale (numpy: rounded to nearest even, subnormals kept). Here the tables stay
// resident in HBM and a step sends only token ids (kernel arguments): one workgroup row per token,
// each thread widening 8 elements (16 bytes in, 32 bytes out) or, for tables whose rows are not
// 16-byte multiples, one element. The library is built with fp32 denormals enabled, so __fmul_rn
// rounds exactly as numpy's float32 multiply does.
//
// Roofline: HBM; 2 bytes read + 4 written per element (a decode step moves one row: latency).
#include "kernels.h"

namespace tars {
namespace {

constexpr int kThreads = 256;

template <bool VEC, bool SCALED>
__global__ __launch_bounds__(kThreads) void embed_rows_kernel(EmbedArgs a) {
  const int i = blockIdx.y;
  const int64_t id = a.ids[i];
  const char* src = reinterpret_cast<const char*>(a.table) + id * a.ld_table;
  char* dst = reinterpret_cast<char*>(a.dst) + static_cast<int64_t>(i) * a.ldd;
  const float s = __uint_as_float(a.scale_bits);
  if constexpr (VEC) {
    const int e = 8 * (blockIdx.x * kThreads + threadIdx.x);
    if (e >= a.cols) return;
    const uint4 v = *reinterpret_cast<const uint4*>(src + 2 * e);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    float f[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[2 * j] = __uint_as_float(w[j] << 16);
      f[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
    }
    if constexpr (SCALED) {
#pragma unroll
      for (int j = 0; j < 8; ++j) f[j] = __fmul_rn(f[j], s);
    }
    float4* out = reinterpret_cast<float4*>(dst + 4 * e);
    out[0] = make_float4(f[0], f[1], f[2], f[3]);
    out[1] = make_float4(f[4], f[5], f[6], f[7]);
  } else {
    const int e = blockIdx.x * kThreads + threadIdx.x;
    if (e >= a.cols) return;
    float f = __uint_as_float(static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(src)[e]) << 16);
    if constexpr (SCALED) f = __fmul_rn(f, s);
    reinterpret_cast<float*>(dst)[e] = f;
  }
}

template <bool VEC>
void go(const EmbedArgs& a, hipStream_t s) {
  const int per = VEC ? 8 * kThreads : kThreads;
  const dim3 grid((a.cols + per - 1) / per, a.n);
  if (a.scaled) hipLaunchKernelGGL((embed_rows_kernel<VEC, true>), grid, dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL((embed_rows_kernel<VEC, false>), grid, dim3(kThreads), 0, s, a);
}

}  // namespace

hipError_t launch_embed_rows(const EmbedArgs& a, hipStream_t s) {
  const bool vec = a.cols % 8 == 0 && a.ld_table % 16 == 0 && a.ldd % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(a.table) % 16 == 0 && reinterpret_cast<uintptr_t>(a.dst) % 16 == 0;
  if (vec) go<true>(a, s);
  else go<false>(a, s);
  return hipGetLastError();
}

}  // namespace tars
