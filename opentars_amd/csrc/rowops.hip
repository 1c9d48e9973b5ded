// fp32 row functions, elementwise ops, rotary embedding and fp32 dot products of the golden model
// (tars_mini/golden.py:351-436, numerics.py:293-424), bit for bit.
//
// The contract fixes every summation order, so the kernels are laid out around the order rather
// than the other way round:
//  * sum16 (numerics.py:306-316): element j of a row goes to lane j mod 16, each lane adds its
//    elements in order from +0, then the 16 lanes fold pairwise (0+1, 2+3, ...) in four levels.
//    Here a row is a group of 16 consecutive lanes: lane l runs the chain of elements l, l+16, ...
//    and the fold is four DPP steps (lane xor 1, xor 2, the other half of each 8, the other 8 of
//    each 16). fadd is commutative bit for bit, and after each level every lane of a group of 2^i
//    holds the same partial, so the mirrored partners deliver exactly the reference's pairs.
//  * row maxima (fmax, order-free) reduce over a monotone unsigned key, NaN tracked beside it.
//  * fdot_nt is sum16 over the products; fdot_nn is one sequential k chain per output, so one lane
//    per output with the k loop unrolled and its loads issued ahead.
// Everything else is elementwise. All of these ops are latency-bound at decode sizes (a few
// thousand elements, tens of dependent steps per lane).
#include "kernels.h"

namespace tars {
namespace {

constexpr int kRowThreads = 256;  // 16 row groups of 16 lanes

__device__ __forceinline__ float fdpp_xor1(float v) { return __int_as_float(dpp<kDppQuadXor1>(__float_as_int(v))); }
__device__ __forceinline__ float fdpp_xor2(float v) { return __int_as_float(dpp<kDppQuadXor2>(__float_as_int(v))); }
__device__ __forceinline__ float fdpp_half(float v) { return __int_as_float(dpp<kDppRowHalfMirror>(__float_as_int(v))); }
__device__ __forceinline__ float fdpp_mirror(float v) { return __int_as_float(dpp<kDppRowMirror>(__float_as_int(v))); }

// The pairwise fold of a 16-lane group's partial sums (every lane receives the row sum).
__device__ __forceinline__ float fold16(float v) {
  v = fadd(v, fdpp_xor1(v));
  v = fadd(v, fdpp_xor2(v));
  v = fadd(v, fdpp_half(v));
  return fadd(v, fdpp_mirror(v));
}

__device__ __forceinline__ const float* frow(const void* base, int64_t ld, int m) {
  return reinterpret_cast<const float*>(static_cast<const char*>(base) + m * ld);
}

// ------------------------------------------------------------------------------ row functions
// One 16-lane group per row (golden.py:358-380; numerics.py:328-380).
__global__ __launch_bounds__(kRowThreads) void row_kernel(RowArgs a) {
  const int m = blockIdx.x * (kRowThreads / 16) + static_cast<int>(threadIdx.x >> 4);
  const int l = threadIdx.x & 15;
  if (m >= a.M) return;  // whole 16-lane groups leave together; the DPP steps stay inside a group
  const float* x = frow(a.x, a.lda, m);
  const int N = a.N;
  const int64_t yrow = m * a.ldy;
  if (a.fn == ROWFN_SOFTMAX) {
    const int V = a.valid ? min(max(a.valid[m], 1), N) : (a.causal_k > 0 ? min(N, a.causal_k + m) : N);
    uint32_t key = 0;
    int nan = 0;
    for (int j = l; j < V; j += 16) {
      const float v = ftz(x[j]);
      if (is_nan(v)) nan = 1;
      else key = max(key, fmax_key(v));
    }
    key = static_cast<uint32_t>(group_reduce<16>(static_cast<int>(key), OpMaxU{}));
    nan = group_reduce<16>(nan, OpOr{});
    const float nmx = fneg(nan ? ffrom(kCanonNaN) : fmax_from_key(key));
    float acc = 0.0f;
    for (int j = l; j < N; j += 16) acc = fadd(acc, j < V ? exp_f(fadd(x[j], nmx)) : 0.0f);
    const float r = recip_f(fold16(acc));
    for (int j = l; j < N; j += 16)
      store_out(a.y, yrow, j, a.out, fmul(j < V ? exp_f(fadd(x[j], nmx)) : 0.0f, r), a.out_scale);
    return;
  }
  float rs;
  float nmean = 0.0f;  // LayerNorm: -(mean); the others use x itself
  const float k = recip_f(i2f(N));
  if (a.fn == ROWFN_LAYERNORM) {
    float acc = 0.0f;
    for (int j = l; j < N; j += 16) acc = fadd(acc, x[j]);
    nmean = fneg(fmul(fold16(acc), k));
    float acc2 = 0.0f;
    for (int j = l; j < N; j += 16) {
      const float d = fadd(x[j], nmean);
      acc2 = fadd(acc2, fmul(d, d));
    }
    rs = rsqrt_f(fadd(fmul(fold16(acc2), k), a.eps));
  } else {
    float acc = 0.0f;
    for (int j = l; j < N; j += 16) acc = fadd(acc, fmul(x[j], x[j]));
    const float ss = fold16(acc);
    rs = rsqrt_f(fadd(a.fn == ROWFN_RMSNORM ? fmul(ss, k) : ss, a.eps));
  }
  for (int j = l; j < N; j += 16) {
    const float d = a.fn == ROWFN_LAYERNORM ? fadd(x[j], nmean) : ftz(x[j]);
    float y = fmul(fmul(d, rs), a.gamma[j]);
    if (a.beta) y = fadd(y, a.beta[j]);
    store_out(a.y, yrow, j, a.out, y, a.out_scale);
  }
}

// ------------------------------------------------------------------------------ elementwise
__device__ __forceinline__ float load_f(const void* base, int64_t ld, int m, int n, bool half) {
  const char* row = static_cast<const char*>(base) + m * ld;
  return half ? from_fp16_bits(reinterpret_cast<const uint16_t*>(row)[n]) : reinterpret_cast<const float*>(row)[n];
}

// golden.py:393-418: y = act(A) op B, each step one rounded operation; A may be fp16 (a state) and
// a broadcast row; B dense, one per column, one per row or one scalar; C (MULADD) in the output's
// float format. In place (Y = A or Y = C) is safe: each element is read before it is written by
// the same thread.
__global__ __launch_bounds__(256) void elt_kernel(EltArgs a) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= a.N) return;
  for (int m = blockIdx.y; m < a.M; m += gridDim.y) {
    const float av = act_fn(load_f(a.A, a.a_row ? 0 : a.lda, m, n, a.a_fp16), a.act);
    float b;
    if (a.bmode == BMODE_DENSE) b = load_f(a.B, a.ldb, m, n, false);
    else if (a.bmode == BMODE_ROW) b = a.B[n];
    else if (a.bmode == BMODE_COL) b = a.B[m];
    else b = a.B[0];
    float y;
    if (a.op == ELTOP_MUL) y = fmul(av, b);
    else if (a.op == ELTOP_ADD) y = fadd(av, b);
    else if (a.op == ELTOP_SUB) y = fadd(av, fneg(ftz(b)));
    else y = fadd(load_f(a.C, a.ldc, m, n, a.out == 3), fmul(av, b));
    store_out(a.Y, m * a.ldy, n, a.out, y, a.out_scale);
  }
}

// numerics.py:412-424 (golden.py:420-424): the first rot elements of each row rotated by table
// row m / rows_per_pos ([cos(0..h-1), sin(0..h-1)], h = rot / 2); the rest copied (flushed).
__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= a.N) return;
  const int h = a.rot / 2;
  for (int m = blockIdx.y; m < a.M; m += gridDim.y) {
    const float* x = frow(a.x, a.lda, m);
    const float* t = a.tab + static_cast<int64_t>(static_cast<unsigned>(m) / static_cast<unsigned>(a.rows_per_pos)) * a.rot;
    float y;
    if (n < h) y = fadd(fmul(x[n], t[n]), fneg(fmul(x[n + h], t[h + n])));
    else if (n < a.rot) y = fadd(fmul(x[n], t[n - h]), fmul(x[n - h], t[n]));
    else y = ftz(x[n]);
    store_out(a.y, m * a.ldy, n, a.out, y, a.out_scale);
  }
}

// golden.py:351-356: act on fp32 rows, converted.
__global__ __launch_bounds__(256) void relu_kernel(ReluArgs a) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= a.N) return;
  for (int m = blockIdx.y; m < a.M; m += gridDim.y) {
    store_out(a.y, m * a.ldy, n, a.out, act_fn(frow(a.x, a.lda, m)[n], a.act), a.out_scale);
  }
}

// ------------------------------------------------------------------------------ fp32 dots
// numerics.py:393-399: y[m][n] = sum16_k a[m][k] * b[n][k]; one 16-lane group per output.
__global__ __launch_bounds__(256) void fdot_nt_kernel(FdotArgs a) {
  const int n = blockIdx.x * 16 + static_cast<int>(threadIdx.x >> 4);
  const int l = threadIdx.x & 15;
  if (n >= a.N) return;  // whole 16-lane groups leave together
  const float* br = frow(a.B, a.ldb, n);
  for (int m = blockIdx.y; m < a.M; m += gridDim.y) {
    const float* ar = frow(a.A, a.lda, m);
    float acc = 0.0f;
    int k = l;
    for (; k + 48 < a.K; k += 64) {  // four chain steps with their loads issued together
      const float p0 = fmul(ar[k], br[k]), p1 = fmul(ar[k + 16], br[k + 16]);
      const float p2 = fmul(ar[k + 32], br[k + 32]), p3 = fmul(ar[k + 48], br[k + 48]);
      acc = fadd(fadd(fadd(fadd(acc, p0), p1), p2), p3);
    }
    for (; k < a.K; k += 16) acc = fadd(acc, fmul(ar[k], br[k]));
    const float y = fold16(acc);
    if (l == 0) store_out(a.Y, m * a.ldy, n, a.out, y, a.out_scale);
  }
}

// numerics.py:402-409: y[m][n] = ((+0 + a[m][0] b[0][n]) + a[m][1] b[1][n]) + ...; one lane per
// output, columns n across the lanes (b rows read coalesced; a[m][k] is the same for the wave's
// lanes of one m).
template <bool HALF>
__global__ __launch_bounds__(256) void fdot_nn_kernel(FdotArgs a) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= a.N) return;
  for (int m = blockIdx.y; m < a.M; m += gridDim.y) {
    const float* ar = frow(a.A, a.lda, m);
    float acc = 0.0f;
    int k = 0;
    for (; k + 8 <= a.K; k += 8) {
      float p[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) p[u] = fmul(ar[k + u], load_f(a.B, a.ldb, k + u, n, HALF));
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = fadd(acc, p[u]);
    }
    for (; k < a.K; ++k) acc = fadd(acc, fmul(ar[k], load_f(a.B, a.ldb, k, n, HALF)));
    store_out(a.Y, m * a.ldy, n, a.out, acc, a.out_scale);
  }
}

// Columns over grid x (per / threads each), rows over grid y with a stride loop past 65535 rows.
dim3 row_grid(int M, int N, int per) {
  return dim3(static_cast<unsigned>((N + per - 1) / per), static_cast<unsigned>(M < 65535 ? M : 65535));
}

}  // namespace

hipError_t launch_row(const RowArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(row_kernel, dim3((a.M + 15) / 16), dim3(kRowThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_elt(const EltArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(elt_kernel, row_grid(a.M, a.N, 256), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_rope(const RopeArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(rope_kernel, row_grid(a.M, a.N, 256), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_relu(const ReluArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(relu_kernel, row_grid(a.M, a.N, 256), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_fdot(const FdotArgs& a, hipStream_t s) {
  if (!a.nn) {
    hipLaunchKernelGGL(fdot_nt_kernel, row_grid(a.M, a.N, 16), dim3(256), 0, s, a);
  } else if (a.b_fp16) {
    hipLaunchKernelGGL(fdot_nn_kernel<true>, row_grid(a.M, a.N, 256), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL(fdot_nn_kernel<false>, row_grid(a.M, a.N, 256), dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace tars
