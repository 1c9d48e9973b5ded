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
#include <mutex>
#include <type_traits>
#include <utility>
#include <vector>

#include "kernels.h"
#include "row_sums.h"

namespace tars {
namespace {

constexpr int kRowThreads = 256;  // 16 row groups of 16 lanes

__device__ __forceinline__ const float* frow(const void* base, int64_t ld, int m) {
  return reinterpret_cast<const float*>(static_cast<const char*>(base) + m * ld);
}

// ------------------------------------------------------------------------------ row functions
// A lane's elements of a row arrive in blocks of kChunk (elements l, l + 16, ... of the block),
// loaded together before the block's dependent chain runs, and the next block is loaded while the
// current one is consumed: one memory round trip per 16 * kChunk elements instead of one per
// element.
constexpr int kChunk = 16;

struct RowBlock {
  float v[kChunk];
};

__device__ __forceinline__ void load_block(RowBlock& b, const float* x, int j0, int l, int n) {
#pragma unroll
  for (int u = 0; u < kChunk; ++u) {
    const int j = j0 + l + 16 * u;
    b.v[u] = load_pred(x + j, x, j < n, 0.0f);
  }
}

// Runs f(j, value) over this lane's elements j = l, l + 16, ... < n, in order.
template <class Fn>
__device__ __forceinline__ void for_lane(const float* x, int l, int n, Fn&& f) {
  RowBlock cur, nxt;
  load_block(cur, x, 0, l, n);
  for (int j0 = 0; j0 < n; j0 += 16 * kChunk) {
    if (j0 + 16 * kChunk < n) load_block(nxt, x, j0 + 16 * kChunk, l, n);
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
      const int j = j0 + l + 16 * u;
      if (j < n) f(j, cur.v[u]);
    }
    cur = nxt;
  }
}

// Rows up to kLdsRow elements: one workgroup per row, the row staged in LDS; the elementwise work
// (exp, differences, squares, outputs) spread over all 256 threads, only the fixed-order sums on
// 16 lanes (golden.py:358-380; numerics.py:328-380).
constexpr int kLdsRow = 12288;

// Elements per thread per pass of row_lds_kernel's staging and output loops: every global load of
// a pass is issued before any of its values is used (one memory round trip per pass, not per
// element); rows up to kRowThreads * kRowE elements take one pass.
constexpr int kRowE = 8;

// A norm whose row fits one pass of kRowThreads * kRowE elements: each thread keeps its elements
// (and then the LayerNorm differences) in registers, and all threads write the terms of each sum
// (x, or the squares) to LDS, so the 16-lane chains only add. xv: the thread's raw elements
// t + u * kRowThreads of row m; gv, bv: gamma and beta there. The same values in the same order as
// the general path of row_lds_kernel.
__device__ __forceinline__ void norm_in_regs(const RowArgs& a, int m, float (&xv)[kRowE], const float (&gv)[kRowE],
                                             const float (&bv)[kRowE], float* v, float* bcast) {
  const int N = a.N, t = threadIdx.x;
  const int64_t yrow = m * a.ldy;
  const float kinv = recip_f(i2f(N));
#pragma unroll
  for (int u = 0; u < kRowE; ++u) xv[u] = ftz(xv[u]);
  float rs;
  if (a.fn == ROWFN_LAYERNORM) {
#pragma unroll
    for (int u = 0; u < kRowE; ++u)
      if (t + u * kRowThreads < N) v[t + u * kRowThreads] = xv[u];
    const float nmean = fneg(fmul(lds_sum16<false>(v, N, bcast), kinv));
#pragma unroll
    for (int u = 0; u < kRowE; ++u) {
      xv[u] = fadd(xv[u], nmean);  // d = x + -mean
      if (t + u * kRowThreads < N) v[t + u * kRowThreads] = fmul(xv[u], xv[u]);
    }
    rs = rsqrt_f(fadd(fmul(lds_sum16<false, true>(v, N, bcast), kinv), a.eps));
  } else {
#pragma unroll
    for (int u = 0; u < kRowE; ++u)
      if (t + u * kRowThreads < N) v[t + u * kRowThreads] = fmul(xv[u], xv[u]);
    const float ss = lds_sum16<false, true>(v, N, bcast);
    rs = rsqrt_f(fadd(a.fn == ROWFN_RMSNORM ? fmul(ss, kinv) : ss, a.eps));
  }
#pragma unroll
  for (int u = 0; u < kRowE; ++u) {
    const int j = t + u * kRowThreads;
    if (j < N) {
      float y = fmul(fmul(xv[u], rs), gv[u]);
      if (a.beta) y = fadd(y, bv[u]);
      store_out(a.y, yrow, j, a.out, y, a.out_scale);
    }
  }
}

__global__ __launch_bounds__(kRowThreads) void row_lds_kernel(RowArgs a) {
  __shared__ float v[kLdsRow];
  __shared__ uint32_t red[kRowThreads / 64 + 1];
  __shared__ float bcast;
  // every kernel argument the first loads need, in one scalar round trip
  __asm__ volatile("" : : "s"(a.x), "s"(a.lda), "s"(a.N), "s"(a.fn), "s"(a.gamma), "s"(a.beta));
  const int m = blockIdx.x;
  const float* x = frow(a.x, a.lda, m);
  const int N = a.N, t = threadIdx.x;
  const int64_t yrow = m * a.ldy;
  const bool norm = a.fn != ROWFN_SOFTMAX;
  if (norm && N <= kRowThreads * kRowE) {
    float xv[kRowE], gv[kRowE], bv[kRowE];
#pragma unroll
    for (int u = 0; u < kRowE; ++u) {
      const int j = t + u * kRowThreads;
      xv[u] = *(j < N ? x + j : x);
      gv[u] = *(j < N ? a.gamma + j : x);
      bv[u] = *(a.beta && j < N ? a.beta + j : x);
    }
    norm_in_regs(a, m, xv, gv, bv, v, &bcast);
    return;
  }
  // the row into LDS; the first pass's gamma and beta (norms) are fetched with it
  float g0[kRowE], b0[kRowE];
  for (int j0 = 0; j0 < N; j0 += kRowThreads * kRowE) {
    float xv[kRowE];
#pragma unroll
    for (int u = 0; u < kRowE; ++u) {
      const int j = j0 + t + u * kRowThreads;
      xv[u] = *(j < N ? x + j : x);
    }
    if (j0 == 0) {
#pragma unroll
      for (int u = 0; u < kRowE; ++u) {
        const int j = t + u * kRowThreads;
        g0[u] = *(norm && j < N ? a.gamma + j : x);
        b0[u] = *(norm && a.beta && j < N ? a.beta + j : x);
      }
    }
#pragma unroll
    for (int u = 0; u < kRowE; ++u) {
      const int j = j0 + t + u * kRowThreads;
      if (j < N) v[j] = ftz(xv[u]);
    }
  }
  if (a.fn == ROWFN_SOFTMAX) {
    const int V = a.valid ? min(max(a.valid[m], 1), N) : (a.causal_k > 0 ? min(N, a.causal_k + m) : N);
    __syncthreads();
    uint32_t key = 0;
    int nan = 0;
    for (int j = t; j < V; j += kRowThreads) {
      if (is_nan(v[j])) nan = 1;
      else key = max(key, fmax_key(v[j]));
    }
    key = static_cast<uint32_t>(group_reduce<64>(static_cast<int>(key), OpMaxU{}));
    nan = group_reduce<64>(nan, OpOr{});
    if ((t & 63) == 0) red[t >> 6] = nan ? 0xFFFFFFFFu : key;  // NaN: a key no value has
    __syncthreads();
    uint32_t k = 0;
#pragma unroll
    for (int w = 0; w < kRowThreads / 64; ++w) k = max(k, red[w]);
    const float nmx = fneg(k == 0xFFFFFFFFu ? ffrom(kCanonNaN) : fmax_from_key(k));
    __syncthreads();  // every thread has read red before v is rewritten
    for (int j = t; j < N; j += kRowThreads) v[j] = j < V ? exp_f(fadd(v[j], nmx)) : 0.0f;
    const float r = recip_f(lds_sum16<false, true>(v, N, &bcast));  // exp_f values: 0, normal, inf or NaN
    for (int j = t; j < N; j += kRowThreads) store_out(a.y, yrow, j, a.out, fmul(v[j], r), a.out_scale);
    return;
  }
  const float kinv = recip_f(i2f(N));
  float rs;
  if (a.fn == ROWFN_LAYERNORM) {
    const float nmean = fneg(fmul(lds_sum16<false>(v, N, &bcast), kinv));
    for (int j = t; j < N; j += kRowThreads) v[j] = fadd(v[j], nmean);  // d = x + -mean
    rs = rsqrt_f(fadd(fmul(lds_sum16<true>(v, N, &bcast), kinv), a.eps));
  } else {
    const float ss = lds_sum16<true>(v, N, &bcast);
    rs = rsqrt_f(fadd(a.fn == ROWFN_RMSNORM ? fmul(ss, kinv) : ss, a.eps));
  }
  for (int j0 = 0; j0 < N; j0 += kRowThreads * kRowE) {
    float gv[kRowE], bv[kRowE];
#pragma unroll
    for (int u = 0; u < kRowE; ++u) {
      const int j = j0 + t + u * kRowThreads;
      gv[u] = j0 == 0 ? g0[u] : *(j < N ? a.gamma + j : a.gamma);
      bv[u] = j0 == 0 ? b0[u] : *(a.beta && j < N ? a.beta + j : a.gamma);
    }
#pragma unroll
    for (int u = 0; u < kRowE; ++u) {
      const int j = j0 + t + u * kRowThreads;
      if (j < N) {
        float y = fmul(fmul(v[j], rs), gv[u]);
        if (a.beta) y = fadd(y, bv[u]);
        store_out(a.y, yrow, j, a.out, y, a.out_scale);
      }
    }
  }
}

// A residual add and the norm that reads it (the executor's fusion of an ELT ADD on dense fp32
// rows with an fp32 output, no activation, and the LayerNorm / RMSNorm / L2Norm of its output, rows
// of at most kRowThreads * kRowE elements): each thread adds its elements as elt_fast_kernel does,
// writes the sums (the ELT's output) and runs the norm on them from registers. In place is as safe
// as for the ELT alone: each element is read and written by one thread.
__global__ __launch_bounds__(kRowThreads) void add_norm_kernel(EltArgs e, RowArgs r) {
  __shared__ float v[kRowThreads * kRowE];
  __shared__ float bcast;
  __asm__ volatile("" : : "s"(e.A), "s"(e.lda), "s"(e.B), "s"(e.ldb), "s"(r.gamma), "s"(r.beta), "s"(r.N));
  const int m = blockIdx.x, t = threadIdx.x, N = r.N;
  const float* A = frow(e.A, e.lda, m);
  const float* B = frow(e.B, e.ldb, m);
  float xa[kRowE], xb[kRowE], gv[kRowE], bv[kRowE];
#pragma unroll
  for (int u = 0; u < kRowE; ++u) {
    const int j = t + u * kRowThreads;
    xa[u] = *(j < N ? A + j : A);
    xb[u] = *(j < N ? B + j : B);
    gv[u] = *(j < N ? r.gamma + j : A);
    bv[u] = *(r.beta && j < N ? r.beta + j : A);
  }
  float* Y = reinterpret_cast<float*>(static_cast<char*>(e.Y) + m * e.ldy);
#pragma unroll
  for (int u = 0; u < kRowE; ++u) {
    const int j = t + u * kRowThreads;
    xa[u] = ftz(fadd(act_fn(xa[u], 0), xb[u]));
    if (j < N) Y[j] = xa[u];
  }
  norm_in_regs(r, m, xa, gv, bv, v, &bcast);
}

// A norm (LayerNorm / RMSNorm / L2Norm, fp32 output) and the RoPE of its output rows (fp32 output;
// the executor's fusion of a decoder's q / k norm and rotation, rows of at most kRowThreads * kRowE
// elements): each workgroup normalizes its row as row_lds_kernel does and stores it; after a
// workgroup barrier, which makes the row's stores visible to the workgroup, it rotates the stored
// values as rope_fast_kernel does.
__device__ __forceinline__ void norm_rope_row(const RowArgs& r, const RopeArgs& p, int m, float* v, float* bcast) {
  __asm__ volatile("" : : "s"(r.x), "s"(r.lda), "s"(r.gamma), "s"(r.beta), "s"(r.N), "s"(p.x), "s"(p.lda), "s"(p.tab),
                   "s"(p.rows_per_pos), "s"(p.rot), "s"(p.y), "s"(p.ldy));
  const int t = threadIdx.x, N = r.N;
  const float* x = frow(r.x, r.lda, m);
  float xv[kRowE], gv[kRowE], bv[kRowE];
#pragma unroll
  for (int u = 0; u < kRowE; ++u) {
    const int j = t + u * kRowThreads;
    xv[u] = *(j < N ? x + j : x);
    gv[u] = *(j < N ? r.gamma + j : x);
    bv[u] = *(r.beta && j < N ? r.beta + j : x);
  }
  norm_in_regs(r, m, xv, gv, bv, v, bcast);
  __syncthreads();
  const float* xr = frow(p.x, p.lda, m);
  const float* tb = p.tab + static_cast<int64_t>(static_cast<unsigned>(m) / static_cast<unsigned>(p.rows_per_pos)) * p.rot;
  const int h = p.rot / 2;
  float* y = reinterpret_cast<float*>(static_cast<char*>(p.y) + m * p.ldy);
  for (int n = t; n < N; n += kRowThreads) {
    const bool lo = n < h, rotated = n < p.rot;
    const int q = lo ? n + h : rotated ? n - h : n;  // rotation partner
    const int c = lo ? n : rotated ? n - h : 0;      // cos index; the sin is at h + c
    const float xn = xr[n], xp = xr[q], tc = tb[c], ts = tb[h + c];
    float o;
    if (lo) o = fadd(fmul(xn, tc), fneg(fmul(xp, ts)));
    else if (rotated) o = fadd(fmul(xn, tc), fmul(xp, ts));
    else o = ftz(xn);
    y[n] = ftz(o);
  }
}

// One or two independent (norm, RoPE) jobs in one launch (a decoder's q and k norms and rotations):
// workgroups [0, M0) take job 0's rows, the rest job 1's.
__global__ __launch_bounds__(kRowThreads) void norm_rope_kernel(RowArgs r0, RopeArgs p0, RowArgs r1, RopeArgs p1, int M0) {
  __shared__ float v[kRowThreads * kRowE];
  __shared__ float bcast;
  const int m = blockIdx.x;
  if (m < M0) norm_rope_row(r0, p0, m, v, &bcast);
  else norm_rope_row(r1, p1, m - M0, v, &bcast);
}

// Longer rows: one 16-lane group per row, the lane's elements streamed in blocks.
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
    for_lane(x, l, V, [&](int, float xv) {
      const float v = ftz(xv);
      if (is_nan(v)) nan = 1;
      else key = max(key, fmax_key(v));
    });
    key = static_cast<uint32_t>(group_reduce<16>(static_cast<int>(key), OpMaxU{}));
    nan = group_reduce<16>(nan, OpOr{});
    const float nmx = fneg(nan ? ffrom(kCanonNaN) : fmax_from_key(key));
    float acc = 0.0f;
    for_lane(x, l, N, [&](int j, float xv) { acc = fadd(acc, j < V ? exp_f(fadd(xv, nmx)) : 0.0f); });
    const float r = recip_f(fold16(acc));
    for_lane(x, l, N, [&](int j, float xv) {
      store_out(a.y, yrow, j, a.out, fmul(j < V ? exp_f(fadd(xv, nmx)) : 0.0f, r), a.out_scale);
    });
    return;
  }
  float rs;
  float nmean = 0.0f;  // LayerNorm: -(mean); the others use x itself
  const float k = recip_f(i2f(N));
  if (a.fn == ROWFN_LAYERNORM) {
    float acc = 0.0f;
    for_lane(x, l, N, [&](int, float xv) { acc = fadd(acc, xv); });
    nmean = fneg(fmul(fold16(acc), k));
    float acc2 = 0.0f;
    for_lane(x, l, N, [&](int, float xv) {
      const float d = fadd(xv, nmean);
      acc2 = fadd(acc2, fmul(d, d));
    });
    rs = rsqrt_f(fadd(fmul(fold16(acc2), k), a.eps));
  } else {
    float acc = 0.0f;
    for_lane(x, l, N, [&](int, float xv) { acc = fadd(acc, fmul(xv, xv)); });
    const float ss = fold16(acc);
    rs = rsqrt_f(fadd(a.fn == ROWFN_RMSNORM ? fmul(ss, k) : ss, a.eps));
  }
  const bool ln = a.fn == ROWFN_LAYERNORM;
  for_lane(x, l, N, [&](int j, float xv) {
    const float d = ln ? fadd(xv, nmean) : ftz(xv);
    float y = fmul(fmul(d, rs), a.gamma[j]);
    if (a.beta) y = fadd(y, a.beta[j]);
    store_out(a.y, yrow, j, a.out, y, a.out_scale);
  });
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

// ELT on dense fp32 rows with an fp32 output and the activation fixed at compile time (a decode
// step's residual adds and gated products): every kernel argument in one scalar round trip and each
// thread's two loads in one batch. Same steps as elt_kernel; in place is as safe.
template <int OP, int ACT>
__global__ __launch_bounds__(256) void elt_fast_kernel(EltArgs a) {
  __asm__ volatile("" : : "s"(a.A), "s"(a.lda), "s"(a.B), "s"(a.ldb), "s"(a.Y), "s"(a.ldy), "s"(a.M), "s"(a.N));
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= a.N) return;
  for (int m = blockIdx.y; m < a.M; m += gridDim.y) {
    const float x = frow(a.A, a.lda, m)[n];
    const float b = frow(a.B, a.ldb, m)[n];
    const float av = act_fn(x, ACT);
    float y;
    if constexpr (OP == ELTOP_MUL) y = fmul(av, b);
    else if constexpr (OP == ELTOP_ADD) y = fadd(av, b);
    else y = fadd(av, fneg(ftz(b)));
    reinterpret_cast<float*>(static_cast<char*>(a.Y) + m * a.ldy)[n] = ftz(y);
  }
}

// RoPE with an fp32 output: the element, its rotation partner and both table entries in one batch
// of loads (partner and table indices chosen without branches), then rope_kernel's steps.
__global__ __launch_bounds__(256) void rope_fast_kernel(RopeArgs a) {
  __asm__ volatile("" : : "s"(a.x), "s"(a.lda), "s"(a.tab), "s"(a.rows_per_pos), "s"(a.rot), "s"(a.y), "s"(a.ldy),
                   "s"(a.M), "s"(a.N));
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= a.N) return;
  const int h = a.rot / 2;
  const bool lo = n < h, rotated = n < a.rot;
  const int p = lo ? n + h : rotated ? n - h : n;   // rotation partner
  const int c = lo ? n : rotated ? n - h : 0;       // cos index; the sin is at h + c
  for (int m = blockIdx.y; m < a.M; m += gridDim.y) {
    const float* x = frow(a.x, a.lda, m);
    const float* t = a.tab + static_cast<int64_t>(static_cast<unsigned>(m) / static_cast<unsigned>(a.rows_per_pos)) * a.rot;
    const float xn = x[n], xp = x[p], tc = t[c], ts = t[h + c];
    float y;
    if (lo) y = fadd(fmul(xn, tc), fneg(fmul(xp, ts)));
    else if (rotated) y = fadd(fmul(xn, tc), fmul(xp, ts));
    else y = ftz(xn);
    reinterpret_cast<float*>(static_cast<char*>(a.y) + m * a.ldy)[n] = ftz(y);
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
// numerics.py:393-399: y[m][n] = sum16_k a[m][k] * b[n][k]; one 16-lane group per output. Lane l's
// chain (k = l, l + 16, ...) consumes blocks of kNtChunk products whose loads were issued one block
// ahead.
constexpr int kNtChunk = 8;

struct NtBlock {
  float a[kNtChunk], b[kNtChunk];
  __device__ __forceinline__ void load(const float* ar, const float* br, int k0, int l, int K) {
#pragma unroll
    for (int u = 0; u < kNtChunk; ++u) {
      const int k = k0 + l + 16 * u;
      a[u] = load_pred(ar + k, ar, k < K, 0.0f);
      b[u] = load_pred(br + k, br, k < K, 0.0f);
    }
  }
};

__global__ __launch_bounds__(256) void fdot_nt_kernel(FdotArgs a) {
  const int n = blockIdx.x * 16 + static_cast<int>(threadIdx.x >> 4);
  const int l = threadIdx.x & 15;
  if (n >= a.N) return;  // whole 16-lane groups leave together
  const float* br = frow(a.B, a.ldb, n);
  for (int m = blockIdx.y; m < a.M; m += gridDim.y) {
    const float* ar = frow(a.A, a.lda, m);
    float acc = 0.0f;
    NtBlock cur, nxt;
    cur.load(ar, br, 0, l, a.K);
    for (int k0 = 0; k0 < a.K; k0 += 16 * kNtChunk) {
      if (k0 + 16 * kNtChunk < a.K) nxt.load(ar, br, k0 + 16 * kNtChunk, l, a.K);
#pragma unroll
      for (int u = 0; u < kNtChunk; ++u)
        if (k0 + l + 16 * u < a.K) acc = fadd_chain(acc, fmul(cur.a[u], cur.b[u]));
      cur = nxt;
    }
    const float y = fold16(acc);
    if (l == 0) store_out(a.Y, m * a.ldy, n, a.out, y, a.out_scale);
  }
}

// numerics.py:402-409: y[m][n] = ((+0 + a[m][0] b[0][n]) + a[m][1] b[1][n]) + ...: one sequential
// k chain per output. A workgroup owns 128 columns; all 256 threads stage B in LDS in blocks of
// kNnRows rows (fp16 widened to fp32 on the way), the next block's global loads in flight while
// the 128 chain threads consume the current one from LDS.
constexpr int kNnCols = 128, kNnRows = 56;
constexpr int kNnPer = kNnRows * kNnCols / 4 / 256;  // 4-element groups per thread per block (7)
static_assert(kNnRows * kNnCols / 4 % 256 == 0 && kNnRows <= 256, "block shape");

template <bool HALF>
struct NnStage {
  float4 r[kNnPer];
  float a;
  __device__ __forceinline__ void load(const FdotArgs& f, const float* ar, int k0, int c0) {
    const int t = threadIdx.x;
#pragma unroll
    for (int u = 0; u < kNnPer; ++u) {
      const int e = t + 256 * u, row = e / (kNnCols / 4), c = c0 + 4 * (e % (kNnCols / 4));
      const int k = k0 + row;
      const bool ok = k < f.K && c < f.N;  // N % 4 == 0 is not required: a partial group is zero-filled
      const char* rowp = static_cast<const char*>(f.B) + static_cast<int64_t>(ok ? k : 0) * f.ldb;
      if constexpr (HALF) {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(rowp);
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = (ok && c + q < f.N) ? from_fp16_bits(h[c + q]) : 0.0f;
        r[u] = make_float4(v[0], v[1], v[2], v[3]);
      } else {
        const float* x = reinterpret_cast<const float*>(rowp);
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = (ok && c + q < f.N) ? x[c + q] : 0.0f;
        r[u] = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
    a = (t < kNnRows && k0 + t < f.K) ? ar[k0 + t] : 0.0f;
  }
  __device__ __forceinline__ void store(float (*lb)[kNnCols], float* la) const {
    const int t = threadIdx.x;
#pragma unroll
    for (int u = 0; u < kNnPer; ++u) {
      const int e = t + 256 * u;
      *reinterpret_cast<float4*>(&lb[e / (kNnCols / 4)][4 * (e % (kNnCols / 4))]) = r[u];
    }
    if (t < kNnRows) la[t] = a;
  }
};

template <bool HALF>
__global__ __launch_bounds__(256) void fdot_nn_kernel(FdotArgs a) {
  __shared__ __align__(16) float lb[2][kNnRows][kNnCols];
  __shared__ float la[2][kNnRows];
  const int c0 = blockIdx.x * kNnCols, t = threadIdx.x;
  const int n = c0 + t;
  const int nb = (a.K + kNnRows - 1) / kNnRows;
  for (int m = blockIdx.y; m < a.M; m += gridDim.y) {
    const float* ar = frow(a.A, a.lda, m);
    NnStage<HALF> st;
    st.load(a, ar, 0, c0);
    __syncthreads();  // the previous row's chains are done with the buffers
    st.store(lb[0], la[0]);
    __syncthreads();
    float acc = 0.0f;
    for (int b = 0; b < nb; ++b) {
      if (b + 1 < nb) st.load(a, ar, (b + 1) * kNnRows, c0);
      if (t < kNnCols) {
        const int rows = min(kNnRows, a.K - b * kNnRows);
        const float(*cb)[kNnCols] = lb[b & 1];
        const float* ca = la[b & 1];
        int kk = 0;
        for (; kk + 8 <= rows; kk += 8) {
          float p[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) p[u] = fmul(ca[kk + u], cb[kk + u][t]);
#pragma unroll
          for (int u = 0; u < 8; ++u) acc = fadd_chain(acc, p[u]);
        }
        for (; kk < rows; ++kk) acc = fadd_chain(acc, fmul(ca[kk], cb[kk][t]));
      }
      if (b + 1 < nb) st.store(lb[(b + 1) & 1], la[(b + 1) & 1]);
      __syncthreads();
    }
    if (t < kNnCols && n < a.N) store_out(a.Y, m * a.ldy, n, a.out, chain_end(acc), a.out_scale);
  }
}

// ------------------------------------------------------------------------------ fused decode attention
// The per-head triple FDOT_NT (scores) -> ROW_SOFTMAX (causal) -> FDOT_NN (P V) of the reference's
// attention lowering, in two forms with the same bits:
//  * one workgroup per query head (attn_kernel): (1) the scores s[j] = sum16_k q[k] K[j][k] for
//    every key (16-lane groups, 16 keys per group (8 at head size 256 or up to 128 keys, 4 up to
//    64) with their K rows loaded together and their chains interleaved), kept in LDS; (2) the
//    causal softmax over them in place (as row_lds_kernel); (3) the P V chains over V staged in LDS
//    by direct global -> LDS loads in a ring of kAttnSlots stages, the first kAttnSlots - 1 of them
//    issued before the scores so that they land while (1) and (2) run.
//  * split over workgroups (attn_split_scores_kernel, then attn_split_pv_kernel): the scores of a
//    group of query heads that share one K / V head, one chunk of keys per workgroup, into a
//    scratch row per head and query row; then per 32 output columns a workgroup that recomputes
//    every query's softmax from those rows (each workgroup the same values) and runs the P V
//    chains of its columns. One workgroup per head reads all of that head's K and V through one
//    CU; the split spreads them over many.
// Each step is the contract's, in the same order as the three separate ops, so every value is the
// same bit for bit; the last head also writes its scores and probabilities where the reference's
// ops leave them.
constexpr int kAttnSlots = 6, kAttnStageBytes = 8192;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(TARS_LDS(p)));
}

// One direct global -> LDS load of the V ring (global_load_lds_dwordx4; dst is the wave-uniform LDS
// address of the 1 KiB block), written as assembly that sets M0 itself. The compiler does not see
// it as a write to LDS, so it adds no wait for every such load in flight before a later LDS read
// (which it does for the builtin, not knowing which bytes it writes); the ring's stage waits and
// barriers order the ring instead. No other code in the kernel keeps a value in M0.
__device__ __forceinline__ void ring_load16(const void* src, uint32_t dst) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "s"(dst) : "memory");
}

// The score chains of Q query rows qv against KF keys whose K elements (this lane's U of each row)
// are in kv, unflushed (qv is flushed) and checked; recomputed with the contract's flushes when a
// key element or a partial sum lies in (0, 2^-100) in magnitude (a subnormal product is then
// absorbed by its partial sum or shows in it, see kSubKeyTiny). acc receives the lane's chains.
template <int U, int KF, int Q>
__device__ __forceinline__ void score_chains(const float (&qv)[Q][U], const float (&kv)[KF][U], float (&acc)[Q][KF]) {
  uint32_t mk = ~0u;
#pragma unroll
  for (int i = 0; i < Q; ++i)
#pragma unroll
    for (int c = 0; c < KF; ++c) acc[i][c] = 0.0f;
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int i = 0; i < Q; ++i)
#pragma unroll
      for (int c = 0; c < KF; ++c) {
        const float pr = __fmul_rn(qv[i][u], kv[c][u]);
        acc[i][c] = __fadd_rn(acc[i][c], pr);
        mk = min_key(mk, kv[c][u], acc[i][c]);
      }
  if (__builtin_expect(mk < kSubKeyTiny, 0)) {
#pragma unroll
    for (int i = 0; i < Q; ++i)
#pragma unroll
      for (int c = 0; c < KF; ++c) acc[i][c] = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < Q; ++i)
#pragma unroll
        for (int c = 0; c < KF; ++c) acc[i][c] = fadd_chain(acc[i][c], fmul(qv[i][u], kv[c][u]));
  }
}

// The scores of query row m of head h: 16-lane group g takes keys g, g + 16, ..., KF of them per
// pass with their K rows loaded together and their chains interleaved.
template <int U, int KF>
__device__ __forceinline__ void attn_scores(const AttnArgs& a, int h, int m, int g, int l, bool last,
                                            const float (&qv)[1][U], float* sp) {
  const int nk = a.nk;
  for (int j0 = g; j0 < nk; j0 += 16 * KF) {
    float kv[KF][U];
#pragma unroll
    for (int c = 0; c < KF; ++c) {
      const int j = min(j0 + 16 * c, nk - 1);  // clamped: a key past the end is computed and dropped
      const float* kr = frow(a.k[h], a.ldk, j);
#pragma unroll
      for (int u = 0; u < U; ++u) kv[c][u] = kr[l + 16 * u];
    }
    float acc[1][KF];
    score_chains<U, KF, 1>(qv, kv, acc);
#pragma unroll
    for (int c = 0; c < KF; ++c) {
      const float sv = fold16(acc[0][c]);
      const int j = j0 + 16 * c;
      if (l == 0 && j < nk) {
        sp[j] = sv;
        if (last && a.sc) store_out(a.sc, m * a.ldsc, j, 0, sv, 0.0f);
      }
    }
  }
}

// The causal softmax (ROW_SOFTMAX with V of the nk values valid) of sp[0..nk) in place, by the
// whole workgroup: the fmax over the valid scores (order-free: an unsigned key, NaN beside it),
// exp_f of each difference (0 past V), the 16-lane sum, recip_f, the products. When pr is not null
// the probabilities are also stored there (fp32 row at byte offset off). Returns whether one of
// this thread's probabilities is above 1 or NaN.
__device__ __forceinline__ int softmax_lds(float* sp, int nk, int V, float* pr, int64_t off, uint32_t* red,
                                           float* bcast) {
  const int t = threadIdx.x, lane = t & 63;
  __syncthreads();  // sp complete
  uint32_t key = 0;
  int nan = 0;
  for (int j = t; j < V; j += 256) {
    if (is_nan(sp[j])) nan = 1;
    else key = max(key, fmax_key(sp[j]));
  }
  key = static_cast<uint32_t>(group_reduce<64>(static_cast<int>(key), OpMaxU{}));
  nan = group_reduce<64>(nan, OpOr{});
  if (lane == 0) red[t >> 6] = nan ? 0xFFFFFFFFu : key;
  __syncthreads();
  const uint32_t k4 = max(max(red[0], red[1]), max(red[2], red[3]));
  const float nmx = fneg(k4 == 0xFFFFFFFFu ? ffrom(kCanonNaN) : fmax_from_key(k4));
  __syncthreads();
  for (int j = t; j < nk; j += 256) sp[j] = j < V ? exp_f(fadd(sp[j], nmx)) : 0.0f;
  const float r = recip_f(lds_sum16<false, true>(sp, nk, bcast));  // exp_f values: 0, normal, inf or NaN
  int above1 = 0;
  for (int j = t; j < nk; j += 256) {
    const float p = fmul(sp[j], r);
    sp[j] = p;
    above1 |= !(p <= 1.0f);
    if (pr) store_out(pr, off, j, 0, p, 0.0f);
  }
  return above1;
}

// One ring stage's P V chain steps for output column d: the stage's rows (ROWB bytes apart in the
// slot, rows of them) times the probabilities ps[0..rows), added to acc in key order. The steps run
// unflushed and checked (a probability is an fmul output: flushed, so only V (when vtest), the
// stage's first value and the partial sums are tested, the products' flushes being absorbed, see
// kSubKeyTiny); recomputed from the stage's first value with the contract's flushes when one lies
// in (0, 2^-100) in magnitude.
template <bool VHALF, int SR, int ROWB>
__device__ __forceinline__ float pv_stage(float acc, const int8_t* slot, int d, const float* ps, int rows, bool vtest) {
  auto vval = [&](int rr) {
    return VHALF ? from_fp16_bits(reinterpret_cast<const uint16_t*>(slot + rr * ROWB)[d])
                 : reinterpret_cast<const float*>(slot + rr * ROWB)[d];
  };
  const float acc0 = acc;
  float mn = acc0 == 0.0f ? __builtin_inff() : fabsf(acc0);
  constexpr int RB = SR < 16 ? SR : 16;  // keys per block
  static_assert(RB % 4 == 0, "probabilities are read 4 at a time");
  const int nb = rows / RB;
  int rr = 0;
  // Blocks of RB keys in two register sets: block b + 1's LDS reads are issued before block b's
  // products and chain steps, so they are in flight while block b runs.
  auto blocks = [&](auto vt) {
    float va[RB], pa[RB], vb[RB], pb[RB];
    auto load = [&](float (&v)[RB], float (&p)[RB], int b) {
#pragma unroll
      for (int u = 0; u < RB; ++u) v[u] = vval(b * RB + u);
#pragma unroll
      for (int u = 0; u < RB; u += 4) {
        const float4 q4 = *reinterpret_cast<const float4*>(ps + b * RB + u);  // 16-byte aligned: SR, RB, ldp multiples of 4
        p[u] = q4.x;
        p[u + 1] = q4.y;
        p[u + 2] = q4.z;
        p[u + 3] = q4.w;
      }
    };
    auto run = [&](const float (&v)[RB], const float (&p)[RB]) {
      float pv[RB], sums[RB];
#pragma unroll
      for (int u = 0; u < RB; ++u) pv[u] = __fmul_rn(p[u], v[u]);
      if constexpr (decltype(vt)::value) {
#pragma unroll
        for (int u = 0; u < RB; u += 2) mn = min_mag(mn, v[u], v[u + 1]);
      }
#pragma unroll
      for (int u = 0; u < RB; ++u) sums[u] = acc = __fadd_rn(acc, pv[u]);
#pragma unroll
      for (int u = 0; u < RB; u += 2) mn = min_mag(mn, sums[u], sums[u + 1]);
    };
    // (the read of block b + 2 is unconditional: past the last block it reads the last one again)
    if (nb > 0) load(va, pa, 0);
    int b = 0;
    for (; b + 1 < nb; b += 2) {
      load(vb, pb, b + 1);
      run(va, pa);
      load(va, pa, min(b + 2, nb - 1));
      run(vb, pb);
    }
    if (b < nb) run(va, pa);
    rr = nb * RB;
  };
  if (vtest) blocks(std::true_type{});
  else blocks(std::false_type{});
  for (; rr < rows; ++rr) {
    const float v = vval(rr), pr = __fmul_rn(ps[rr], v);
    acc = __fadd_rn(acc, pr);
    mn = min_mag(mn, v, acc);
  }
  if (__builtin_expect(mn < kTiny, 0)) {
    acc = acc0;
    for (rr = 0; rr < rows; ++rr) acc = fadd_chain(acc, fmul(ps[rr], vval(rr)));
  }
  return acc;
}

template <int HD, bool VHALF>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
  constexpr int U = HD / 16;                                  // elements per lane of a key row
  constexpr int KF = HD <= 128 ? 16 : 8;                      // keys in flight per 16-lane group (4 up to 64 keys, 8 up to 128)
  constexpr int ES = VHALF ? 2 : 4;
  constexpr int ROWB = HD * ES;                               // bytes of one V row
  constexpr int SR = kAttnStageBytes / ROWB;                  // V rows per stage
  constexpr int IPS = kAttnStageBytes / 1024;                 // 1 KiB loads per stage (16)
  constexpr int L = IPS / 4;                                  // per wave (4)
  static_assert(ROWB <= 1024 && 1024 % ROWB == 0 && IPS % 4 == 0, "attention shape");
  __shared__ __align__(16) float sp[kAttnMaxKeys];
  __shared__ __align__(16) int8_t ring[kAttnSlots * kAttnStageBytes];
  __shared__ uint32_t red[4];
  __shared__ float bcast;
  const int h = blockIdx.x, t = threadIdx.x, g = t >> 4, l = t & 15, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const bool last = h == a.heads - 1;
  const int nk = a.nk;
  const int NS = (nk + SR - 1) / SR;
  const char* vbase = static_cast<const char*>(a.v[h]);
  auto issue = [&](int st) {
    int8_t* slot = ring + kAttnStageBytes * (st % kAttnSlots);
#pragma unroll
    for (int u = 0; u < L; ++u) {
      const int i = wave + 4 * u;
      const int byte = i * 1024 + lane * 16;
      const int row = min(st * SR + byte / ROWB, nk - 1);
      ring_load16(vbase + static_cast<int64_t>(row) * a.ldv + byte % ROWB,
                  __builtin_amdgcn_readfirstlane(lds_addr(slot + i * 1024)));
    }
  };
  for (int m = 0; m < a.M; ++m) {
    // the V ring's first stages stream in while the scores and the softmax run (V depends on neither)
#pragma unroll
    for (int st = 0; st < kAttnSlots - 1; ++st)
      if (st < NS) issue(st);
    // (1) scores
    const float* qr = frow(a.q[h], a.ldq, m);
    float qv[1][U];
#pragma unroll
    for (int u = 0; u < U; ++u) qv[0][u] = ftz(qr[l + 16 * u]);
    if (nk <= 64) attn_scores<U, 4>(a, h, m, g, l, last, qv, sp);
    else if (nk <= 128) attn_scores<U, 8>(a, h, m, g, l, last, qv, sp);
    else attn_scores<U, KF>(a, h, m, g, l, last, qv, sp);
    // (2) causal softmax in place
    const int V = a.causal_k > 0 ? min(nk, a.causal_k + m) : nk;
    const int above1 = softmax_lds(sp, nk, V, last ? a.pr : nullptr, m * a.ldpr, red, &bcast);
    wait_vmcnt<0>();  // the first V stages have landed; nothing else outstanding before the ring's counts
    // V elements need their own test only when fp32 and some probability is above 1 or NaN: with
    // every p <= 1, a subnormal V element gives |p v| < 2^-126, a subnormal product (tested) or
    // the zero of sign(p) ^ sign(v) that its flush gives too.
    const bool vtest = __syncthreads_or(above1) && !VHALF;
    // (3) P V over the V ring (its first kAttnSlots - 1 stages were issued before the scores)
    float acc = 0.0f;
    for (int st = 0; st < NS; ++st) {
      if (st + kAttnSlots - 1 < NS) issue(st + kAttnSlots - 1);
      wait_stages_ahead<L, kAttnSlots - 1>(min(NS - 1 - st, kAttnSlots - 1));
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");  // the slot's reads stay after the barrier
      if (t < HD)
        acc = pv_stage<VHALF, SR, ROWB>(acc, ring + kAttnStageBytes * (st % kAttnSlots), t, sp + st * SR,
                                        min(SR, nk - st * SR), vtest);
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of the slot are done
      __builtin_amdgcn_s_barrier();
    }
    if (t < HD) store_out(a.att[h], m * a.ldatt, t, a.out, chain_end(acc), a.out_scale);
    __syncthreads();  // sp and the ring are free for the next row
  }
}

// Split form, first kernel: workgroup (hg, c) computes the scores of the Q = group * M query rows
// of head group hg (heads hg * group .. + group - 1, which share K and V) for keys
// [c * keys_per_wg, (c + 1) * keys_per_wg): 16-lane group g takes keys g, g + 16, ... of the chunk,
// KF at a time, each K row loaded once for all Q queries. Scores go to scratch row h * M + m (and,
// for the last head, to its score rows).
// The norm and full-width RoPE (AttnNormRope) of row `row` of U * 16 values, held by one 16-lane
// group in sum16 order (lane l: elements l + 16 u): the row sums are the lane's chain and the
// fold, as the row kernels' (golden.py:358-380); each rotation partner (element n +- hd / 2) is on
// the same lane (u +- U / 2). yn: the norm's output values, yr: the RoPE's, as fp32 outputs store
// them (norm_rope_kernel's values). p may differ between the groups of a wave; fn may not.
template <int U>
__device__ __forceinline__ void group_norm_rope(const AttnNormRope& p, int fn, int row, float (&yn)[U], float (&yr)[U]) {
  static_assert(U % 2 == 0, "rotation partners on the same lane");
  const int l = threadIdx.x & 15;
  const float* x = frow(p.x, p.ldx, row);
  const float* tb = p.tab + static_cast<int64_t>(static_cast<unsigned>(row) / static_cast<unsigned>(p.rows_per_pos)) * (16 * U);
  float xv[U], gv[U], bv[U], tc[U / 2], ts[U / 2];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    xv[u] = x[l + 16 * u];
    gv[u] = p.gamma[l + 16 * u];
    bv[u] = p.beta ? p.beta[l + 16 * u] : 0.0f;
  }
#pragma unroll
  for (int u = 0; u < U / 2; ++u) {
    tc[u] = tb[l + 16 * u];
    ts[u] = tb[8 * U + l + 16 * u];
  }
  const float kinv = recip_f(i2f(16 * U));
#pragma unroll
  for (int u = 0; u < U; ++u) xv[u] = ftz(xv[u]);
  // the lane's chain: unflushed with the check of the row kernels (NONNEG: terms that never make a
  // subnormal partial sum), then the fold
  auto lane_sum = [&](const float (&t)[U], auto nonneg) {
    float acc = 0.0f;
    uint32_t mk = ~0u;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      acc = __fadd_rn(acc, t[u]);
      if constexpr (!decltype(nonneg)::value) mk = min(mk, sub_key(acc));
    }
    if constexpr (!decltype(nonneg)::value) {
      if (__builtin_expect(mk < kSubKeyNormal || is_nan(acc), 0)) {
        acc = 0.0f;
#pragma unroll
        for (int u = 0; u < U; ++u) acc = fadd_chain(acc, t[u]);
      }
    }
    return fold16(acc);
  };
  // the contract's operations written out where their wrappers are identities (as norm_row_f4): a
  // square of a flushed value is the raw product flushed (its NaN payload only feeds a sum that is
  // canonicalized at its end); the output and rotation chains take their inputs flushed once and
  // canonicalize once at the end (an intermediate NaN stays NaN to the end)
  float sq[U];
  float rs;
  if (fn == ROWFN_LAYERNORM) {
    const float nmean = fneg(fmul(lane_sum(xv, std::false_type{}), kinv));
#pragma unroll
    for (int u = 0; u < U; ++u) {
      xv[u] = fadd(xv[u], nmean);
      sq[u] = ftz(__fmul_rn(xv[u], xv[u]));
    }
    rs = rsqrt_f(fadd(fmul(lane_sum(sq, std::true_type{}), kinv), p.eps));
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) sq[u] = ftz(__fmul_rn(xv[u], xv[u]));
    const float ss = lane_sum(sq, std::true_type{});
    rs = rsqrt_f(fadd(fn == ROWFN_RMSNORM ? fmul(ss, kinv) : ss, p.eps));
  }
  // rs is canonical and never subnormal (rsqrt_f's results are 0, normal, infinite or the NaN)
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float y = ftz(__fmul_rn(ftz(__fmul_rn(xv[u], rs)), ftz(gv[u])));
    if (p.beta) y = ftz(__fadd_rn(y, ftz(bv[u])));
    yn[u] = canon(y);
  }
  // RoPE of the stored norm values: fadd(fmul(xn, tc), +-fmul(xp, ts)), flushed, canonicalized once
#pragma unroll
  for (int u = 0; u < U / 2; ++u) {
    const float c = ftz(tc[u]), sn = ftz(ts[u]);
    const float a0 = ftz(__fmul_rn(yn[u], c)), b0 = ftz(__fmul_rn(yn[u + U / 2], sn));
    const float a1 = ftz(__fmul_rn(yn[u + U / 2], c)), b1 = ftz(__fmul_rn(yn[u], sn));
    yr[u] = canon(ftz(__fadd_rn(a0, -b0)));
    yr[u + U / 2] = canon(ftz(__fadd_rn(a1, b1)));
  }
}

template <int HD, int Q, bool ROPE>
__global__ __launch_bounds__(256) void attn_split_scores_kernel(AttnArgs a) {
  constexpr int U = HD / 16, KF = 2;
  const int hg = blockIdx.x, t = threadIdx.x, g = t >> 4, l = t & 15;
  const int G = a.group, M = a.M, nk = a.nk;
  // every argument the kernel reads, in one scalar round trip (see attn_split_pv_kernel); ROPE:
  // the norm + RoPE fields too (read where first used, they measured as a wait of microseconds)
  __asm__ volatile("" : : "s"(a.q[hg * G]), "s"(a.ldq), "s"(a.k[hg * G]), "s"(a.ldk), "s"(a.keys_per_wg),
                   "s"(a.scratch), "s"(a.ld_scratch), "s"(a.heads), "s"(a.sc), "s"(a.ldsc));
  if constexpr (ROPE) {
    __asm__ volatile("" : : "s"(a.rope), "s"(a.rope_key), "s"(a.rq.x), "s"(a.rq.ldx), "s"(a.rq.gamma), "s"(a.rq.beta),
                     "s"(a.rq.eps), "s"(a.rq.fn), "s"(a.rq.n), "s"(a.rq.ldn), "s"(a.rq.tab), "s"(a.rq.rows_per_pos));
    __asm__ volatile("" : : "s"(a.rk.x), "s"(a.rk.ldx), "s"(a.rk.gamma), "s"(a.rk.beta), "s"(a.rk.eps), "s"(a.rk.fn),
                     "s"(a.rk.n), "s"(a.rk.ldn), "s"(a.rk.tab), "s"(a.rk.rows_per_pos));
  }
  const int jb = blockIdx.y * a.keys_per_wg, je = min(nk, jb + a.keys_per_wg);
  const float* kb = a.k[hg * G];
  // this 16-lane group's first key rows, issued before anything else
  auto load_keys = [&](float (&kv)[KF][U], int j0) {
#pragma unroll
    for (int c = 0; c < KF; ++c) {
      const float* kr = frow(kb, a.ldk, min(j0 + 16 * c, nk - 1));  // clamped: computed and dropped
#pragma unroll
      for (int u = 0; u < U; ++u) kv[c][u] = kr[l + 16 * u];
    }
  };
  int j0 = jb + g;
  float kv[KF][U];
  float qv[Q][U];
  if constexpr (!ROPE) {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const float* qr = frow(a.q[hg * G + i / M], a.ldq, i % M);
#pragma unroll
      for (int u = 0; u < U; ++u) qv[i][u] = ftz(qr[l + 16 * u]);
    }
  }
  load_keys(kv, j0);
  // ROPE: the new key row when this workgroup's keys include it (its loads read the cache before
  // it is written and are replaced by these values)
  const bool new_key = ROPE && jb <= a.rope_key && a.rope_key < je;
  float knew[U];
  if constexpr (ROPE) {
    // one query row per head; 16-lane group r < Q forms query row r of the group (head hg * G + r),
    // group Q the new key row (the groups of one wave run side by side), and they share the rows
    // through LDS
    __shared__ __align__(16) float rows[kAttnSplitMaxQ + 1][HD];
    const bool qrow = g < Q, krow = g == Q && new_key;
    if (qrow || krow) {
      const AttnNormRope p = qrow ? a.rq : a.rk;
      const int r = qrow ? hg * G + g : hg * G / a.rope;  // the query head, or the K / V head
      float yn[U], yr[U];
      group_norm_rope<U>(p, a.rq.fn, r, yn, yr);
#pragma unroll
      for (int u = 0; u < U; ++u) rows[g][l + 16 * u] = yr[u];
      if (krow || blockIdx.y == 0) {  // the norm's output, and the RoPE's (the query row, or the cache row)
        float* nrow = reinterpret_cast<float*>(reinterpret_cast<char*>(p.n) + r * p.ldn);
        float* orow = qrow ? const_cast<float*>(a.q[r]) : const_cast<float*>(frow(kb, a.ldk, a.rope_key));
#pragma unroll
        for (int u = 0; u < U; ++u) {
          nrow[l + 16 * u] = yn[u];
          orow[l + 16 * u] = yr[u];
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < Q; ++i)
#pragma unroll
      for (int u = 0; u < U; ++u) qv[i][u] = rows[i][l + 16 * u];
    if (new_key) {
#pragma unroll
      for (int u = 0; u < U; ++u) knew[u] = rows[Q][l + 16 * u];
    }
  }
  for (; j0 < je; j0 += 16 * KF) {
    if (new_key) {
#pragma unroll
      for (int c = 0; c < KF; ++c)
        if (j0 + 16 * c == a.rope_key) {
#pragma unroll
          for (int u = 0; u < U; ++u) kv[c][u] = knew[u];
        }
    }
    float acc[Q][KF];
    score_chains<U, KF, Q>(qv, kv, acc);
    if (j0 + 16 * KF < je) load_keys(kv, j0 + 16 * KF);  // the next rows, while these scores are stored
#pragma unroll
    for (int i = 0; i < Q; ++i)
#pragma unroll
      for (int c = 0; c < KF; ++c) {
        const float sv = fold16(acc[i][c]);
        const int j = j0 + 16 * c, h = hg * G + i / M, m = i % M;
        if (l == 0 && j < je) {
          a.scratch[(static_cast<int64_t>(h) * M + m) * a.ld_scratch + j] = sv;
          if (h == a.heads - 1 && a.sc) store_out(a.sc, m * a.ldsc, j, 0, sv, 0.0f);
        }
      }
  }
}

// The causal softmax (ROW_SOFTMAX) of Q rows of scores in LDS, in place and side by side: row i at
// sp + i * ldp is query row i % M of its head, with min(nk, causal_k + i % M) valid keys (nk when
// causal_k is 0). Every step of every row is spread over the whole workgroup, each thread taking
// the same element of every row together (independent work for the latency of exp_f), and the
// rows' 16-lane sums run together (lds_sum16_rows); each row's values are softmax_lds's. Rows from
// pr_first on also go to pr (row i - pr_first at ldpr bytes) when pr is not null. Returns whether
// one of this thread's probabilities is above 1 or NaN.
template <int Q>
__device__ __forceinline__ int softmax_rows_lds(float* sp, int ldp, int M, int nk, int causal_k, int pr_first,
                                                float* pr, int64_t ldpr, uint32_t (*red)[4], float* bcast) {
  const int t = threadIdx.x, lane = t & 63;
  int V[Q];
#pragma unroll
  for (int i = 0; i < Q; ++i) V[i] = causal_k > 0 ? min(nk, causal_k + i % M) : nk;
  __syncthreads();  // the rows are complete
  // the maximum key of each row's valid keys, a NaN counting as 0xFFFFFFFF (above every other key:
  // +inf's is 0xFF800000), branch-free, then one whole-wave maximum per row
  uint32_t key[Q];
#pragma unroll
  for (int i = 0; i < Q; ++i) key[i] = 0;
  for (int j = t; j < nk; j += 256) {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const float x = sp[i * ldp + j];
      const uint32_t k = is_nan(x) ? 0xFFFFFFFFu : fmax_key(x);
      key[i] = j < V[i] ? max(key[i], k) : key[i];
    }
  }
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    key[i] = wave_max_u32(key[i]);
    if (lane == 0) red[i][t >> 6] = key[i];
  }
  __syncthreads();
  float nmx[Q];
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    const uint32_t k4 = max(max(red[i][0], red[i][1]), max(red[i][2], red[i][3]));
    nmx[i] = fneg(k4 == 0xFFFFFFFFu ? ffrom(kCanonNaN) : fmax_from_key(k4));
  }
  for (int j = t; j < nk; j += 256) {
    float e[Q];
#pragma unroll
    for (int i = 0; i < Q; ++i) e[i] = exp_f(fadd(sp[i * ldp + j], nmx[i]));
#pragma unroll
    for (int i = 0; i < Q; ++i) sp[i * ldp + j] = j < V[i] ? e[i] : 0.0f;
  }
  lds_sum16_rows<false, true>(sp, ldp, Q, nk, bcast);  // exp_f values: 0, normal, inf or NaN
  float r[Q];
#pragma unroll
  for (int i = 0; i < Q; ++i) r[i] = recip_f(bcast[i]);
  int above1 = 0;
  for (int j = t; j < nk; j += 256) {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const float p = fmul(sp[i * ldp + j], r[i]);
      sp[i * ldp + j] = p;
      above1 |= !(p <= 1.0f);
      if (pr && i >= pr_first) store_out(pr, (i - pr_first) * ldpr, j, 0, p, 0.0f);
    }
  }
  return above1;
}

// Split form, second kernel: workgroup (hg, c) loads the scratch scores of the Q = group * M query
// rows of head group hg (Q consecutive scratch rows) into LDS by direct loads, then issues the
// first stages of a ring of direct loads of V's columns [32 c, 32 c + 32), runs the Q softmaxes
// side by side (the same probabilities in every workgroup of the group; workgroup 0 of the last
// head's group stores that head's), then the P V chains of those columns for every query row,
// one thread per (query row, column).
template <int HD, bool VHALF, int Q>
__global__ __launch_bounds__(256) void attn_split_pv_kernel(AttnArgs a) {
  constexpr int DS = kAttnSplitCols, ES = VHALF ? 2 : 4;
  constexpr int ROWB = DS * ES;                      // bytes of a V row's columns (128 / 64)
  constexpr int LPR = ROWB / 16;                     // lanes per row in a 1 KiB load
  constexpr int SB = 8192, SR = SB / ROWB;           // rows per stage
  constexpr int SLOTS = 5, L = SB / 1024 / 4;        // 1 KiB loads per wave per stage (2)
  static_assert(HD % DS == 0 && 1024 % ROWB == 0 && kAttnSplitProbs % 256 == 0, "split attention shape");
  __shared__ __align__(16) float sp[kAttnSplitProbs];
  __shared__ __align__(16) int8_t ring[SLOTS * SB];
  __shared__ uint32_t red[kAttnSplitMaxQ][4];
  __shared__ float bcast[kAttnSplitMaxQ];
  const int hg = blockIdx.x, c = blockIdx.y, t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int G = a.group, M = a.M, nk = a.nk;  // G * M == Q
  // every argument the kernel reads, in one scalar round trip: the argument block spans many cache
  // lines, and a field first read mid-kernel (the softmax's causal_k, pr, the outputs' fields)
  // stalled there for a scalar cache miss each
  __asm__ volatile("" : : "s"(a.v[hg * G]), "s"(a.ldv), "s"(a.scratch), "s"(a.ld_scratch), "s"(a.causal_k),
                   "s"(a.pr), "s"(a.ldpr), "s"(a.att[hg * G]), "s"(a.ldatt), "s"(a.out), "s"(a.out_scale));
  const int ldp = static_cast<int>(a.ld_scratch);
  const int NS = (nk + SR - 1) / SR;
  const char* vbase = static_cast<const char*>(a.v[hg * G]) + c * ROWB;
  auto issue = [&](int st) {
    int8_t* slot = ring + SB * (st % SLOTS);
#pragma unroll
    for (int u = 0; u < L; ++u) {
      const int i = wave + 4 * u;
      const int row = min(st * SR + i * (1024 / ROWB) + lane / LPR, nk - 1);
      ring_load16(vbase + static_cast<int64_t>(row) * a.ldv + 16 * (lane % LPR),
                  __builtin_amdgcn_readfirstlane(lds_addr(slot + i * 1024)));
    }
  };
  // the Q score rows (4 Q ldp bytes, contiguous in the scratch) in 1 KiB blocks; a block's lanes
  // past the end read the last 16 bytes again (into LDS past the rows, inside sp)
  const int sbytes = 4 * Q * ldp;
  const char* sbase = reinterpret_cast<const char*>(a.scratch + static_cast<int64_t>(hg) * Q * a.ld_scratch);
  for (int b = wave; 1024 * b < sbytes; b += 4)
    ring_load16(sbase + min(1024 * b + 16 * lane, sbytes - 16), __builtin_amdgcn_readfirstlane(lds_addr(sp + 256 * b)));
#pragma unroll
  for (int st = 0; st < SLOTS - 1; ++st)
    if (st < NS) issue(st);
  wait_stages_ahead<L, SLOTS - 1>(min(NS, SLOTS - 1));  // this wave's score blocks have landed
  const int pr_first = hg == gridDim.x - 1 && c == 0 ? (G - 1) * M : Q;
  const int above1 = softmax_rows_lds<Q>(sp, ldp, M, nk, a.causal_k, pr_first, a.pr, a.ldpr, red, bcast);
  wait_vmcnt<0>();  // the first V stages have landed; nothing else outstanding before the ring's counts
  // V elements need their own test only when fp32 and some probability is above 1 or NaN (as in
  // attn_kernel)
  const bool vtest = __syncthreads_or(above1) && !VHALF;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");  // the slots' reads stay after the barrier
  const int i = t / DS, d = t % DS;
  const bool active = i < Q;
  float acc = 0.0f;
  if (NS <= SLOTS - 1) {
    // every stage was issued before the softmax, has landed (each wave's wait_vmcnt<0> above) and is
    // visible (the barrier): the stages sit in consecutive slots, so the chains run over all keys in
    // one pipelined pass, without the per-stage waits and barrier pairs
    if (active) acc = pv_stage<VHALF, SR, ROWB>(acc, ring, d, sp + i * ldp, nk, vtest);
    if (active) store_out(a.att[hg * G + i / M], (i % M) * a.ldatt, c * DS + d, a.out, chain_end(acc), a.out_scale);
    return;
  }
  for (int st = 0; st < NS; ++st) {
    if (st + SLOTS - 1 < NS) issue(st + SLOTS - 1);
    wait_stages_ahead<L, SLOTS - 1>(min(NS - 1 - st, SLOTS - 1));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");  // the slot's reads stay after the barrier
    if (active)
      acc = pv_stage<VHALF, SR, ROWB>(acc, ring + SB * (st % SLOTS), d, sp + i * ldp + st * SR, min(SR, nk - st * SR),
                                      vtest);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of the slot are done
    __builtin_amdgcn_s_barrier();
  }
  if (active) store_out(a.att[hg * G + i / M], (i % M) * a.ldatt, c * DS + d, a.out, chain_end(acc), a.out_scale);
}

// Columns over grid x (per / threads each), rows over grid y with a stride loop past 65535 rows.
dim3 row_grid(int M, int N, int per) {
  return dim3(static_cast<unsigned>((N + per - 1) / per), static_cast<unsigned>(M < 65535 ? M : 65535));
}

}  // namespace

bool add_norm_supported(int M, int N) { return M >= 1 && M <= 65535 && N >= 1 && N <= kRowThreads * kRowE; }

hipError_t launch_norm_rope(const RowArgs& r, const RopeArgs& p, hipStream_t s) {
  hipLaunchKernelGGL(norm_rope_kernel, dim3(r.M), dim3(kRowThreads), 0, s, r, p, r, p, r.M);
  return hipGetLastError();
}

hipError_t launch_norm_rope2(const RowArgs& r0, const RopeArgs& p0, const RowArgs& r1, const RopeArgs& p1, hipStream_t s) {
  hipLaunchKernelGGL(norm_rope_kernel, dim3(r0.M + r1.M), dim3(kRowThreads), 0, s, r0, p0, r1, p1, r0.M);
  return hipGetLastError();
}

hipError_t launch_add_norm(const EltArgs& e, const RowArgs& r, hipStream_t s) {
  hipLaunchKernelGGL(add_norm_kernel, dim3(r.M), dim3(kRowThreads), 0, s, e, r);
  return hipGetLastError();
}

hipError_t launch_row(const RowArgs& a, hipStream_t s) {
  if (a.N <= kLdsRow)
    hipLaunchKernelGGL(row_lds_kernel, dim3(a.M), dim3(kRowThreads), 0, s, a);
  else
    hipLaunchKernelGGL(row_kernel, dim3((a.M + 15) / 16), dim3(kRowThreads), 0, s, a);
  return hipGetLastError();
}

template <int OP>
bool elt_fast(const EltArgs& a, hipStream_t s) {
  const dim3 g = row_grid(a.M, a.N, 256);
  switch (a.act) {
    case 0: hipLaunchKernelGGL((elt_fast_kernel<OP, 0>), g, dim3(256), 0, s, a); return true;
    case 3: hipLaunchKernelGGL((elt_fast_kernel<OP, 3>), g, dim3(256), 0, s, a); return true;
    case 4: hipLaunchKernelGGL((elt_fast_kernel<OP, 4>), g, dim3(256), 0, s, a); return true;
    default: return false;
  }
}

hipError_t launch_elt(const EltArgs& a, hipStream_t s) {
  // dense fp32 operands, fp32 output, no activation / GELU / SiLU: the one-batch instances
  if (!a.a_fp16 && !a.a_row && a.bmode == BMODE_DENSE && a.out == 0) {
    if (a.op == ELTOP_MUL && elt_fast<ELTOP_MUL>(a, s)) return hipGetLastError();
    if (a.op == ELTOP_ADD && elt_fast<ELTOP_ADD>(a, s)) return hipGetLastError();
    if (a.op == ELTOP_SUB && elt_fast<ELTOP_SUB>(a, s)) return hipGetLastError();
  }
  hipLaunchKernelGGL(elt_kernel, row_grid(a.M, a.N, 256), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_rope(const RopeArgs& a, hipStream_t s) {
  if (a.out == 0) {
    hipLaunchKernelGGL(rope_fast_kernel, row_grid(a.M, a.N, 256), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL(rope_kernel, row_grid(a.M, a.N, 256), dim3(256), 0, s, a);
  }
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
    hipLaunchKernelGGL(fdot_nn_kernel<true>, row_grid(a.M, a.N, kNnCols), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL(fdot_nn_kernel<false>, row_grid(a.M, a.N, kNnCols), dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace tars

namespace tars {

bool attention_supported(int hd, int nk) {
  return (hd == 64 || hd == 128 || hd == 256) && nk >= 1 && nk <= kAttnMaxKeys;
}

namespace {

// Query heads per K / V head for the split form: the largest G in {4, 2} with G * M <= 4 that
// divides the heads such that every run of G consecutive heads reads the same K and V rows, else 1.
int query_group(const AttnArgs& a) {
  for (int G : {4, 2}) {
    if (a.heads % G || G * a.M > kAttnSplitMaxQ) continue;
    bool same = true;
    for (int h = 0; h < a.heads && same; ++h) same = a.k[h] == a.k[h - h % G] && a.v[h] == a.v[h - h % G];
    if (same) return G;
  }
  return 1;
}

template <int HD, int Q>
void launch_split_q(const AttnArgs& a, dim3 gs, dim3 gp, hipStream_t s) {
  if (a.rope) hipLaunchKernelGGL((attn_split_scores_kernel<HD, Q, true>), gs, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((attn_split_scores_kernel<HD, Q, false>), gs, dim3(256), 0, s, a);
  if (a.v_fp16) hipLaunchKernelGGL((attn_split_pv_kernel<HD, true, Q>), gp, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((attn_split_pv_kernel<HD, false, Q>), gp, dim3(256), 0, s, a);
}

template <int HD>
void launch_split(const AttnArgs& a, hipStream_t s) {
  const int NG = a.heads / a.group, Q = a.group * a.M;
  const dim3 gs(NG, (a.nk + a.keys_per_wg - 1) / a.keys_per_wg), gp(NG, HD / kAttnSplitCols);
  switch (Q) {
    case 1: launch_split_q<HD, 1>(a, gs, gp, s); break;
    case 2: launch_split_q<HD, 2>(a, gs, gp, s); break;
    case 3: launch_split_q<HD, 3>(a, gs, gp, s); break;
    default: launch_split_q<HD, 4>(a, gs, gp, s); break;
  }
}

}  // namespace

float* attention_workspace(hipStream_t s) {
  // One scratch per (device, stream): work on one stream runs in order, so two calls can share a
  // scratch only when they are ordered; calls on different streams get different scratches and
  // may overlap in time. At most kMaxStreams streams per device get one; further streams (and a
  // stream that is capturing a graph when it would get its first) run the one-workgroup-per-head
  // form, which needs none.
  constexpr int kMaxDevices = 64;
  constexpr size_t kMaxStreams = 64;
  static std::mutex mu;
  static std::vector<std::pair<hipStream_t, float*>> ws[kMaxDevices];
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  for (const auto& e : ws[dev])
    if (e.first == s) return e.second;
  if (ws[dev].size() >= kMaxStreams) return nullptr;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess || st != hipStreamCaptureStatusNone) return nullptr;
  // hipMalloc outside any graph capture this thread may have open on another stream
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  (void)hipThreadExchangeStreamCaptureMode(&mode);
  void* p = nullptr;
  const hipError_t e = hipMalloc(&p, static_cast<size_t>(kAttnScratchFloats) * sizeof(float));
  (void)hipThreadExchangeStreamCaptureMode(&mode);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  ws[dev].emplace_back(s, static_cast<float*>(p));
  return static_cast<float*>(p);
}

// The scores scratch of tars_attention_noalloc: a file-scope device array (each GPU holds its own
// copy from module load until the process ends), so that entry point allocates nothing. Host code
// must not pass `scratch` itself to a kernel (on the host it names a stand-in, not device memory):
// its device address on each GPU comes from hipGetSymbolAddress, looked up once per device with
// that device current.
__device__ __align__(256) float scratch[kAttnScratchFloats];

float* attention_static_scratch() {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static float* ptr[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
      (void)hipGetLastError();
      return nullptr;
    }
    ptr[dev] = static_cast<float*>(p);
  }
  return ptr[dev];
}

bool attention_split_fits(int heads, int M, int nk, int64_t scratch_floats) {
  const int64_t ld = (nk + 3) / 4 * 4;
  return M >= 1 && M <= kAttnSplitMaxQ && M * ld <= kAttnSplitProbs && static_cast<int64_t>(heads) * M * ld <= scratch_floats;
}

hipError_t launch_attention(const AttnArgs& in, hipStream_t s) {
  const dim3 grid(in.heads), block(256);
  const bool split = in.scratch && attention_split_fits(in.heads, in.M, in.nk, in.scratch_floats);
  if (in.rope && !(split && in.M == 1 && in.hd % 32 == 0 && in.rope_key >= 0 && in.rope_key < in.nk))
    return hipErrorInvalidValue;  // split form only
  if (split) {
    // the split form: scratch rows of the scores, 32 keys per scores workgroup (more past 512 keys,
    // at most 16 chunks)
    AttnArgs a = in;
    a.ld_scratch = (a.nk + 3) / 4 * 4;
    a.group = query_group(a);
    while (a.group > 1 && a.group * a.M * a.ld_scratch > kAttnSplitProbs) a.group /= 2;
    a.keys_per_wg = 32 * ((a.nk + 511) / 512);
    if (a.hd == 64) launch_split<64>(a, s);
    else if (a.hd == 128) launch_split<128>(a, s);
    else launch_split<256>(a, s);
    return hipGetLastError();
  }
  const AttnArgs& a = in;
  if (a.hd == 64) {
    if (a.v_fp16) hipLaunchKernelGGL((attn_kernel<64, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((attn_kernel<64, false>), grid, block, 0, s, a);
  } else if (a.hd == 128) {
    if (a.v_fp16) hipLaunchKernelGGL((attn_kernel<128, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((attn_kernel<128, false>), grid, block, 0, s, a);
  } else {
    if (a.v_fp16) hipLaunchKernelGGL((attn_kernel<256, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((attn_kernel<256, false>), grid, block, 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace tars
