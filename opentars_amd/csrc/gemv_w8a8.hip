// W8A8 GEMV (tars_mini/golden.py:326-349 at small M; the decode-step linears and the lm_head).
//
// Weight-streaming kernel: every weight byte is read from HBM exactly once. A row of W is cut into
// 16-byte chunks; a group of L lanes (L = 64 for K >= 1024) owns one row, lane `sub` taking chunks
// sub, sub + L, ... so each wave-wide load instruction reads L * 16 contiguous bytes of a row.
// Each lane keeps its activation chunks in registers (the activation row is tiny and shared by
// all rows), issues the loads of U rows back to back so U * CPL 16-byte loads are in flight, and
// accumulates with the packed signed 8-bit dot product (v_dot4, 4 MACs per instruction) into
// exact int32 sums. The L partial sums of a row are combined with DPP lane permutes (exact
// integer adds, so the order is free), and lane `u` of the group runs the fp32 epilogue for row u.
//
// Latency rules (each measured on MI355X; together 3.02 -> 2.4 us at K = 1024, N = 3072):
//  * every global load of a lane is issued back to back, activations first, then the epilogue
//    operands, then the weights, with only address arithmetic in between; values are masked after
//    the whole batch is in flight (a select placed between two loads makes the compiler wait for
//    the first before issuing the second, and an epilogue load issued after the weights waits for
//    them);
//  * the scalar epilogue fields (output pointer, formats) are pinned in SGPRs right after the
//    batch, so their kernel-argument load overlaps the weight stream instead of following it;
//  * workgroup b of n takes row block xcd_block(b, n): the workgroups of one XCD own consecutive
//    rows, so each 128-byte line of the output is written from one XCD's L2.
//
// Roofline: HBM. Algorithmic bytes per row: K (weights) + 4 (scale) + 4 (output) (+4 bias).
#include <algorithm>

#include "kernels.h"
#include "row_sums.h"

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

// CPL > 0: exactly CPL chunks per lane with the activations held in registers (K <= 128 * L).
// CPL == 0: any K, chunks walked in a loop with the activation chunk re-read from cache.
// MR activation rows per block (prefill chunks, M <= 8): every weight chunk loaded feeds the
// dot products of all MR rows, so the weights are read once per MR rows (MR * U <= L).
// The epilogue of QM_ROWCOL with fp32 output and neither bias nor activation (the decode-step
// linears and the lm_head): the golden's steps fmul(fmul(i2f(acc), srow), scol) and the output
// flush, with the general epilogue's code (every activation and output format) compiled out, which
// a cold launch otherwise fetches (measured: 0.05 - 0.2 us per launch). The contract's wrappers
// are written out where they act: i2f(acc) is 0 or at least 1 in magnitude (no flush), the scales
// are flushed (off the dependent path), each product's output is flushed, and a NaN stays NaN to
// the one canonicalization at the end.
__device__ __forceinline__ float simple_epilogue(int acc, float sr, float sc) {
  const float p = ftz(__fmul_rn(i2f(acc), ftz(sr)));
  return canon(ftz(__fmul_rn(p, ftz(sc))));
}

// Whether an epilogue is that simple one (plain GEMV: it also needs a row scale).
bool simple_epi(const RowColEpilogue& e, bool need_srow) {
  return (!need_srow || e.srow != nullptr) && !e.scol_per_tensor && !e.bias && e.act == 0 && e.out == 0;
}

// What the first loads need leads the kernel arguments as scalars (preloaded into SGPRs at wave
// launch); the epilogue's other fields follow in `a` and are read through the kernel-argument
// segment once the streams are in flight.
struct W8A8Kernargs {
  const int8_t* A;
  int64_t lda;
  const int8_t* W;
  const float* scol;
  const float* srow;
  int K, N, M, scol_per_tensor;
  W8A8Args a;
};
constexpr size_t kW8A8ArgsOffset = offsetof(W8A8Kernargs, a);
static_assert(kW8A8ArgsOffset == 56, "the preloaded scalars take 56 bytes before the argument block");

template <int L, int CPL, int U, int MR, bool SIMPLE>
__global__ __launch_bounds__(kThreads) void gemv_w8a8_kernel(const int8_t* A, int64_t lda, const int8_t* W,
                                                             const float* scol, const float* srow, int K, int N,
                                                             int M, int per_tensor, W8A8Args a) {
  static_assert(MR == 1 || CPL > 0, "several activation rows need the register-held activations");
  static_assert(MR * U <= L, "one epilogue lane per (row, weight row)");
  constexpr int kSlots = 64 / L;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int slot = lane / L;
  const int sub = lane % L;
  const int m0 = blockIdx.y * MR;
  const int C = K >> 4;
  const int bx = xcd_block(blockIdx.x, (N + kWaves * kSlots * U - 1) / (kWaves * kSlots * U));  // the grid's x extent
  const int n0 = (bx * (kWaves * kSlots) + wave * kSlots + slot) * U;
  const v4i zero = {0, 0, 0, 0};

  int acc[MR][U];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int u = 0; u < U; ++u) acc[r][u] = 0;
  // this lane's epilogue element (element e = (activation row m0 + e / U, weight row n0 + e % U))
  // and its operands: a whole-wave row group (L = 64) of up to 8 elements ends its reduction
  // scattered, element scatter_row(lane) stored by its first lane (wave_sum_scatter); otherwise
  // lane `sub` finishes element sub
  constexpr int kE = MR * U;
  constexpr bool kScatter = L == 64 && (kE == 1 || kE == 2 || kE == 4 || kE == 8);
  const int e = kScatter ? scatter_row<kScatter ? kE : 1>(lane) : sub;
  const int ne = n0 + e % U, me = m0 + e / U;
  const bool owner = kScatter ? scatter_owner<kScatter ? kE : 1>(lane) : sub < kE;
  const bool epi_lane = owner && ne < N && (MR == 1 || me < M);  // MR = 1: grid.y == M
  const int nc = epi_lane ? ne : 0, mc = epi_lane ? me : 0;
  float sr = 0.0f, sc = 0.0f, bi = 0.0f;
  // the epilogue's fields: their loads are issued after the streams and waited for at first use
  const KArg ka = kernarg_at(kW8A8ArgsOffset);
  void* Y;
  int64_t ldy;
  RowColEpilogue epi{};

  if constexpr (CPL > 0) {
    // one batch of loads: weights, activations, epilogue operands (rows past N and chunks past K
    // read the matrix start; a chunk past K is zeroed on the activation side, which zeroes its
    // products, and rows past N are never stored). The weights go first: they come from HBM and
    // are the call's long pole, nothing runs before every load of the batch has landed, and each
    // load instruction costs issue time.
    const v4i* wbase = reinterpret_cast<const v4i*>(W);
    v4i wv[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int n = n0 + u;
      const v4i* wrow = reinterpret_cast<const v4i*>(W + static_cast<int64_t>(n) * K);
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = sub + j * L;
        wv[u][j] = __builtin_nontemporal_load(n < N && c < C ? wrow + c : wbase);
      }
    }
    v4i xv[MR][CPL];
#pragma unroll
    for (int r = 0; r < MR; ++r) {
      const bool live = MR == 1 || m0 + r < M;
      const v4i* xrow = reinterpret_cast<const v4i*>(A + (live ? m0 + r : 0) * lda);
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = sub + j * L;
        xv[r][j] = *(c < C ? xrow + c : xrow);
      }
    }
    sc = scol[per_tensor ? 0 : nc];
    sr = *(srow ? srow + mc : scol);
    issue_fence();
    Y = kload<void*>(ka + offsetof(W8A8Args, Y));
    ldy = kload<int64_t>(ka + offsetof(W8A8Args, ldy));
    if constexpr (!SIMPLE) {
      const KArg ke = ka + offsetof(W8A8Args, epi);
      epi = RowColEpilogue{srow, scol, per_tensor, kload<const float*>(ke + offsetof(RowColEpilogue, bias)),
                           kload<int>(ke + offsetof(RowColEpilogue, act)), kload<int>(ke + offsetof(RowColEpilogue, out)),
                           kload<float>(ke + offsetof(RowColEpilogue, out_scale))};
      bi = *(epi.bias ? epi.bias + nc : scol);
    }
    issue_fence();
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      if (sub + j * L >= C)
#pragma unroll
        for (int r = 0; r < MR; ++r) xv[r][j] = zero;
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int j = 0; j < CPL; ++j) acc[r][u] = dot16(wv[u][j], xv[r][j], acc[r][u]);
  } else {
    sc = scol[per_tensor ? 0 : nc];
    sr = *(srow ? srow + mc : scol);
    Y = kload<void*>(ka + offsetof(W8A8Args, Y));
    ldy = kload<int64_t>(ka + offsetof(W8A8Args, ldy));
    if constexpr (!SIMPLE) {
      const KArg ke = ka + offsetof(W8A8Args, epi);
      epi = RowColEpilogue{srow, scol, per_tensor, kload<const float*>(ke + offsetof(RowColEpilogue, bias)),
                           kload<int>(ke + offsetof(RowColEpilogue, act)), kload<int>(ke + offsetof(RowColEpilogue, out)),
                           kload<float>(ke + offsetof(RowColEpilogue, out_scale))};
      bi = *(epi.bias ? epi.bias + nc : scol);
    }
    issue_fence();
    const v4i* xrow = reinterpret_cast<const v4i*>(A + m0 * lda);
    const v4i* wbase = reinterpret_cast<const v4i*>(W);
    for (int c = sub; c < C; c += L) {
      const v4i xv = xrow[c];
      v4i wv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int n = n0 + u;
        wv[u] = load_stream_pred(reinterpret_cast<const v4i*>(W + static_cast<int64_t>(n) * K) + c, wbase,
                                 n < N, zero);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) acc[0][u] = dot16(wv[u], xv, acc[0][u]);
    }
  }

  int mine = 0;
  if constexpr (kScatter) {
    int flat[kE];
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
      for (int u = 0; u < U; ++u) flat[r * U + u] = acc[r][u];
    mine = wave_sum_scatter<kE>(flat);
  } else {
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
      for (int u = 0; u < U; ++u) acc[r][u] = group_sum<L>(acc[r][u]);
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (sub == r * U + u) mine = acc[r][u];
  }
  if (epi_lane) {
    if constexpr (SIMPLE) {
      reinterpret_cast<float*>(static_cast<char*>(Y) + me * ldy)[ne] = simple_epilogue(mine, sr, sc);
    } else {
      const float y = epi.apply(mine, sr, srow != nullptr, sc, bi);
      store_out(Y, me * ldy, ne, epi.out, y, epi.out_scale);
    }
  }
}

// ---- K split in two blocks, one wave per row (the Gemma 3 down projection's 4096 + 2816) ----
// The concatenated row of both blocks is cut into 16-byte chunks like a plain row: lane `sub` takes
// chunks sub, sub + 64, ... (every chunk of the row in one batch of loads, the activation chunks
// held in registers); a chunk below C0 = K0 / 16 is block 0's (W0, rows K0 bytes apart), the rest
// block 1's (W1, rows K1 bytes apart). Each lane keeps one exact int32 sum per block and row; the
// wave's sums end scattered over the lanes (wave_sum_scatter, the block in lane bit 5), and one
// permlane32 swap hands block 1's total to the lane 32 below, which forms both blocks' fp32
// partials (i2f(acc) * srow) * scol and adds them in block order (llm.py:303-321,
// golden.py:411-412). The first loads need only the leading scalar arguments (preloaded); the
// output pointer and stride follow in `t`.
struct KSplit2Tail {
  void* Y;
  int64_t ldy;
};
struct KSplit2Kernargs {
  const int8_t *A, *W0, *W1;
  const float *scol, *srow;
  int lda, K0, K1, N;
  KSplit2Tail t;
};
static_assert(offsetof(KSplit2Kernargs, t) == 56, "the preloaded scalars take 56 bytes before the tail");

template <int CPL, int U, int NWG>
__global__ __launch_bounds__(64 * NWG) void gemv_w8a8_ksplit2_kernel(const int8_t* A, const int8_t* W0, const int8_t* W1,
                                                                     const float* scol, const float* srow, int lda,
                                                                     int K0, int K1, int N, KSplit2Tail t) {
  constexpr int kE = 2 * U;  // (row, block) sums per wave: value 2 u + b
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m = blockIdx.y;
  const int C0 = K0 >> 4, C = C0 + (K1 >> 4);
  const int bx = xcd_block(blockIdx.x, (N + NWG * U - 1) / (NWG * U));  // the grid's x extent
  const int n0 = (bx * NWG + wave) * U;
  const v4i zero = {0, 0, 0, 0};
  const int e = scatter_row<kE>(lane);
  const int ne = n0 + (e >> 1);
  const bool epi_lane = scatter_owner<kE>(lane) && (e & 1) == 0 && ne < N;
  const int nc = epi_lane ? ne : 0;

  // one batch of loads: activations, epilogue operands, weights (a chunk past the row re-reads the
  // row's last chunk and is zeroed on the activation side; a row past N re-reads row N - 1, never
  // stored). The activations go first: loads complete in issue order, so each chunk's dot can run
  // as its weights land (weights first, every dot waited for the last activation load: 3.48 ->
  // 3.72 us at C2).
  const v4i* xrow = reinterpret_cast<const v4i*>(A + static_cast<int64_t>(m) * lda);
  v4i xv[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) xv[j] = xrow[min(lane + 64 * j, C - 1)];
  const float sc = scol[nc];
  const float sr = *(srow ? srow + m : scol);
  v4i wv[U][CPL];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int n = min(n0 + u, N - 1);
    const v4i* r0 = reinterpret_cast<const v4i*>(W0 + static_cast<int64_t>(n) * K0);
    const v4i* r1 = reinterpret_cast<const v4i*>(W1 + static_cast<int64_t>(n) * K1) - C0;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = min(lane + 64 * j, C - 1);
      wv[u][j] = __builtin_nontemporal_load(c < C0 ? r0 + c : r1 + c);
    }
  }
  issue_fence();
  const KArg ka = kernarg_at(offsetof(KSplit2Kernargs, t));
  void* const Y = kload<void*>(ka + offsetof(KSplit2Tail, Y));
  const int64_t ldy = kload<int64_t>(ka + offsetof(KSplit2Tail, ldy));
  issue_fence();
#pragma unroll
  for (int j = 0; j < CPL; ++j)
    if (lane + 64 * j >= C) xv[j] = zero;
  int v[kE];
#pragma unroll
  for (int i = 0; i < kE; ++i) v[i] = 0;
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int d = dot16(wv[u][j], xv[j], 0);
      const bool first = lane + 64 * j < C0;
      v[2 * u] += first ? d : 0;
      v[2 * u + 1] += first ? 0 : d;
    }
  const int mine = wave_sum_scatter<kE>(v);
  const int other = static_cast<int>(__builtin_amdgcn_permlane32_swap(mine, mine, false, false)[1]);  // lane + 32
  if (epi_lane) {
    float y0 = i2f(mine), y1 = i2f(other);
    if (srow) {
      y0 = fmul(y0, sr);
      y1 = fmul(y1, sr);
    }
    const float y = fadd(fmul(y0, sc), fmul(y1, sc));
    reinterpret_cast<float*>(static_cast<char*>(Y) + m * ldy)[ne] = ftz(y);
  }
}

// ---- K split: blocks over consecutive column ranges of A, partials added in block order ----
template <int U>
__global__ __launch_bounds__(kThreads) void gemv_w8a8_ksplit_kernel(KSplitArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m = blockIdx.y;
  const int n0 = (blockIdx.x * kWaves + wave) * U;
  const float sr = *(a.srow ? a.srow + m : a.scol);  // unconditional (see fp32_contract.h)
  const v4i zero = {0, 0, 0, 0};
  float sc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) sc[u] = a.scol[min(n0 + u, a.N - 1)];  // fetched before the stream
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
        wv[u] = load_stream_pred(reinterpret_cast<const v4i*>(a.W[b] + static_cast<int64_t>(n) * a.K[b]) + c,
                                 reinterpret_cast<const v4i*>(a.W[b]), n < a.N, zero);
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
      part = fmul(part, sc[u]);
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

// K split with each row's chunks spread over WPR waves of the workgroup (4 / WPR rows per
// workgroup): wave part p of a row takes the 1 KiB slices p, p + WPR, ... of the concatenated row
// (lane l: chunk 64 (p + WPR j) + l, CPL of them), so a launch has WPR times the workgroups of one
// wave per row and each lane keeps only CPL loads in flight. Per block, a wave's exact int32 sum
// meets the row's other parts in LDS after one barrier (integer adds, order-free), then lane 0 of
// part 0 forms each block's partial (i2f(acc) * srow) * scol and adds them in block order.
template <int CPL, int WPR>
__global__ __launch_bounds__(kThreads) void gemv_w8a8_ksplit_rows_kernel(KSplitArgs a) {
  constexpr int kRowsPerWg = kWaves / WPR;
  __shared__ int part_sum[kWaves][kMaxBlocks];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rs = wave / WPR, kp = wave % WPR;
  const int m = blockIdx.y;
  const int n = xcd_block(blockIdx.x, gridDim.x) * kRowsPerWg + rs;
  const int nc = min(n, a.N - 1);
  const v4i zero = {0, 0, 0, 0};
  int cstart[kMaxBlocks + 1];
  cstart[0] = 0;
#pragma unroll
  for (int b = 0; b < kMaxBlocks; ++b) cstart[b + 1] = cstart[b] + (b < a.nblocks ? a.K[b] >> 4 : 0);
  const int ctot = cstart[kMaxBlocks];
  const v4i* xrow = reinterpret_cast<const v4i*>(a.A + m * a.lda);
  int blk[CPL], cin[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = min(64 * (kp + WPR * j) + lane, ctot - 1);
    int b = 0;
#pragma unroll
    for (int i = 1; i < kMaxBlocks; ++i) b += (i < a.nblocks && c >= cstart[i]) ? 1 : 0;
    blk[j] = b;
    cin[j] = c;
  }
  // one batch of loads: activations, epilogue operands, weights (every address in bounds: chunks
  // past the row re-read its last chunk and are zeroed on the activation side after the batch)
  v4i xv[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) xv[j] = xrow[cin[j]];
  const float sr = *(a.srow ? a.srow + m : a.scol);  // unconditional (see fp32_contract.h)
  const float sc = a.scol[nc];
  v4i wv[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int b = blk[j];
    const int8_t* Wb = a.W[0];
    int Kb = a.K[0], cb = 0;
#pragma unroll
    for (int i = 1; i < kMaxBlocks; ++i)
      if (b == i) {
        Wb = a.W[i];
        Kb = a.K[i];
        cb = cstart[i];
      }
    wv[j] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(Wb + static_cast<int64_t>(nc) * Kb) + (cin[j] - cb));
  }
  issue_fence();
#pragma unroll
  for (int j = 0; j < CPL; ++j)
    if (64 * (kp + WPR * j) + lane >= ctot) xv[j] = zero;
  int d[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) d[j] = dot16(wv[j], xv[j], 0);
  for (int b = 0; b < a.nblocks; ++b) {
    int acc = 0;
#pragma unroll
    for (int j = 0; j < CPL; ++j) acc += blk[j] == b ? d[j] : 0;
    acc = group_sum<64>(acc);
    if (lane == 0) part_sum[wave][b] = acc;
  }
  __syncthreads();
  if (kp == 0 && lane == 0 && n < a.N) {
    float y = 0.0f;
    for (int b = 0; b < a.nblocks; ++b) {
      int s = 0;
#pragma unroll
      for (int p = 0; p < WPR; ++p) s += part_sum[rs * WPR + p][b];
      float pb = i2f(s);
      if (a.srow) pb = fmul(pb, sr);
      pb = fmul(pb, sc);
      y = b == 0 ? pb : fadd(y, pb);
    }
    reinterpret_cast<float*>(reinterpret_cast<char*>(a.Y) + m * a.ldy)[n] = ftz(y);
  }
}

// ---- fused per-token quantizer + grouped GEMV ----
// Each workgroup quantizes the activation row once: its 256 threads read the fp32 row in float4s
// (a single pass over 4K bytes, mostly L2 hits after the first workgroup), the row maximum meets
// through wave shuffles and 4 LDS words, every thread runs the fixed recip_f sequence, and the
// q8 bytes land in LDS where each lane picks up the 16-byte chunks its dot products need; rows
// whose maximum allows it take q8's fast form (q8_fast_row). The weight loads are issued with the
// activations, so the quantizer runs under their HBM latency.
// A launch carries up to four weight matrices (pieces) of one height N, matrix z as grid z. What
// a wave needs before its loads (x, lda, the four matrix pointers, K, N) comes first among the
// kernel arguments as scalars: the library is built with kernel-argument preloading, so gfx950
// places these in SGPRs at wave launch and the activation and weight streams are issued without
// waiting for a kernel-argument load (measured 0.13 us per launch on a dependent chain). The rest
// (epilogue operands, outputs, the optional quantized-row outputs) is read from `a` after the
// streams are issued. The first workgroup of matrix 0 also stores the quantized row and its scale
// (the ROW_QUANT outputs the golden model writes).
// The kernel's arguments as laid out in the kernel-argument segment (natural alignment, in order).
struct QuantGemvKernargs {
  const float* x;
  int64_t lda;
  const int8_t* W[4];
  int K, N;
  QuantGemvArgs a;
};
constexpr size_t kQuantGemvArgsOffset = offsetof(QuantGemvKernargs, a);
static_assert(kQuantGemvArgsOffset == 56, "the preloaded scalars take 56 bytes before the argument block");

// The kernel body. NORM (quant_gemv_norm_kernel, one activation row): pB0 and pgamma are the
// prologue's residual row (x itself when there is none) and gamma, loaded before the weights so the
// norm waits for them alone; matrix 3's pointer comes from a (W3 is null).
template <int L, int CPL, int U, bool SIMPLE, bool PAIR, bool NORM>
__device__ __forceinline__ void quant_gemv_body(const float* x, int64_t lda, const int8_t* W0, const int8_t* W1,
                                                const int8_t* W2, const int8_t* W3, int K, int N, const QuantGemvArgs& a,
                                                const float* pB0, const float* pgamma) {
  extern __shared__ __align__(16) int8_t qsh[];  // the quantized row, K bytes
  __shared__ uint32_t wave_max[kWaves];
  // PAIR: a wave's U rows are U / 2 row pairs (row n of matrix 0, row n of matrix 1), for the gated
  // product; otherwise U rows of matrix z
  static_assert(!PAIR || (L == 64 && CPL > 0 && U % 2 == 0), "row pairs on whole-wave rows");
  // NORM: a.pro's residual add and norm form the quantizer's input row (whole-wave rows, K <= 2048)
  static_assert(!NORM || (L == 64 && CPL >= 1 && CPL <= 2), "norm prologue on rows of at most 2048");
  __shared__ __align__(16) float nrm[NORM ? 2 * (2048 + 64) : 4];
  constexpr int kSlots = 64 / L;
  constexpr int UR = PAIR ? U / 2 : U;          // row indices per wave
  constexpr int kRows = kWaves * kSlots * UR;  // row indices per workgroup
  const int z = blockIdx.z;
  const int8_t* W = z == 0 ? W0 : z == 1 ? W1 : z == 2 ? W2 : W3;
  if constexpr (NORM)
    if (z == 3)
      W = kload<const int8_t*>(kernarg_at(kQuantGemvArgsOffset) + offsetof(QuantGemvArgs, g) + 3 * sizeof(GemvGroup) +
                               offsetof(GemvGroup, W));
  const int nblk = (N + kRows - 1) / kRows;  // the grid's x extent
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // a scalar: row addresses on the SALU
  const int slot = lane / L;
  const int sub = lane % L;
  const int m = blockIdx.y;
  const int C = K >> 4;
  const int K4 = K >> 2;
  const int n0 = (xcd_block(blockIdx.x, nblk) * (kWaves * kSlots) + wave * kSlots + slot) * UR;
  const v4i zero = {0, 0, 0, 0};

  // one batch of loads: the fp32 activations (the quantizer waits on them alone), the weights
  // (rows past N read row N - 1 and chunks past K chunk C - 1, or with NORM the matrix start: rows
  // past N are never stored and a chunk past K meets a zero activation chunk), then the epilogue
  // operands, whose addresses come from the kernel-argument load
  constexpr int XV = CPL > 0 ? (L == 64 ? CPL : 1) : 1;  // float4s of the row per thread (K <= 1024 XV)
  const float4* xrow = reinterpret_cast<const float4*>(reinterpret_cast<const char*>(x) + m * lda);
  float4 xr[XV];
  if constexpr (CPL > 0) {
#pragma unroll
    for (int j = 0; j < XV; ++j) {
      const int i = threadIdx.x + j * kThreads;
      xr[j] = *(i < K4 ? xrow + i : xrow);
    }
  }
  // NORM: the residual row and gamma (the prologue's operands: beta, rarely present, follows the
  // weights), before the weights
  float4 rb[XV], gb[XV], bb[XV];
  if constexpr (NORM) {
#pragma unroll
    for (int j = 0; j < XV; ++j) {
      const int i = threadIdx.x + j * kThreads;
      const int ii = i < K4 ? i : 0;
      rb[j] = reinterpret_cast<const float4*>(pB0)[ii];
      gb[j] = reinterpret_cast<const float4*>(pgamma)[ii];
    }
  }
  v4i wv[U][CPL > 0 ? CPL : 1];
  if constexpr (CPL > 0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int n = n0 + (PAIR ? u % UR : u);
      const int8_t* Wu = PAIR && u >= UR ? W1 : W;
      if constexpr (NORM) {  // (measured: the clamped form below made the prologue kernels slower)
        const v4i* wrow = reinterpret_cast<const v4i*>(Wu + static_cast<int64_t>(n) * K);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          const int c = sub + j * L;
          wv[u][j] = __builtin_nontemporal_load(n < N && c < C ? wrow + c : reinterpret_cast<const v4i*>(Wu));
        }
      } else {
        const v4i* wrow = reinterpret_cast<const v4i*>(Wu + static_cast<int64_t>(min(n, N - 1)) * K);
#pragma unroll
        for (int j = 0; j < CPL; ++j) wv[u][j] = __builtin_nontemporal_load(wrow + min(sub + j * L, C - 1));
      }
    }
  }
  issue_fence();  // nothing that waits for the kernel-argument load moves above the streams
  // a whole-wave row (L = 64) ends its reduction scattered: the lane that stores row u is the
  // first lane holding u's total (wave_sum_scatter)
  // PAIR: values 2p and 2p + 1 are pair p's rows of matrices 0 and 1, which land on lanes l and
  // l ^ 32 (scatter_row's bit 0 is lane bit 5); the lane of matrix 0's row finishes the pair
  constexpr int UP = U == 6 ? 8 : U;  // six rows reduce as eight (two zero rows)
  const int eu = L == 64 ? scatter_row<UP>(lane) : sub;
  const int er = PAIR ? eu >> 1 : eu;
  const int ne = n0 + er;
  const bool epi_lane = (L == 64 ? scatter_owner<UP>(lane) : true) && (!PAIR || lane < 32) && er < UR && ne < N;
  // the epilogue operands' addresses from the kernel arguments: read here, through the
  // kernel-argument segment (volatile: the loads stay here instead of sinking to their use), and
  // waited for only after the row maximum
  KArg ka = kernarg_at(kQuantGemvArgsOffset);
  KArg kg = ka + offsetof(QuantGemvArgs, g) + z * sizeof(GemvGroup) + offsetof(GemvGroup, epi);
  const float* const scol = kload<const float*>(kg + offsetof(RowColEpilogue, scol));
  const int per_tensor = kload<int>(kg + offsetof(RowColEpilogue, scol_per_tensor));
  const float* const bias = SIMPLE ? nullptr : kload<const float*>(kg + offsetof(RowColEpilogue, bias));
  int8_t* const qout = kload<int8_t*>(ka + offsetof(QuantGemvArgs, q));  // the optional ROW_QUANT outputs
  const int64_t ldq = kload<int64_t>(ka + offsetof(QuantGemvArgs, ldq));
  KArg kg1 = ka + offsetof(QuantGemvArgs, g) + sizeof(GemvGroup) + offsetof(GemvGroup, epi);  // PAIR: matrix 1
  const float* const scol1 = PAIR ? kload<const float*>(kg1 + offsetof(RowColEpilogue, scol)) : nullptr;
  const int per_tensor1 = PAIR ? kload<int>(kg1 + offsetof(RowColEpilogue, scol_per_tensor)) : 0;
  const float* const bias1 = PAIR && !SIMPLE ? kload<const float*>(kg1 + offsetof(RowColEpilogue, bias)) : nullptr;
  // the outputs' fields, read with the others: left to their use at the end, they cost a scalar
  // cache miss there
  float* const sout = kload<float*>(ka + offsetof(QuantGemvArgs, s));
  const KArg kgz = ka + offsetof(QuantGemvArgs, g) + z * sizeof(GemvGroup);
  void* const Yz = kload<void*>(kgz + offsetof(GemvGroup, Y));
  const int64_t ldyz = kload<int64_t>(kgz + offsetof(GemvGroup, ldy));
  const RowColEpilogue epi{nullptr, scol, per_tensor, bias, SIMPLE ? 0 : kload<int>(kg + offsetof(RowColEpilogue, act)),
                           SIMPLE ? 0 : kload<int>(kg + offsetof(RowColEpilogue, out)),
                           SIMPLE ? 0.0f : kload<float>(kg + offsetof(RowColEpilogue, out_scale))};
  const KArg kgo1 = ka + offsetof(QuantGemvArgs, g) + sizeof(GemvGroup);  // PAIR: matrix 1's output, the product
  void* const Y1 = PAIR ? kload<void*>(kgo1 + offsetof(GemvGroup, Y)) : nullptr;
  const int64_t ldy1 = PAIR ? kload<int64_t>(kgo1 + offsetof(GemvGroup, ldy)) : 0;
  const RowColEpilogue epi1{nullptr, scol1, per_tensor1, bias1,
                            PAIR && !SIMPLE ? kload<int>(kg1 + offsetof(RowColEpilogue, act)) : 0, 0, 0.0f};
  float* const prod = PAIR ? kload<float*>(ka + offsetof(QuantGemvArgs, prod)) : nullptr;
  const int64_t ldprod = PAIR ? kload<int64_t>(ka + offsetof(QuantGemvArgs, ldprod)) : 0;
  float sc, bi, sc1 = 0.0f, bi1 = 0.0f;
  auto load_epilogue_operands = [&] {
    sc = scol[per_tensor || !epi_lane ? 0 : ne];
    bi = *(bias ? bias + (epi_lane ? ne : 0) : scol);
    if constexpr (PAIR) {
      sc1 = scol1[per_tensor1 || !epi_lane ? 0 : ne];
      bi1 = *(bias1 ? bias1 + (epi_lane ? ne : 0) : scol1);
    }
  };
  // NORM: the prologue's other fields and beta
  const float* pB = nullptr;
  const float* pbeta = nullptr;
  float* psum = nullptr;
  float* py = nullptr;
  int64_t ldsum = 0, ldpy = 0;
  int pfn = 0;
  float peps = 0.0f;
  if constexpr (NORM) {
    const KArg kp = ka + offsetof(QuantGemvArgs, pro);
    pB = kload<const float*>(kp + offsetof(NormPrologue, B));
    pbeta = kload<const float*>(kp + offsetof(NormPrologue, beta));
    pfn = kload<int>(kp + offsetof(NormPrologue, fn));
    peps = kload<float>(kp + offsetof(NormPrologue, eps));
    psum = kload<float*>(kp + offsetof(NormPrologue, sum));
    ldsum = kload<int64_t>(kp + offsetof(NormPrologue, ldsum));
    py = kload<float*>(kp + offsetof(NormPrologue, y));
    ldpy = kload<int64_t>(kp + offsetof(NormPrologue, ldy));
    const float4* b4 = reinterpret_cast<const float4*>(pbeta ? pbeta : pgamma);
#pragma unroll
    for (int j = 0; j < XV; ++j) {
      const int i = threadIdx.x + j * kThreads;
      bb[j] = b4[i < K4 ? i : 0];
    }
  }

  // NORM: every workgroup forms the row (ftz(x + B), or ftz(x)) and its norm; the first
  // workgroup stores both (the ELT's and the norm's outputs)
  if constexpr (NORM) {
    const bool store_pro = blockIdx.x == 0 && blockIdx.z == 0;
#pragma unroll
    for (int j = 0; j < XV; ++j) {
      const int i = threadIdx.x + j * kThreads;
      const float4 v = xr[j];
      // the ELT's sum (the contract's fadd of flushed operands), canonicalized only where it is
      // stored: the norm canonicalizes its own results
      auto add = [](float a, float c) { return ftz(__fadd_rn(ftz(a), ftz(c))); };
      xr[j] = pB ? make_float4(add(v.x, rb[j].x), add(v.y, rb[j].y), add(v.z, rb[j].z), add(v.w, rb[j].w))
                 : make_float4(ftz(v.x), ftz(v.y), ftz(v.z), ftz(v.w));
      if (pB && psum && store_pro && i < K4)
        reinterpret_cast<float4*>(reinterpret_cast<char*>(psum) + m * ldsum)[i] =
            make_float4(canon(xr[j].x), canon(xr[j].y), canon(xr[j].z), canon(xr[j].w));
    }
    norm_row_f4<XV>(pfn, K, peps, xr, gb, bb, pbeta != nullptr, nrm);
    if (py && store_pro) {
#pragma unroll
      for (int j = 0; j < XV; ++j) {
        const int i = threadIdx.x + j * kThreads;
        if (i < K4) reinterpret_cast<float4*>(reinterpret_cast<char*>(py) + m * ldpy)[i] = xr[j];
      }
    }
  }

  // the workgroup quantizes row m into LDS
  uint32_t mx = 0;
  float inv, sr;
  const bool store_q = qout != nullptr && blockIdx.x == 0 && blockIdx.z == 0;
  if constexpr (CPL > 0) {
#pragma unroll
    for (int j = 0; j < XV; ++j) {
      if (threadIdx.x + j * kThreads >= K4) xr[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      mx = max_abs_bits4(mx, xr[j]);
    }
  } else {
    for (int i = threadIdx.x; i < K4; i += kThreads) mx = max_abs_bits4(mx, xrow[i]);
  }
  mx = wave_max_u32(mx);  // DPP within rows, then permlane swaps (no lane reads)
  if (lane == 0) wave_max[wave] = mx;
  // the epilogue operands, once the activations are in (their addresses wait for the
  // kernel-argument load, which is then long done)
  load_epilogue_operands();
  __syncthreads();
  // the row maximum is uniform: one scalar value, and a branch (not a select) between the q8 forms
  mx = flush_max_bits(__builtin_amdgcn_readfirstlane(max(max(wave_max[0], wave_max[1]), max(wave_max[2], wave_max[3]))));
  quant_scales(mx, inv, sr);
  uint32_t* qw = reinterpret_cast<uint32_t*>(qsh);
  uint32_t* qg = reinterpret_cast<uint32_t*>(qout + m * ldq);
  if constexpr (CPL > 0) {
    if (q8_fast_row(mx)) {
#pragma unroll
      for (int j = 0; j < XV; ++j) {
        const int i = threadIdx.x + j * kThreads;
        const uint32_t b = q8x4_fast(xr[j].x, xr[j].y, xr[j].z, xr[j].w, inv);
        if (i < K4) {
          qw[i] = b;
          if (store_q) qg[i] = b;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < XV; ++j) {
        const int i = threadIdx.x + j * kThreads;
        const uint32_t b = q8x4(xr[j].x, xr[j].y, xr[j].z, xr[j].w, inv);
        if (i < K4) {
          qw[i] = b;
          if (store_q) qg[i] = b;
        }
      }
    }
  } else {
    for (int i = threadIdx.x; i < K4; i += kThreads) {
      const float4 v = xrow[i];
      const uint32_t b = q8x4(v.x, v.y, v.z, v.w, inv);
      qw[i] = b;
      if (store_q) qg[i] = b;
    }
  }
  if (store_q && threadIdx.x == 0) sout[m] = sr;
  __syncthreads();

  // exact int32 dot products
  int acc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) acc[u] = 0;
  const v4i* xq = reinterpret_cast<const v4i*>(qsh);
  if constexpr (CPL > 0) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = sub + j * L;
      const v4i xl = xq[c < C ? c : 0];
      const v4i xv = c < C ? xl : zero;
#pragma unroll
      for (int u = 0; u < U; ++u) acc[u] = dot16(wv[u][j], xv, acc[u]);
    }
  } else {
    for (int c = sub; c < C; c += L) {
      v4i w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int n = n0 + u;
        w[u] = load_stream_pred(reinterpret_cast<const v4i*>(W + static_cast<int64_t>(n) * K) + c,
                                reinterpret_cast<const v4i*>(W), n < N, zero);
      }
      const v4i xv = xq[c];
#pragma unroll
      for (int u = 0; u < U; ++u) acc[u] = dot16(w[u], xv, acc[u]);
    }
  }

  int mine = 0;
  int mine1 = 0;  // PAIR: the total of matrix 1's row, from lane l ^ 32
  if constexpr (L == 64) {
    int accp[UP];
#pragma unroll
    for (int u = 0; u < UP; ++u) {
      const int src = PAIR ? (u & 1) * UR + (u >> 1) : u;  // PAIR: 2p -> row p of matrix 0, 2p + 1 -> of matrix 1
      accp[u] = (PAIR ? (u >> 1) < UR : u < U) ? acc[min(src, U - 1)] : 0;
    }
    mine = wave_sum_scatter<UP>(accp);
    if constexpr (PAIR) mine1 = static_cast<int>(__builtin_amdgcn_permlane32_swap(mine, mine, false, false)[1]);
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] = group_sum<L>(acc[u]);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (sub == u) mine = acc[u];
  }
  if (epi_lane) {
    if constexpr (PAIR) {
      // both outputs fp32: the stored values are ftz(y0), ftz(y1), which fmul flushes the same way
      const float y0 = SIMPLE ? simple_epilogue(mine, sr, sc) : epi.apply(mine, sr, true, sc, bi);
      const float y1 = SIMPLE ? simple_epilogue(mine1, sr, sc1) : epi1.apply(mine1, sr, true, sc1, bi1);
      float* const y0row = reinterpret_cast<float*>(static_cast<char*>(Yz) + m * ldyz);
      float* const prow = reinterpret_cast<float*>(reinterpret_cast<char*>(prod) + m * ldprod);
      reinterpret_cast<float*>(static_cast<char*>(Y1) + m * ldy1)[ne] = ftz(y1);
      if (prow != y0row) y0row[ne] = ftz(y0);
      prow[ne] = fmul(y0, y1);
    } else if constexpr (SIMPLE) {
      reinterpret_cast<float*>(static_cast<char*>(Yz) + m * ldyz)[ne] = simple_epilogue(mine, sr, sc);
    } else {
      const float y = epi.apply(mine, sr, true, sc, bi);
      store_out(Yz, m * ldyz, ne, epi.out, y, epi.out_scale);
    }
  }
}

template <int L, int CPL, int U, bool SIMPLE, bool PAIR>
__global__ __launch_bounds__(kThreads) void quant_gemv_w8a8_kernel(const float* x, int64_t lda, const int8_t* W0,
                                                                   const int8_t* W1, const int8_t* W2,
                                                                   const int8_t* W3, int K, int N, QuantGemvArgs a) {
  quant_gemv_body<L, CPL, U, SIMPLE, PAIR, false>(x, lda, W0, W1, W2, W3, K, N, a, nullptr, nullptr);
}

// With the norm prologue (a.pro; one activation row): the residual row B (x itself when the norm
// reads x alone) and gamma lead the preloaded arguments in place of lda and matrix 3's pointer.
struct QuantGemvNormKernargs {
  const float* x;
  const float* B;
  const float* gamma;
  const int8_t* W[3];
  int K, N;
  QuantGemvArgs a;
};
static_assert(offsetof(QuantGemvNormKernargs, a) == kQuantGemvArgsOffset, "both kernels' argument blocks at 56");

template <int L, int CPL, int U, bool SIMPLE, bool PAIR>
__global__ __launch_bounds__(kThreads) void quant_gemv_norm_kernel(const float* x, const float* B, const float* gamma,
                                                                   const int8_t* W0, const int8_t* W1, const int8_t* W2,
                                                                   int K, int N, QuantGemvArgs a) {
  quant_gemv_body<L, CPL, U, SIMPLE, PAIR, true>(x, 0, W0, W1, W2, nullptr, K, N, a, B, gamma);
}

// Rows per wave (measured on MI355X with the kernels above, weights cold). A launch wants at least
// 256 workgroups (one per CU); below that, more rows per wave only lengthen each wave's chain.
// Plain GEMV: 1 row per wave below 32768 rows (K = 1024, N = 3072: 2.76 us at U = 1, 2.78 at 2,
// 3.04 at 4), 4 above (the head). Three or more activation rows (4 per workgroup row, the weight
// loads issued first): 2 rows per wave where that still leaves >= 256 workgroups, which halves
// the activation loads per weight row (M = 4, K = 1024, N = 3072: 2.83 -> 2.66 us; K = 2048,
// N = 2048: 2.99 -> 2.80 us; with 1024 rows, 2.25 / 2.66 us at U = 1 against 2.36 / 2.89 at 2).
// Rows of more than 8192 k (no activation chunks held in registers) keep one row per wave.
int plain_rows_per_wave(int64_t rows, int M, int K) {
  if (K <= 512) {
    // rows of at most 32 chunks: L = 8, 16 or 32 lanes per row, so a workgroup holds
    // kWaves * (64 / L) * U rows; the fewest rows per wave (U = 1, 2, 4, 8) that keep the grid at
    // most 1024 workgroups. Measured (weights cold): K = 512: N = 4096 M = 1 / 4 2.82 / 3.97 ->
    // 2.21 / 2.69 us, N = 16384 M = 4 4.64 -> 3.92 us, N = 32768 M = 1 4.73 -> 4.64 us; K = 256,
    // N = 4096 M = 1 2.66 -> 2.05 us; K = 128, N = 4096 M = 1 2.70 -> 2.04 us (against U = 8 at every N)
    const int L = K <= 128 ? 8 : K <= 256 ? 16 : 32;
    const int64_t per = static_cast<int64_t>(kWaves) * (64 / L);
    int u = 1;
    while (u < 8 && (rows + per * u - 1) / (per * u) > 1024) u *= 2;
    return u;
  }
  return rows >= 32768 ? 4 : (M >= 3 && rows >= 2048 && K <= 8192) ? 2 : 1;
}

// Fused quantize + GEMV: every workgroup re-quantizes the activation row, so U is the largest of
// 1, 2, 4 that still leaves >= 256 workgroups, doubled when the grid would fill one wave of
// workgroups and part of a second (256 < workgroups < 512). Measured: q/k/v (4096 rows, K = 1024)
// 3.15 us at U = 4 (3.59 at 2, 3.43 at 8); gate/up (6144 rows) 3.65 us at U = 8 (3.72 at 4),
// or six rows per wave where the chunks fit one per lane (K <= 1024): 256 workgroups, one per CU;
// o (K = 2048) and down (K = 3072), 1024 rows, 2.85 / 3.11 us at U = 1 (3.10 / 3.38 at 2); the
// head (151936 rows) 25.5 us at U = 4 (26.7 at 8).
int fused_rows_per_wave(int64_t rows, int K) {
  if (K <= 512) return 8;  // rows of at most 32 chunks: 8 rows per lane group
  int u = 1;
  while (u < 4 && rows / (kWaves * 2 * u) >= 256) u *= 2;
  const int64_t wgs = (rows + kWaves * u - 1) / (kWaves * u);
  if (wgs > 256 && wgs < 512) u = K <= 1024 && (rows + kWaves * 6 - 1) / (kWaves * 6) <= 256 ? 6 : 2 * u;
  return u;
}

// Rows per wave of the K-split loop kernel (total K > 8192).
int ksplit_rows_per_wave(int64_t rows) {
  if (rows < 16384) return 1;
  if (rows < 32768) return 2;
  return 4;
}

template <int L, int CPL, int U, bool SIMPLE>
hipError_t go(const W8A8Args& a, hipStream_t s) {
  constexpr int rows_per_block = kWaves * (64 / L) * U;
  const unsigned nb = (a.N + rows_per_block - 1) / rows_per_block;
  if constexpr (CPL > 0 && 4 * U <= L) {
    if (a.M >= 3) {
      hipLaunchKernelGGL((gemv_w8a8_kernel<L, CPL, U, 4, SIMPLE>), dim3(nb, (a.M + 3) / 4), dim3(kThreads), 0, s, a.A, a.lda,
                       a.W, a.epi.scol, a.epi.srow, a.K, a.N, a.M, a.epi.scol_per_tensor, a);
      return hipGetLastError();
    }
    if (a.M == 2) {
      hipLaunchKernelGGL((gemv_w8a8_kernel<L, CPL, U, 2, SIMPLE>), dim3(nb, 1), dim3(kThreads), 0, s, a.A, a.lda,
                       a.W, a.epi.scol, a.epi.srow, a.K, a.N, a.M, a.epi.scol_per_tensor, a);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((gemv_w8a8_kernel<L, CPL, U, 1, SIMPLE>), dim3(nb, a.M), dim3(kThreads), 0, s, a.A, a.lda,
                       a.W, a.epi.scol, a.epi.srow, a.K, a.N, a.M, a.epi.scol_per_tensor, a);
  return hipGetLastError();
}

// Output element size of an epilogue format (fp32, bf16, int8, fp16).
int out_bytes(int out) { return out == 0 ? 4 : out == 2 ? 1 : 2; }

int gcd(int a, int b) {
  while (b) {
    const int t = a % b;
    a = b;
    b = t;
  }
  return a;
}

// Matrix pieces as grid z: matrices of unequal height are cut into pieces of their greatest
// common height when that gives at most kMaxPieces pieces (q/k/v: 2048 + 1024 + 1024 rows ->
// four pieces of 1024), so every z slice has the same number of workgroups. Each launch takes up
// to four consecutive pieces of one height (the kernel's preloaded arguments hold four matrix
// pointers and one N); other shapes take more than one launch.
// Instances with row pairs (the gated product): whole-wave rows of up to four chunks per lane, one
// to three pairs per wave.
template <int L, int CPL, int U>
constexpr bool kPairs = L == 64 && CPL >= 1 && CPL <= 4 && (U == 2 || U == 4 || U == 6);

// One launch of the fused kernel, with the norm prologue when b carries one (instances exist for
// whole-wave rows of at most two chunks per lane; launch_quant_gemv_w8a8 refuses other K).
template <int L, int CPL, int U, bool SIMPLE, bool PAIR>
hipError_t launch_qg(dim3 grid, size_t lds, hipStream_t s, const int8_t* const* Wz, int N, const QuantGemvArgs& b) {
  constexpr bool kNorm = L == 64 && CPL >= 1 && CPL <= 2;
  if (b.pro.fn) {
    if constexpr (!kNorm) {
      return hipErrorInvalidValue;
    } else {
      hipLaunchKernelGGL((quant_gemv_norm_kernel<L, CPL, U, SIMPLE, PAIR>), grid, dim3(kThreads), lds, s, b.x,
                         b.pro.B ? b.pro.B : b.x, b.pro.gamma, Wz[0], Wz[1], Wz[2], b.K, N, b);
    }
  } else {
    hipLaunchKernelGGL((quant_gemv_w8a8_kernel<L, CPL, U, SIMPLE, PAIR>), grid, dim3(kThreads), lds, s, b.x, b.lda,
                       Wz[0], Wz[1], Wz[2], Wz[3], b.K, N, b);
  }
  return hipGetLastError();
}

template <int L, int CPL, int U, bool SIMPLE>
hipError_t go_fused(QuantGemvArgs& a, hipStream_t s) {
  constexpr int rows_per_block = kWaves * (64 / L) * U;
  if (a.prod) {  // two matrices of one height as row pairs, one launch, no pieces
    if constexpr (kPairs<L, CPL, U>) {
      const int N = a.g[0].N;
      const unsigned blocks = (N + kWaves * (U / 2) - 1) / (kWaves * (U / 2));
      const size_t lds = static_cast<size_t>((a.K + 15) / 16 * 16);
      const int8_t* const Wz[4] = {a.g[0].W, a.g[1].W, a.g[0].W, a.g[0].W};
      return launch_qg<L, CPL, U, SIMPLE, true>(dim3(blocks, a.M, 1), lds, s, Wz, N, a);
    }
    return hipErrorInvalidValue;
  }
  int h = 0, rows = 0;
  for (int i = 0; i < a.ngroups; ++i) {
    h = gcd(h, a.g[i].N);
    rows += a.g[i].N;
  }
  if (a.ngroups > 1 && rows / h <= kMaxPieces) {
    GemvGroup pieces[kMaxPieces];
    int np = 0;
    for (int i = 0; i < a.ngroups; ++i) {
      const GemvGroup& gi = a.g[i];
      for (int r = 0; r < gi.N; r += h) {
        GemvGroup p = gi;
        p.W = gi.W + static_cast<int64_t>(r) * a.K;
        if (!gi.epi.scol_per_tensor) p.epi.scol = gi.epi.scol + r;
        if (gi.epi.bias) p.epi.bias = gi.epi.bias + r;
        p.Y = static_cast<char*>(gi.Y) + static_cast<int64_t>(r) * out_bytes(gi.epi.out);
        p.N = h;
        pieces[np++] = p;
      }
    }
    for (int i = 0; i < np; ++i) a.g[i] = pieces[i];
    a.ngroups = np;
  }
  // launches of up to four consecutive matrices (pieces) of one height; only the first stores the
  // quantized rows and the norm prologue's outputs (outputs never overlap x, so every launch reads
  // the same row)
  const size_t lds = static_cast<size_t>((a.K + 15) / 16 * 16);
  QuantGemvArgs b = a;
  for (int first = 0; first < a.ngroups;) {
    int n = 1;
    while (first + n < a.ngroups && n < 4 && a.g[first + n].N == a.g[first].N) ++n;
    for (int i = 0; i < n; ++i) b.g[i] = a.g[first + i];
    b.ngroups = n;
    if (first > 0) {
      b.q = nullptr;
      b.s = nullptr;
      b.pro.sum = nullptr;
      b.pro.y = nullptr;
    }
    const int N = b.g[0].N;
    const int8_t* Wz[4];
    for (int i = 0; i < 4; ++i) Wz[i] = b.g[i < n ? i : 0].W;
    const unsigned blocks = (N + rows_per_block - 1) / rows_per_block;
    const hipError_t e = launch_qg<L, CPL, U, SIMPLE, false>(dim3(blocks, a.M, n), lds, s, Wz, N, b);
    if (e != hipSuccess) return e;
    first += n;
  }
  return hipSuccess;
}

// Kernel instance for (K, u): lanes per row L, 16-byte chunks per lane CPL, rows per wave U (u,
// capped by the instances that exist for the chunk count).
template <class Args, template <int, int, int> class Go>
hipError_t dispatch(Args& a, int K, int u, hipStream_t s) {
  const int C = K / 16;
  if (C <= 8)
    return u == 1 ? Go<8, 1, 1>::run(a, s) : u == 2 ? Go<8, 1, 2>::run(a, s) : u == 4 ? Go<8, 1, 4>::run(a, s)
                                                                               : Go<8, 1, 8>::run(a, s);
  if (C <= 16)
    return u == 1 ? Go<16, 1, 1>::run(a, s) : u == 2 ? Go<16, 1, 2>::run(a, s) : u == 4 ? Go<16, 1, 4>::run(a, s)
                                                                                 : Go<16, 1, 8>::run(a, s);
  if (C <= 32)
    return u == 1 ? Go<32, 1, 1>::run(a, s) : u == 2 ? Go<32, 1, 2>::run(a, s) : u == 4 ? Go<32, 1, 4>::run(a, s)
                                                                                 : Go<32, 1, 8>::run(a, s);
  switch ((C + 63) / 64) {
    case 1:
      return u == 1 ? Go<64, 1, 1>::run(a, s) : u == 2 ? Go<64, 1, 2>::run(a, s)
           : u == 4 ? Go<64, 1, 4>::run(a, s) : u == 6 ? Go<64, 1, 6>::run(a, s) : Go<64, 1, 8>::run(a, s);
    case 2:
      return u == 1 ? Go<64, 2, 1>::run(a, s) : u == 2 ? Go<64, 2, 2>::run(a, s) : Go<64, 2, 4>::run(a, s);
    case 3: return u == 1 ? Go<64, 3, 1>::run(a, s) : Go<64, 3, 2>::run(a, s);
    case 4: return u == 1 ? Go<64, 4, 1>::run(a, s) : Go<64, 4, 2>::run(a, s);
    case 5: return Go<64, 5, 1>::run(a, s);
    case 6: return Go<64, 6, 1>::run(a, s);
    case 7: return Go<64, 7, 1>::run(a, s);
    case 8: return Go<64, 8, 1>::run(a, s);
    default: return u == 1 ? Go<64, 0, 1>::run(a, s) : Go<64, 0, 4>::run(a, s);
  }
}

template <int L, int CPL, int U>
struct GoPlain {
  static hipError_t run(const W8A8Args& a, hipStream_t s) {
    return simple_epi(a.epi, true) ? go<L, CPL, U, true>(a, s) : go<L, CPL, U, false>(a, s);
  }
};
template <int L, int CPL, int U>
struct GoFused {
  static hipError_t run(QuantGemvArgs& a, hipStream_t s) {
    bool simple = true;
    for (int i = 0; i < a.ngroups; ++i) simple = simple && simple_epi(a.g[i].epi, false);
    return simple ? go_fused<L, CPL, U, true>(a, s) : go_fused<L, CPL, U, false>(a, s);
  }
};

}  // namespace

hipError_t launch_gemv_w8a8(const W8A8Args& a, hipStream_t s) {
  return dispatch<const W8A8Args, GoPlain>(a, a.K, plain_rows_per_wave(a.N, a.M, a.K), s);
}

// Consecutive matrices that continue one another (weights, column scales, biases and outputs each
// directly after the previous matrix's, one epilogue) run as one taller matrix: the same rows with
// the same arithmetic, in one launch of the full height instead of equal pieces in grid z (an
// exported lm_head's row blocks, 4 x 37984 rows of one embedding, then run as the one 151936-row
// launch the direct call gives the whole head).
static void merge_continuing(QuantGemvArgs& a) {
  int n = 0;
  for (int i = 0; i < a.ngroups; ++i) {
    const GemvGroup& c = a.g[i];
    if (n > 0) {
      GemvGroup& p = a.g[n - 1];
      const int64_t r = p.N;
      const RowColEpilogue &pe = p.epi, &ce = c.epi;
      const bool same_epi = !pe.scol_per_tensor && !ce.scol_per_tensor && pe.act == ce.act && pe.out == ce.out &&
                            pe.out_scale == ce.out_scale && (pe.bias == nullptr) == (ce.bias == nullptr);
      if (same_epi && c.W == p.W + r * a.K && ce.scol == pe.scol + r && (!pe.bias || ce.bias == pe.bias + r) &&
          c.ldy == p.ldy && c.Y == static_cast<char*>(p.Y) + r * out_bytes(pe.out) && r + c.N <= INT32_MAX) {
        p.N += c.N;
        continue;
      }
    }
    a.g[n++] = c;
  }
  a.ngroups = n;
}

hipError_t launch_quant_gemv_w8a8(QuantGemvArgs& a, hipStream_t s) {
  if (!a.prod) merge_continuing(a);
  int64_t rows = 0;
  for (int i = 0; i < a.ngroups; ++i) rows += a.g[i].N;
  int u = fused_rows_per_wave(rows, a.K);
  if (a.prod) u = u == 1 ? 2 : u == 8 ? 4 : u;  // an even number of rows: whole pairs
  if (a.pro.fn && !quant_gemv_norm_supported(a.K)) return hipErrorInvalidValue;
  return dispatch<QuantGemvArgs, GoFused>(a, a.K, u, s);
}

bool quant_gemv_pairs_supported(int K) {
  const int C = K / 16;  // whole-wave rows (more than 32 chunks), at most four chunks per lane
  return K % 16 == 0 && C > 32 && C <= 256;
}

bool quant_gemv_norm_supported(int K) {
  const int C = K / 16;  // whole-wave rows (more than 32 chunks), at most two chunks per lane, whole float4s
  return K % 64 == 0 && C > 32 && C <= 128;  // of each chain lane's terms
}

// K split up to a total K of 8192: four waves per row (measured on MI355X at C2, K = 6912 in two
// blocks, N = 1152: 4.65 us, against 5.7 us for two waves per row and for one wave per row with
// every chunk of the row in flight).
template <int CPL, int WPR>
hipError_t go_ksplit_rows(const KSplitArgs& a, hipStream_t s) {
  constexpr int rows = kWaves / WPR;
  const dim3 grid((a.N + rows - 1) / rows, a.M);
  hipLaunchKernelGGL((gemv_w8a8_ksplit_rows_kernel<CPL, WPR>), grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

// Two blocks of a total K up to 8192 (the Gemma 3 down projection): one wave per row with every
// chunk in flight (gemv_w8a8_ksplit2_kernel), ceil(N / 256) waves per workgroup (4 to 8) so the
// grid gives each CU at most one workgroup; four rows per wave past 32768 rows. Measured on MI355X
// at K = 4096 + 2816 and 3456 + 3456, N = 1152 (weights cold): 4.54 us with four waves per row
// (1152 workgroups, each reading the 6.9 KB quantized row) -> 3.84 us one row per wave in 4-wave
// workgroups (288) -> 3.49 us in 5-wave workgroups (231); 6- and 8-wave workgroups 3.53 / 3.66 us;
// two rows per wave 3.6 - 3.8 us; the activation row staged once per workgroup in LDS 3.77 us,
// and by global -> LDS loads (no VGPR round trip, one barrier) 3.58 / 3.62 us, with two rows per
// wave in 4-wave workgroups 3.36 - 3.43 / 3.46 us.
template <int CPL, int U, int NWG>
hipError_t go_ks2(const KSplitArgs& a, hipStream_t s) {
  const KSplit2Tail t{a.Y, a.ldy};
  hipLaunchKernelGGL((gemv_w8a8_ksplit2_kernel<CPL, U, NWG>), dim3((a.N + NWG * U - 1) / (NWG * U), a.M), dim3(64 * NWG),
                     0, s, a.A, a.W[0], a.W[1], a.scol, a.srow, static_cast<int>(a.lda), a.K[0], a.K[1], a.N, t);
  return hipGetLastError();
}

template <int CPL>
hipError_t go_ksplit2(const KSplitArgs& a, hipStream_t s) {
  if (a.N >= 32768) return go_ks2<CPL, 4, 4>(a, s);
  switch (std::min(8, std::max(4, (a.N + 255) / 256))) {
    case 4: return go_ks2<CPL, 1, 4>(a, s);
    case 5: return go_ks2<CPL, 1, 5>(a, s);
    case 6: return go_ks2<CPL, 1, 6>(a, s);
    default: return go_ks2<CPL, 1, 8>(a, s);
  }
}

hipError_t launch_gemv_w8a8_ksplit(const KSplitArgs& a, hipStream_t s) {
  int ctot = 0;
  for (int i = 0; i < a.nblocks; ++i) ctot += a.K[i] >> 4;
  if (a.nblocks == 2 && ctot <= 512 && a.koff[1] == a.K[0] && a.lda <= INT32_MAX) {
    switch ((ctot + 63) / 64) {
      case 1: return go_ksplit2<1>(a, s);
      case 2: return go_ksplit2<2>(a, s);
      case 3: return go_ksplit2<3>(a, s);
      case 4: return go_ksplit2<4>(a, s);
      case 5: return go_ksplit2<5>(a, s);
      case 6: return go_ksplit2<6>(a, s);
      case 7: return go_ksplit2<7>(a, s);
      default: return go_ksplit2<8>(a, s);
    }
  }
  if (ctot <= 512) return ctot <= 256 ? go_ksplit_rows<1, 4>(a, s) : go_ksplit_rows<2, 4>(a, s);
  const int u = ksplit_rows_per_wave(a.N);
  const int rows_per_block = kWaves * u;
  const dim3 grid((a.N + rows_per_block - 1) / rows_per_block, a.M);
  if (u == 1) {
    hipLaunchKernelGGL((gemv_w8a8_ksplit_kernel<1>), grid, dim3(kThreads), 0, s, a);
  } else if (u == 2) {
    hipLaunchKernelGGL((gemv_w8a8_ksplit_kernel<2>), grid, dim3(kThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL((gemv_w8a8_ksplit_kernel<4>), dim3((a.N + kWaves * 4 - 1) / (kWaves * 4), a.M), dim3(kThreads), 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace tars
