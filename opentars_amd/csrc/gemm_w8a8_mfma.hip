// W8A8 GEMM on INT8 MFMA (tars_mini/golden.py:326-349 for prefill rows, M >= 2).
//
// v_mfma_i32_16x16x64_i8 computes a 16x16 int32 tile over 64 k per instruction. Lane l supplies
// 16 bytes of A row (l % 16) and 16 bytes of B column (l % 16) at k = 16 * (l / 16) .. + 15 of
// the step; both operands use the same lane -> k map, so each dot product is the exact sum over
// all 64 k whatever the hardware's internal k order. Lane l receives D[4 * (l / 16) + v][l % 16],
// v = 0..3. Integer accumulation is exact, so K may be split across waves and summed in any order.
//
// Two kernels:
//  * skinny (M <= 16, K <= 4096 per block): the decode/prefill chunk (M = 4). The activation rows
//    are staged once in LDS (every wave and every column tile reuses them); weights have no reuse
//    at this M, so each wave streams its 16 weight rows straight into B fragments (16 contiguous
//    bytes per lane, 4 steps in flight). A workgroup owns 16 output columns and its waves split
//    the K steps; partial int32 tiles meet in LDS.
//  * tiled (any M): BM x BN tiles, 128-byte K tiles of A and W staged through padded LDS rows
//    (16 bytes of padding keep ds_read_b128 conflict-free), the next K tile prefetched into
//    registers while the current one feeds the MFMAs; 2 x 2 waves, each BM/2 x BN/2.
// Both run the golden fp32 epilogue per element (or, for a K split, the partial and the in-order
// fp32 adds across blocks).
//
// Roofline: at M = 4 HBM (every weight byte read once); at M = 256 still HBM on this chip's
// ~625 op/B ridge, with INT8 MFMA utilisation reported beside it.
#include "kernels.h"

namespace tars {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

struct Seg {
  const int8_t* W;
  int K;
  int koff;
};

struct MfmaArgs {
  const int8_t* A;
  int64_t lda;
  Seg seg[kMaxBlocks];
  int nseg;
  RowColEpilogue epi;  // a K split uses srow/scol only (no bias, no activation, fp32 out)
  int ksplit;
  void* Y;
  int64_t ldy;
  int M, N;
};

__device__ __forceinline__ v4i load_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
}

__device__ __forceinline__ v4i mfma(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------------------------ skinny
template <int KW>
__global__ __launch_bounds__(64 * KW) void mfma_skinny_kernel(MfmaArgs a) {
  extern __shared__ __align__(16) int8_t smem[];
  __shared__ v4i red[KW > 1 ? KW - 1 : 1][64];
  const v4i zero = {0, 0, 0, 0};
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * 16;
  float chain[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  // epilogue operands of this lane's column and rows, fetched before the weight stream
  const float sc = a.epi.load_scol(n0 + li);
  const float bi = a.epi.load_bias(n0 + li);
  float sr[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) sr[v] = a.epi.load_srow(min(lg * 4 + v, a.M - 1));

  for (int sgi = 0; sgi < a.nseg; ++sgi) {
    const Seg sg = a.seg[sgi];
    const int steps = (sg.K + 63) >> 6;
    const int ldsrow = steps * 64 + 16;
    const int cpr = steps * 4;  // 16-byte chunks per staged row
    __syncthreads();            // the previous block's readers are done with smem / red
    for (int i = threadIdx.x; i < a.M * cpr; i += 64 * KW) {
      const int r = i / cpr, c = i - r * cpr;
      v4i v = zero;
      if (c * 16 < sg.K) v = *reinterpret_cast<const v4i*>(a.A + r * a.lda + sg.koff + c * 16);
      *reinterpret_cast<v4i*>(smem + r * ldsrow + c * 16) = v;
    }
    __syncthreads();

    const int s0 = (steps * wave) / KW, s1 = (steps * (wave + 1)) / KW;
    const int8_t* wrow = sg.W + static_cast<int64_t>(n0 + li) * sg.K + lg * 16;
    const bool a_live = li < a.M;
    const int8_t* arow = smem + (a_live ? li : 0) * ldsrow + lg * 16;  // dead rows read row 0, zeroed below
    v4i acc = zero;
    int s = s0;
    for (; s + 4 <= s1; s += 4) {
      v4i b[4], x[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        b[j] = load_stream_pred(reinterpret_cast<const v4i*>(wrow + (s + j) * 64), reinterpret_cast<const v4i*>(sg.W),
                                (s + j) * 64 + lg * 16 < sg.K, zero);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v4i t = *reinterpret_cast<const v4i*>(arow + (s + j) * 64);
        x[j] = a_live ? t : zero;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = mfma(x[j], b[j], acc);
    }
    for (; s < s1; ++s) {
      const v4i b = load_stream_pred(reinterpret_cast<const v4i*>(wrow + s * 64), reinterpret_cast<const v4i*>(sg.W),
                                     s * 64 + lg * 16 < sg.K, zero);
      const v4i t = *reinterpret_cast<const v4i*>(arow + s * 64);
      const v4i x = a_live ? t : zero;
      acc = mfma(x, b, acc);
    }
    if (KW > 1) {
      if (wave > 0) red[wave - 1][lane] = acc;
      __syncthreads();
    }
    if (wave == 0) {
#pragma unroll
      for (int w = 1; w < KW; ++w) acc += red[w - 1][lane];
      const int n = n0 + li;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = lg * 4 + v;
        if (m < a.M) {
          const float y = a.epi.apply(acc[v], sr[v], a.epi.srow != nullptr, sc, bi);
          if (a.ksplit) {
            chain[v] = sgi == 0 ? y : fadd(chain[v], y);
          } else {
            store_out(a.Y, m * a.ldy, n, a.epi.out, y, a.epi.out_scale);
          }
        }
      }
    }
  }
  if (a.ksplit && wave == 0) {
    const int n = n0 + li;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = lg * 4 + v;
      if (m < a.M) reinterpret_cast<float*>(static_cast<char*>(a.Y) + m * a.ldy)[n] = ftz(chain[v]);
    }
  }
}

// ------------------------------------------------------------------------------------ tiled
constexpr int kBK = 128;          // bytes of K per LDS tile (two MFMA steps)
constexpr int kLdr = kBK + 16;    // padded LDS row

template <int BM, int BN>
__global__ __launch_bounds__(256) void mfma_tiled_kernel(MfmaArgs a) {
  constexpr int TM = BM / 32, TN = BN / 32;           // 16x16 tiles per wave (2 x 2 waves)
  constexpr int ACH = BM * (kBK / 16) / 256;           // A chunks per thread per K tile
  constexpr int WCH = BN * (kBK / 16) / 256;
  static_assert(ACH >= 1 && WCH >= 1, "tile too small for 256 threads");
  __shared__ __align__(16) int8_t As[BM * kLdr];
  __shared__ __align__(16) int8_t Ws[BN * kLdr];
  const v4i zero = {0, 0, 0, 0};
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 15, lg = lane >> 4;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  float chain[TM][TN][4];
  // epilogue operands of this lane's columns and rows, fetched before the K loop
  float sc[TN], bi[TN], sr[TM][4];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = min(n0 + (wn * TN + j) * 16 + li, a.N - 1);
    sc[j] = a.epi.load_scol(n);
    bi[j] = a.epi.load_bias(n);
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) sr[i][v] = a.epi.load_srow(min(m0 + (wm * TM + i) * 16 + lg * 4 + v, a.M - 1));

  for (int sgi = 0; sgi < a.nseg; ++sgi) {
    const Seg sg = a.seg[sgi];
    const int ktiles = (sg.K + kBK - 1) / kBK;
    v4i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = zero;

    v4i ra[ACH], rw[WCH];
    auto fetch = [&](int kt) {
#pragma unroll
      for (int t = 0; t < ACH; ++t) {
        const int i = threadIdx.x + t * 256, r = i >> 3, k = kt * kBK + (i & 7) * 16;
        ra[t] = load_pred(reinterpret_cast<const v4i*>(a.A + (m0 + r) * a.lda + sg.koff + k),
                          reinterpret_cast<const v4i*>(a.A), m0 + r < a.M && k < sg.K, zero);
      }
#pragma unroll
      for (int t = 0; t < WCH; ++t) {
        const int i = threadIdx.x + t * 256, r = i >> 3, k = kt * kBK + (i & 7) * 16;
        rw[t] = load_stream_pred(reinterpret_cast<const v4i*>(sg.W + static_cast<int64_t>(n0 + r) * sg.K + k),
                                 reinterpret_cast<const v4i*>(sg.W), n0 + r < a.N && k < sg.K, zero);
      }
    };
    fetch(0);
    for (int kt = 0; kt < ktiles; ++kt) {
      __syncthreads();
#pragma unroll
      for (int t = 0; t < ACH; ++t) {
        const int i = threadIdx.x + t * 256;
        *reinterpret_cast<v4i*>(As + (i >> 3) * kLdr + (i & 7) * 16) = ra[t];
      }
#pragma unroll
      for (int t = 0; t < WCH; ++t) {
        const int i = threadIdx.x + t * 256;
        *reinterpret_cast<v4i*>(Ws + (i >> 3) * kLdr + (i & 7) * 16) = rw[t];
      }
      __syncthreads();
      if (kt + 1 < ktiles) fetch(kt + 1);
#pragma unroll
      for (int s = 0; s < kBK / 64; ++s) {
        v4i af[TM], bf[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
          af[i] = *reinterpret_cast<const v4i*>(As + ((wm * TM + i) * 16 + li) * kLdr + s * 64 + lg * 16);
#pragma unroll
        for (int j = 0; j < TN; ++j)
          bf[j] = *reinterpret_cast<const v4i*>(Ws + ((wn * TN + j) * 16 + li) * kLdr + s * 64 + lg * 16);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma(af[i], bf[j], acc[i][j]);
      }
    }

#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + (wn * TN + j) * 16 + li;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int m = m0 + (wm * TM + i) * 16 + lg * 4 + v;
          if (m < a.M && n < a.N) {
            const float y = a.epi.apply(acc[i][j][v], sr[i][v], a.epi.srow != nullptr, sc[j], bi[j]);
            if (a.ksplit) {
              chain[i][j][v] = sgi == 0 ? y : fadd(chain[i][j][v], y);
            } else {
              store_out(a.Y, m * a.ldy, n, a.epi.out, y, a.epi.out_scale);
            }
          }
        }
      }
  }
  if (a.ksplit) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + (wn * TN + j) * 16 + li;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int m = m0 + (wm * TM + i) * 16 + lg * 4 + v;
          if (m < a.M && n < a.N)
            reinterpret_cast<float*>(static_cast<char*>(a.Y) + m * a.ldy)[n] = ftz(chain[i][j][v]);
        }
      }
  }
}

// ------------------------------------------------------------------------------------ dispatch
constexpr int kSkinnyMaxM = 16;
constexpr int kSkinnyMaxK = 4096;

hipError_t run(const MfmaArgs& a, hipStream_t s) {
  int kmax = 0;
  for (int i = 0; i < a.nseg; ++i) kmax = a.seg[i].K > kmax ? a.seg[i].K : kmax;
  if (a.M <= kSkinnyMaxM && kmax <= kSkinnyMaxK) {
    const int steps = (kmax + 63) / 64;
    const size_t lds = static_cast<size_t>(a.M) * (steps * 64 + 16);
    const dim3 grid(a.N / 16);
    if (steps >= 32) {
      hipLaunchKernelGGL(mfma_skinny_kernel<8>, grid, dim3(512), lds, s, a);
    } else {
      hipLaunchKernelGGL(mfma_skinny_kernel<4>, grid, dim3(256), lds, s, a);
    }
    return hipGetLastError();
  }
  if (a.M <= 32) {
    const dim3 grid((a.N + 63) / 64, (a.M + 31) / 32);
    hipLaunchKernelGGL((mfma_tiled_kernel<32, 64>), grid, dim3(256), 0, s, a);
  } else {
    const dim3 grid((a.N + 63) / 64, (a.M + 63) / 64);
    hipLaunchKernelGGL((mfma_tiled_kernel<64, 64>), grid, dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_w8a8_mfma(const W8A8Args& w, hipStream_t s) {
  MfmaArgs a{};
  a.A = w.A;
  a.lda = w.lda;
  a.seg[0] = Seg{w.W, w.K, 0};
  a.nseg = 1;
  a.epi = w.epi;
  a.ksplit = 0;
  a.Y = w.Y;
  a.ldy = w.ldy;
  a.M = w.M;
  a.N = w.N;
  return run(a, s);
}

hipError_t launch_gemm_w8a8_ksplit_mfma(const KSplitArgs& k, hipStream_t s) {
  MfmaArgs a{};
  a.A = k.A;
  a.lda = k.lda;
  for (int i = 0; i < k.nblocks; ++i) a.seg[i] = Seg{k.W[i], k.K[i], k.koff[i]};
  a.nseg = k.nblocks;
  a.epi = RowColEpilogue{k.srow, k.scol, 0, nullptr, 0, 0, 0.0f};
  a.ksplit = 1;
  a.Y = k.Y;
  a.ldy = k.ldy;
  a.M = k.M;
  a.N = k.N;
  return run(a, s);
}

}  // namespace tars
