// W8A8 GEMM on INT8 MFMA (tars_mini/golden.py:326-349 for prefill rows, M >= 2).
//
// v_mfma_i32_16x16x64_i8 computes a 16x16 int32 tile over 64 k per instruction. Lane l supplies
// 16 bytes of A row (l % 16) and 16 bytes of B column (l % 16); lane l receives
// D[4 * (l / 16) + v][l % 16], v = 0..3. Which 16 bytes of K a lane supplies is free as long as A
// and B use the same map: each dot product is then the exact sum over the instruction's 64 k.
// Integer accumulation is exact, so K may be split across waves and summed in any order.
//
// One kernel family (mfma_direct_kernel<TM, TN, KW, D>): a workgroup owns a 16 TM x 16 TN output
// tile and KW waves that split its K range; every wave loads its share of all 16 (TM + TN) rows
// straight into MFMA operand registers (no LDS staging: at these sizes the operands have no reuse
// inside a workgroup once K is split across its waves), and the int32 partial tiles meet in LDS
// for the golden fp32 epilogue (or, for a K split, the per-block epilogue and the in-order fp32
// adds across blocks). Measured on MI355X against the earlier LDS-staged 64 x 64 tiles with one
// K tile in flight: M=256 K=1024 N=3072 19.2 -> 10.2 us, M=256 K=3072 N=1024 40.0 -> 10.6 us,
// M=4 K=3072 N=1024 6.6 -> 5.9 us, bit-identical outputs.
//
// Roofline: at M = 4 HBM (every weight byte read once); at M = 256 the int32 MFMA work is small
// (1.6 GOP) and the kernel is bound by operand traffic from L2 (the 32 x 32 tiles re-read A and W
// 8 and 96 times), with INT8 MFMA utilisation reported beside it.
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

__device__ __forceinline__ v4i mfma(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------------------------ direct
// MFMA operands loaded straight from global memory into registers, no LDS staging. A 128-byte K
// chunk of a 16-row tile is read as 32 contiguous bytes per lane: lane l takes row l % 16, bytes
// 32 * (l / 16) .. + 31 of the chunk; the first 16 bytes feed the chunk's first MFMA and the last
// 16 its second. A and W use the same byte -> (instruction, lane) map, so the two MFMAs together
// add every k of the chunk exactly once. The KW waves of a workgroup split the chunks (each wave
// reads its own K range of all BM + BN rows once, the next chunk in flight while the current one
// feeds the MFMAs); the int32 partial tiles meet in LDS, where each thread then owns 4 consecutive
// columns of one row for the epilogue and a 4-wide store.
// int32 pitch of a reduction row: 4 words of padding (spreads the 4 row groups of an MFMA tile
// over the banks) unless that would push the tile past 64 KiB of LDS.
constexpr int red_pitch(int kw, int bm, int bn) { return kw * bm * (bn + 4) * 4 <= 65536 ? bn + 4 : bn; }

template <int TM, int TN, int KW, int D, bool STREAM_W>
__global__ __launch_bounds__(64 * KW) void mfma_direct_kernel(MfmaArgs a) {
  constexpr int BM = 16 * TM, BN = 16 * TN;
  constexpr int LDR = red_pitch(KW, BM, BN);
  constexpr int NT = 64 * KW;
  constexpr int SLOTS = BM * BN / 4;      // 4-column groups of the tile
  constexpr int PER = (SLOTS + NT - 1) / NT;
  extern __shared__ __align__(16) int32_t red[];  // [KW][BM][LDR]
  const v4i zero = {0, 0, 0, 0};
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  // Tile order: the hardware deals workgroup ids round-robin over the 8 XCDs (id % 8). With the
  // grid a multiple of 8, XCD x gets the contiguous tile range [x * G / 8, (x + 1) * G / 8), M
  // tiles fastest, so each XCD's L2 holds 1/8 of the weight rows instead of all of them.
  const int mt = gridDim.y, G = gridDim.x * gridDim.y;
  const int b = blockIdx.y * gridDim.x + blockIdx.x;
  const int t = (G % 8 == 0) ? (b % 8) * (G / 8) + b / 8 : b;
  const int m0 = (t % mt) * BM, n0 = (t / mt) * BN;

  // Epilogue operands of this thread's slots (row scale, 4 column scales, 4 biases), fetched
  // before the K loop when a thread owns at most two slots, else when the slot is stored.
  constexpr bool PRE = PER <= 2;
  constexpr int PP = PRE ? PER : 1;
  auto operands = [&](int p, float& sr, float (&sc)[4], float (&bi)[4]) {
    const int slot = min(static_cast<int>(threadIdx.x) + p * NT, SLOTS - 1);
    const int row = slot / (BN / 4), col = (slot % (BN / 4)) * 4;
    sr = a.epi.load_srow(min(m0 + row, a.M - 1));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = min(n0 + col + q, a.N - 1);
      sc[q] = a.epi.load_scol(n);
      bi[q] = a.epi.load_bias(n);
    }
  };
  float psr[PP], psc[PP][4], pbi[PP][4], chain[PER][4];
  if constexpr (PRE) {
#pragma unroll
    for (int p = 0; p < PER; ++p) operands(p, psr[p], psc[p], pbi[p]);
  }
#pragma unroll
  for (int p = 0; p < PER; ++p)
#pragma unroll
    for (int q = 0; q < 4; ++q) chain[p][q] = 0.0f;

  for (int sgi = 0; sgi < a.nseg; ++sgi) {
    const Seg sg = a.seg[sgi];
    const int chunks = (sg.K + 127) >> 7;
    const int c0 = (chunks * wave) / KW, c1 = (chunks * (wave + 1)) / KW;
    const int8_t* arow[TM];
    const int8_t* wrow[TN];
    bool alive[TM], wlive[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = m0 + 16 * i + li;
      alive[i] = r < a.M;
      arow[i] = a.A + static_cast<int64_t>(alive[i] ? r : 0) * a.lda + sg.koff + 32 * lg;
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int r = n0 + 16 * j + li;
      wlive[j] = r < a.N;
      wrow[j] = sg.W + static_cast<int64_t>(wlive[j] ? r : 0) * sg.K + 32 * lg;
    }
    // Loads of chunk c (all lanes of a wave take the same branch-free path; a dead piece reads
    // the block's first 16 bytes and is replaced by zeros). Weights are streamed past the caches
    // only when no other workgroup reads the same rows (a single M tile).
    auto fetch = [&](int c, bool live, v4i (&fa)[TM][2], v4i (&fw)[TN][2]) {
      const int k = c * 128 + 32 * lg;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          fa[i][h] = load_pred(reinterpret_cast<const v4i*>(arow[i] + c * 128 + 16 * h),
                               reinterpret_cast<const v4i*>(a.A), live && alive[i] && k + 16 * h < sg.K, zero);
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const v4i* p = reinterpret_cast<const v4i*>(wrow[j] + c * 128 + 16 * h);
          const bool ok = live && wlive[j] && k + 16 * h < sg.K;
          fw[j][h] = STREAM_W ? load_stream_pred(p, reinterpret_cast<const v4i*>(sg.W), ok, zero)
                              : load_pred(p, reinterpret_cast<const v4i*>(sg.W), ok, zero);
        }
    };
    v4i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = zero;
    // D chunks in flight per wave: a batch of D chunk loads is issued, then its 2 * D MFMA steps.
    for (int c = c0; c < c1; c += D) {
      v4i fa[D][TM][2], fw[D][TN][2];
#pragma unroll
      for (int d = 0; d < D; ++d) fetch(c + d, c + d < c1, fa[d], fw[d]);
      issue_fence();
#pragma unroll
      for (int d = 0; d < D; ++d)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = mfma(fa[d][i][h], fw[d][j][h], acc[i][j]);
    }

    if (sgi > 0) __syncthreads();  // the previous block's epilogue has read red
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) red[(wave * BM + 16 * i + 4 * lg + v) * LDR + 16 * j + li] = acc[i][j][v];
    __syncthreads();
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int slot = static_cast<int>(threadIdx.x) + p * NT;
      const int row = slot / (BN / 4), col = (slot % (BN / 4)) * 4;
      if (SLOTS % NT == 0 || slot < SLOTS) {
        v4i sum = *reinterpret_cast<const v4i*>(red + row * LDR + col);
#pragma unroll
        for (int w = 1; w < KW; ++w) sum += *reinterpret_cast<const v4i*>(red + (w * BM + row) * LDR + col);
        const int m = m0 + row, n = n0 + col;
        float sr, sc[4], bi[4];
        if constexpr (PRE) {
          sr = psr[p];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            sc[q] = psc[p][q];
            bi[q] = pbi[p][q];
          }
        } else {
          operands(p, sr, sc, bi);
        }
        float y[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          y[q] = a.epi.apply(sum[q], sr, a.epi.srow != nullptr, sc[q], bi[q]);
          if (a.ksplit) chain[p][q] = sgi == 0 ? y[q] : fadd(chain[p][q], y[q]);
        }
        if (!a.ksplit && m < a.M && n < a.N) store_out4(a.Y, m * a.ldy, n, a.epi.out, y, a.epi.out_scale);
      }
    }
  }
  if (a.ksplit) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int slot = static_cast<int>(threadIdx.x) + p * NT;
      const int row = slot / (BN / 4), col = (slot % (BN / 4)) * 4;
      const int m = m0 + row, n = n0 + col;
      if ((SLOTS % NT == 0 || slot < SLOTS) && m < a.M && n < a.N)
        *reinterpret_cast<float4*>(static_cast<char*>(a.Y) + m * a.ldy + 4 * n) =
            make_float4(ftz(chain[p][0]), ftz(chain[p][1]), ftz(chain[p][2]), ftz(chain[p][3]));
    }
  }
}

template <int TM, int TN, int KW, int D>
hipError_t go_direct(const MfmaArgs& a, hipStream_t s) {
  constexpr int BM = 16 * TM, BN = 16 * TN;
  const dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM);
  static_assert(KW * BM * red_pitch(KW, BM, BN) * 4 <= 65536, "reduction tile exceeds 64 KiB of LDS");
  const size_t lds = static_cast<size_t>(KW) * BM * red_pitch(KW, BM, BN) * 4;
  const dim3 block(64 * KW);
  if (grid.y == 1) {
    hipLaunchKernelGGL((mfma_direct_kernel<TM, TN, KW, D, true>), grid, block, lds, s, a);
  } else {
    hipLaunchKernelGGL((mfma_direct_kernel<TM, TN, KW, D, false>), grid, block, lds, s, a);
  }
  return hipGetLastError();
}

// ------------------------------------------------------------------------------------ dispatch
// Chunk rows (M <= 16): one 16-column tile per workgroup and 8 waves over K (the weights have no
// reuse, so the most workgroups and the most weight bytes in flight). Prompt rows: 32 x 32 tiles
// and 4 waves over K, one chunk in flight per wave (the fastest of the measured 16/32/64-row x
// 16/32/64-column tiles, 2/4/8/16 waves over K, 1-4 chunk depths, and 2 x 2 / 4 x 2 waves sharing
// a 64 x 64 / 128 x 64 tile's operands through L1, at M = 256 and M = 1024).
hipError_t run(const MfmaArgs& a, hipStream_t s) {
  if (a.M <= 16) return go_direct<1, 1, 8, 1>(a, s);
  return go_direct<2, 2, 4, 1>(a, s);
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
