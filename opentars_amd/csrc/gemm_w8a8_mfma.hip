// W8A8 GEMM on INT8 MFMA (tars_mini/golden.py:326-349 for prefill rows, M >= 2).
//
// v_mfma_i32_16x16x64_i8 computes a 16x16 int32 tile over 64 k per instruction. Lane l supplies
// 16 bytes of A row (l % 16) and 16 bytes of B column (l % 16); lane l receives
// D[4 * (l / 16) + v][l % 16], v = 0..3. Which 16 bytes of K a lane supplies is free as long as A
// and B use the same map: each dot product is then the exact sum over the instruction's 64 k.
// Integer accumulation is exact, so K may be split across waves and summed in any order.
//
// Two kernel families:
//  * mfma_direct_kernel<TM, TN, KW, D>: a workgroup owns a 16 TM x 16 TN output tile and KW waves
//    that split its K range; every wave loads its share of all 16 (TM + TN) rows straight into
//    MFMA operand registers, and the int32 partial tiles meet in LDS for the golden fp32 epilogue
//    (or, for a K split, the per-block epilogue and the in-order fp32 adds across blocks). Used for
//    chunk rows (M <= 16) and for K blocks that are not a whole number of stages.
//  * mfma_staged_kernel<BM, BN, WM, WN, KS, S>: prompt rows. The tile's A and W rows are staged
//    in LDS by direct global -> LDS loads in a ring of S stages of KS bytes of K, every wave of
//    the workgroup reading the shared operands from LDS (64 x 64 tiles cut the L2 -> CU operand
//    traffic to half that of 32 x 32 tiles); each wave owns whole 16 x 16 output tiles over the
//    full K, so there is no cross-wave reduction.
//
// Roofline: at M = 4 HBM (every weight byte read once); at M = 256 the int32 MFMA work is small
// (1.6 GOP) and the kernels are bound by operand traffic from L2 into the CUs and by the fixed
// cost of launch, first loads and the fp32 output stores, with INT8 MFMA utilisation reported
// beside it.
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

// ------------------------------------------------------------------------------------ staged
// Prompt-row tiles with the operands staged in LDS by direct global -> LDS loads
// (global_load_lds_dwordx4: 64 lanes x 16 bytes land in a 1 KiB LDS block in lane order, with no
// VGPR round trip, so a wave keeps several stages of loads in flight at no register cost).
//
// LDS layout of one stage (KS bytes of K): 1 KiB blocks (g, kb), g over the 16-row groups of the
// tile's BM A rows then its BN W rows, kb over the stage's 64-byte k blocks. Lane l's 16 bytes in
// a block are row 16 g + l % 16, bytes 64 kb + 16 (l / 16) .. + 15, at offset 16 l: exactly the
// MFMA operand a lane supplies, so the MFMA reads are one contiguous ds_read_b128 per wave and
// A and W share the byte -> (instruction, lane) map.
//
// S stage slots form a ring: stage st + S - 1 is issued into the slot of stage st - 1 (free since
// the barrier that ended st - 1), then each wave waits until only its later stages' loads are
// outstanding (vmcnt counts this wave's own loads), a barrier makes every wave's loads of stage st
// visible, and the waves run its MFMAs. WM x WN waves each own TI x TJ 16 x 16 output tiles over
// the full K, so the int32 sums need no reduction; the epilogue runs in MFMA layout (D transposed:
// W is the MFMA's first operand, so lane l holds 4 consecutive columns of row l % 16) with a 4-wide
// store. K blocks (a K split) run one after another through the same pipeline, their fp32
// partials added in block order.
// Stage st of this wave's L blocks into its ring slot (st % S).
template <int L, int NW, int KS, int S>
__device__ __forceinline__ void issue_stage(int8_t* lds, const int8_t* const (&src)[L], int wave, int st) {
  int8_t* slot = lds + 1024 * NW * L * (st % S);
#pragma unroll
  for (int u = 0; u < L; ++u) stage16(src[u] + static_cast<int64_t>(KS) * st, slot + 1024 * (wave + u * NW));
}

template <int BM, int BN, int WM, int WN, int KS, int S, bool SIMPLE>
__global__ __launch_bounds__(64 * WM * WN) void mfma_staged_kernel(MfmaArgs a) {
  constexpr int NW = WM * WN, TI = BM / 16 / WM, TJ = BN / 16 / WN, GA = BM / 16, G = (BM + BN) / 16;
  constexpr int KBS = KS / 64, BLK = G * KBS, L = BLK / NW, SLOT = 1024 * BLK;
  static_assert(TI >= 1 && TJ >= 1 && BLK % NW == 0 && L * (S - 1) < 64, "stage shape");
  extern __shared__ __align__(16) int8_t lds[];  // [S][BLK] 1 KiB blocks
  // every kernel argument the first stages need (with the grid size), in one scalar round trip
  __asm__ volatile("" : : "s"(a.A), "s"(a.lda), "s"(a.nseg), "s"(a.seg[0].W), "s"(a.seg[0].K), "s"(a.seg[0].koff),
                   "s"(a.M), "s"(a.N), "s"(a.epi.scol), "s"(a.epi.srow), "s"(a.epi.bias), "s"(a.epi.scol_per_tensor),
                   "s"(gridDim.x), "s"(gridDim.y));
  const v4i zero = {0, 0, 0, 0};
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane & 15, lg = lane >> 4;
  const int mt = gridDim.y, G8 = gridDim.x * gridDim.y;
  const int b = blockIdx.y * gridDim.x + blockIdx.x;
  const int t = (G8 % 8 == 0) ? (b % 8) * (G8 / 8) + b / 8 : b;  // XCD-contiguous tiles, as above
  const int m0 = (t % mt) * BM, n0 = (t / mt) * BN;

  // Epilogue operands of this lane's outputs: rows (wm TI + i) 16 + li, columns
  // (wn TJ + j) 16 + 4 lg + v; loaded once the first stages are in flight.
  float sr[TI], sc[TJ][4], bi[TJ][4], chain[TI][TJ][4];

  for (int sgi = 0; sgi < a.nseg; ++sgi) {
    const Seg sg = sgi == 0 ? a.seg[0] : a.seg[sgi];  // the first block's fields are already loaded
    const int NS = sg.K / KS;
    // This lane's source of each block it loads. A row past the matrix is clamped to the last
    // row: it feeds only outputs that are not stored.
    const int8_t* src[L];
#pragma unroll
    for (int u = 0; u < L; ++u) {
      const int blk = wave + u * NW, g = blk / KBS, kb = blk % KBS;
      if (g < GA) {
        const int r = min(m0 + 16 * g + li, a.M - 1);
        src[u] = a.A + static_cast<int64_t>(r) * a.lda + sg.koff + 64 * kb + 16 * lg;
      } else {
        const int r = min(n0 + 16 * (g - GA) + li, a.N - 1);
        src[u] = sg.W + static_cast<int64_t>(r) * sg.K + 64 * kb + 16 * lg;
      }
    }
#pragma unroll
    for (int st = 0; st < S - 1; ++st)
      if (st < NS) issue_stage<L, NW, KS, S>(lds, src, wave, st);
    if (sgi == 0) {
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int n = min(n0 + (wn * TJ + j) * 16 + 4 * lg + v, a.N - 1);
          sc[j][v] = a.epi.load_scol(n);
          bi[j][v] = a.epi.load_bias(n);
        }
#pragma unroll
      for (int i = 0; i < TI; ++i) sr[i] = a.epi.load_srow(min(m0 + (wm * TI + i) * 16 + li, a.M - 1));
    }
    v4i acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j) acc[i][j] = zero;
    for (int st = 0; st < NS; ++st) {
      if (st + S - 1 < NS) {
        issue_stage<L, NW, KS, S>(lds, src, wave, st + S - 1);
        wait_vmcnt<L * (S - 1)>();
      } else {
        const int ahead = NS - 1 - st;  // stages issued after st (fewer than S - 1)
        if constexpr (S >= 4) {
          if (ahead == 2) wait_vmcnt<2 * L>();
        }
        if constexpr (S >= 3) {
          if (ahead == 1) wait_vmcnt<L>();
        }
        static_assert(S <= 4, "waits above cover at most 2 stages ahead");
        if (ahead == 0) wait_vmcnt<0>();
      }
      __builtin_amdgcn_s_barrier();
      const int8_t* slot = lds + SLOT * (st % S) + 16 * lane;
#pragma unroll
      for (int kb = 0; kb < KBS; ++kb) {
        v4i fa[TI], fw[TJ];
#pragma unroll
        for (int i = 0; i < TI; ++i) fa[i] = *reinterpret_cast<const v4i*>(slot + 1024 * (KBS * (wm * TI + i) + kb));
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          fw[j] = *reinterpret_cast<const v4i*>(slot + 1024 * (KBS * (GA + wn * TJ + j) + kb));
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int j = 0; j < TJ; ++j) acc[i][j] = mfma(fw[j], fa[i], acc[i][j]);
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of the slot are done
      __builtin_amdgcn_s_barrier();        // ... and every wave's, before the slot is refilled
    }
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float y = SIMPLE ? fmul(fmul(i2f(acc[i][j][v]), sr[i]), sc[j][v])
                                 : a.epi.apply(acc[i][j][v], sr[i], a.epi.srow != nullptr, sc[j][v], bi[j][v]);
          chain[i][j][v] = sgi == 0 ? y : fadd(chain[i][j][v], y);
        }
  }
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int m = m0 + (wm * TI + i) * 16 + li, n = n0 + (wn * TJ + j) * 16 + 4 * lg;
      if (m < a.M && n < a.N) {
        if constexpr (SIMPLE) {
          *reinterpret_cast<float4*>(static_cast<char*>(a.Y) + m * a.ldy + 4 * n) =
              make_float4(ftz(chain[i][j][0]), ftz(chain[i][j][1]), ftz(chain[i][j][2]), ftz(chain[i][j][3]));
        } else {
          store_out4(a.Y, m * a.ldy, n, a.epi.out, chain[i][j], a.epi.out_scale);
        }
      }
    }
}

template <int BM, int BN, int WM, int WN, int KS, int S>
hipError_t go_staged(const MfmaArgs& a, hipStream_t s) {
  constexpr size_t lds = static_cast<size_t>(S) * (BM + BN) * KS;
  static_assert(lds <= 65536, "stage ring exceeds 64 KiB of LDS");
  const dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM);
  // QM_ROWCOL with fp32 output and neither bias nor activation (every K split): the general
  // epilogue's code compiled out, as in the GEMV kernels
  const RowColEpilogue& e = a.epi;
  if (e.srow && !e.scol_per_tensor && !e.bias && e.act == 0 && e.out == 0)
    hipLaunchKernelGGL((mfma_staged_kernel<BM, BN, WM, WN, KS, S, true>), grid, dim3(64 * WM * WN), lds, s, a);
  else
    hipLaunchKernelGGL((mfma_staged_kernel<BM, BN, WM, WN, KS, S, false>), grid, dim3(64 * WM * WN), lds, s, a);
  return hipGetLastError();
}

// ------------------------------------------------------------------------------------ dispatch
// Chunk rows (M <= 16): the direct kernel with one 16-column tile per workgroup and 8 waves over
// K (the weights have no reuse, so the most workgroups and the most weight bytes in flight).
// Prompt rows: the staged kernel when every K block is a whole number of stages -- 64 x 64 tiles
// (16 waves, 128-byte stages, 4 slots) once they alone give about 192 or more workgroups, else
// 32 x 32 tiles (4 waves, 256-byte stages, 3 slots) -- and the direct kernel's 32 x 32 tiles with
// 4 waves over K otherwise. Measured on MI355X with the weights cold (rotated over 384 MiB):
// M=256 K=1024 N=3072 10.7 -> 8.0 us, M=256 K=3072 N=1024 10.6 -> 9.1 us,
// M=1024 K=1024 N=3072 28.9 -> 17.6 us, M=64 K=1024 N=3072 6.8 -> 5.6 us, bit-identical.
bool whole_stages(const MfmaArgs& a, int ks) {
  for (int i = 0; i < a.nseg; ++i)
    if (a.seg[i].K % ks) return false;
  return true;
}

hipError_t run(const MfmaArgs& a, hipStream_t s) {
  if (a.M <= 16) return go_direct<1, 1, 8, 1>(a, s);
  const int64_t tiles64 = static_cast<int64_t>((a.M + 63) / 64) * ((a.N + 63) / 64);
  if (tiles64 >= 192 && whole_stages(a, 128)) return go_staged<64, 64, 4, 4, 128, 4>(a, s);
  if (whole_stages(a, 256)) return go_staged<32, 32, 2, 2, 256, 3>(a, s);
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
