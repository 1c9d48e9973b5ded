// W8A8 GEMM on INT8 MFMA (tars_mini/golden.py:326-349 for prefill rows, M >= 2).
//
// v_mfma_i32_16x16x64_i8 computes a 16x16 int32 tile over 64 k per instruction. Lane l supplies
// 16 bytes of A row (l % 16) and 16 bytes of B column (l % 16); lane l receives
// D[4 * (l / 16) + v][l % 16], v = 0..3. Which 16 bytes of K a lane supplies is free as long as A
// and B use the same map: each dot product is then the exact sum over the instruction's 64 k.
// Integer accumulation is exact, so K may be split across waves and summed in any order.
//
// Four kernel families:
//  * mfma_chunk_kernel<KW, DB>: chunk rows (M <= 16) with one K block of whole 256-byte blocks: one
//    16 x 16 output tile per workgroup, its weight and activation rows staged in LDS by each wave
//    for its own share of K, the int32 partial tiles summed in LDS.
//  * mfma_direct_kernel<TM, TN, KW, D>: a workgroup owns a 16 TM x 16 TN output tile and KW waves
//    that split its K range; every wave loads its share of all 16 (TM + TN) rows straight into
//    MFMA operand registers, and the int32 partial tiles meet in LDS for the golden fp32 epilogue
//    (or, for a K split, the per-block epilogue and the in-order fp32 adds across blocks). Used for
//    K splits and for K blocks that are not a whole number of 256-byte stages.
//  * mfma_tile_kernel<BM, BN, WM, WN, KS, S>: prompt rows. The tile's A and W rows are staged
//    in LDS by direct global -> LDS loads of 4 rows x 256 bytes in a ring of S stages of KS bytes
//    of K, every wave of the workgroup reading the shared operands from LDS; each wave owns whole
//    16 x 16 output tiles over the full K, so there is no cross-wave reduction.
//  * mfma_panel_kernel<KQ>: prompt rows at K <= 1280 on 64 x 48 tiles. The whole K of the tile's
//    rows is resident in LDS, loaded in three phases, and each 16-column block of the output is
//    computed and stored as its weight rows land.
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

// ------------------------------------------------------------------------------------ tiles
// Prompt-row tiles with the operands staged in LDS by direct global -> LDS loads
// (global_load_lds_dwordx4: 64 lanes x 16 bytes land in a 1 KiB LDS block in lane order, with no
// VGPR round trip, so a wave keeps several stages of loads in flight at no register cost).
//
// Each 1 KiB load covers 4 rows x 256 contiguous bytes of K (16 lanes per row). Measured on
// MI355X, a tile streams from L2 into LDS twice as fast that way as with loads of 16 rows x 64
// bytes (each load then touches 4 rows' cache lines instead of 16). A stage holds KS bytes of K
// of the tile's BM A rows and BN W rows: per 16-row group, KS / 256 blocks of 16 rows x 256 bytes,
// row r of a block at byte 256 r and its 16-byte chunk c in slot c ^ r (the lane that fills slot
// s of row r reads chunk s ^ r). An MFMA operand read takes one chunk of each of 16 rows; with the
// swizzle the 16 chunks sit in 16 distinct slots, so a ds_read_b128 covers every bank once.
//
// S stage slots form a ring: stage st + S - 1 is issued into the slot of stage st - 1 (free since
// the barrier that ended st - 1), then each wave waits until only its later stages' loads are
// outstanding (vmcnt counts this wave's own loads, in issue order), a barrier makes every wave's
// loads of stage st visible, and the waves run its MFMAs. WM x WN waves each own TI x TJ 16 x 16
// output tiles over the full K, so the int32 sums need no reduction. K blocks (a K split) run one
// after another through the same ring, their fp32 partials added in block order.
//
// Latency: the fields the first loads need are the leading scalar kernel arguments (preloaded
// into SGPRs at wave launch, so no kernel-argument round trip precedes the first loads); the
// epilogue operands are loaded before the first stage (loads complete in issue order, so a load
// issued after a stage's would also have to land before the wait for that stage returns). The
// output tile goes through LDS (the ring is free after the last stage) and is stored row by row,
// consecutive threads writing consecutive 16-byte pieces of a row.

// The fields of a tile launch that its first loads do not need: the later blocks of a K split
// and the general epilogue.
struct TileTail {
  const int8_t* W[kMaxBlocks];
  int K[kMaxBlocks];
  int koff[kMaxBlocks];
  int nseg;
  const float* bias;
  int scol_per_tensor, act, out;
  float out_scale;
};

// Stage st of this wave's L blocks into its ring slot (st % S).
template <int L, int NW, int KS, int S>
__device__ __forceinline__ void issue_stage(int8_t* lds, const int8_t* const (&src)[L], int wave, int st) {
  int8_t* slot = lds + 1024 * NW * L * (st % S);
#pragma unroll
  for (int u = 0; u < L; ++u) stage16(src[u] + static_cast<int64_t>(KS) * st, slot + 1024 * (wave + u * NW));
}

template <int BM, int BN, int WM, int WN, int KS, int S, bool SIMPLE, bool KSPLIT>
__global__ __launch_bounds__(64 * WM * WN) void mfma_tile_kernel(const int8_t* A, const int8_t* W, const float* scol,
                                                                 const float* srow, int lda, int K, int M, int N, int mt,
                                                                 int ldy, void* Y, TileTail tl) {
  constexpr int NW = WM * WN, NT = 64 * NW, TI = BM / 16 / WM, TJ = BN / 16 / WN, GA = BM / 16, G = (BM + BN) / 16;
  constexpr int KQ = KS / 256, BLK = G * KQ * 4, L = BLK / NW, SLOT = 1024 * BLK;
  constexpr int TP = BN + 4;  // output tile pitch in LDS (floats; rows land on distinct banks)
  static_assert(TI >= 1 && TJ >= 1 && KS % 256 == 0 && BLK % NW == 0 && L * (S - 1) < 64, "stage shape");
  static_assert(BM * TP * 4 <= S * SLOT, "the output tile reuses the stage ring");
  __shared__ __align__(16) int8_t lds[S * SLOT];
  const v4i zero = {0, 0, 0, 0};
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane & 15, lg = lane >> 4;
  // Tile order: the hardware deals workgroup ids round-robin over the 8 XCDs (id % 8). With the
  // grid a multiple of 8, XCD x gets the contiguous tile range [x * G8 / 8, (x + 1) * G8 / 8), M
  // tiles fastest, so each XCD's L2 holds 1/8 of the weight rows instead of all of them.
  const int G8 = mt * ((N + BN - 1) / BN);
  const int b = blockIdx.x;
  const int t = (G8 % 8 == 0) ? (b % 8) * (G8 / 8) + b / 8 : b;
  const int m0 = (t % mt) * BM, n0 = (t / mt) * BN;

  // Epilogue operands of this lane's outputs: rows (wm TI + i) 16 + li, columns
  // (wn TJ + j) 16 + 4 lg + v, the four columns of a lane as one 16-byte load (every vector
  // memory instruction costs issue time, whatever its width). N % 16 == 0, so a 16-column block
  // lies wholly inside or wholly past the matrix; one past it reads the last block (its outputs
  // are not stored). A per-tensor scale (one float) and an absent bias take the general
  // instance's uniform branches instead.
  float sr[TI], sc[TJ][4], bi[TJ][4], chain[TI][TJ][4];
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int nb = min(n0 + (wn * TJ + j) * 16, N - 16) + 4 * lg;
    float4 c4, b4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (SIMPLE || !tl.scol_per_tensor) c4 = *reinterpret_cast<const float4*>(scol + nb);
    else c4 = make_float4(scol[0], scol[0], scol[0], scol[0]);
    if (!SIMPLE && tl.bias) b4 = *reinterpret_cast<const float4*>(tl.bias + nb);
    sc[j][0] = c4.x, sc[j][1] = c4.y, sc[j][2] = c4.z, sc[j][3] = c4.w;
    bi[j][0] = b4.x, bi[j][1] = b4.y, bi[j][2] = b4.z, bi[j][3] = b4.w;
  }
#pragma unroll
  for (int i = 0; i < TI; ++i) sr[i] = *(srow ? srow + min(m0 + (wm * TI + i) * 16 + li, M - 1) : scol);
  issue_fence();

  const int nseg = KSPLIT ? tl.nseg : 1;
  for (int sgi = 0; sgi < nseg; ++sgi) {
    const int8_t* Wg = (KSPLIT && sgi) ? tl.W[sgi] : W;
    const int Kg = (KSPLIT && sgi) ? tl.K[sgi] : K;
    const int ko = (KSPLIT && sgi) ? tl.koff[sgi] : 0;
    const int NS = Kg / KS;
    // This lane's source of each block it loads. A row past the matrix is clamped to the last
    // row: it feeds only outputs that are not stored.
    const int8_t* src[L];
#pragma unroll
    for (int u = 0; u < L; ++u) {
      const int i = wave + u * NW, quad = i & 3, kq = (i >> 2) % KQ, g = (i >> 2) / KQ;
      const int r = 4 * quad + lg, chunk = li ^ r;
      if (g < GA) {
        const int row = min(m0 + 16 * g + r, M - 1);
        src[u] = A + static_cast<int64_t>(row) * lda + ko + 256 * kq + 16 * chunk;
      } else {
        const int row = min(n0 + 16 * (g - GA) + r, N - 1);
        src[u] = Wg + static_cast<int64_t>(row) * Kg + 256 * kq + 16 * chunk;
      }
    }
#pragma unroll
    for (int st = 0; st < S - 1; ++st)
      if (st < NS) issue_stage<L, NW, KS, S>(lds, src, wave, st);
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
        wait_stages_ahead<L, S - 2>(NS - 1 - st);  // fewer than S - 1 stages were issued after st
      }
      __builtin_amdgcn_s_barrier();
      const int8_t* slot = lds + SLOT * (st % S) + 256 * li;
#pragma unroll
      for (int kb = 0; kb < KS / 64; ++kb) {
        const int off = 4096 * (kb / 4) + 16 * ((4 * (kb % 4) + lg) ^ li);
        v4i fa[TI], fw[TJ];
#pragma unroll
        for (int i = 0; i < TI; ++i) fa[i] = *reinterpret_cast<const v4i*>(slot + 4096 * KQ * (wm * TI + i) + off);
#pragma unroll
        for (int j = 0; j < TJ; ++j) fw[j] = *reinterpret_cast<const v4i*>(slot + 4096 * KQ * (GA + wn * TJ + j) + off);
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int j = 0; j < TJ; ++j) acc[i][j] = mfma(fw[j], fa[i], acc[i][j]);
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of the slot are done
      __builtin_amdgcn_s_barrier();        // ... and every wave's, before the slot is refilled
    }
    // W is the MFMA's first operand, so lane l holds columns 4 lg .. 4 lg + 3 of row li
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float y;
          if constexpr (SIMPLE) {
            y = fmul(fmul(i2f(acc[i][j][v]), sr[i]), sc[j][v]);
          } else {
            y = i2f(acc[i][j][v]);
            if (srow) y = fmul(y, sr[i]);
            y = fmul(y, sc[j][v]);
            if (tl.bias) y = fadd(y, bi[j][v]);
            y = act_fn(y, tl.act);
          }
          chain[i][j][v] = sgi == 0 ? y : fadd(chain[i][j][v], y);
        }
  }
  // The output tile through LDS (every wave passed the last stage's barrier, so the ring is free),
  // then stored row by row.
  float* tile = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
      *reinterpret_cast<float4*>(tile + ((wm * TI + i) * 16 + li) * TP + (wn * TJ + j) * 16 + 4 * lg) =
          make_float4(chain[i][j][0], chain[i][j][1], chain[i][j][2], chain[i][j][3]);
  __syncthreads();
  constexpr int CH = BM * BN / 4, PER = (CH + NT - 1) / NT;
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const int c = static_cast<int>(threadIdx.x) + p * NT;
    const int row = c / (BN / 4), cq = c % (BN / 4);
    const int m = m0 + row, n = n0 + 4 * cq;
    if ((CH % NT == 0 || c < CH) && m < M && n < N) {
      const float4 v = *reinterpret_cast<const float4*>(tile + row * TP + 4 * cq);
      if constexpr (SIMPLE) {
        *reinterpret_cast<float4*>(static_cast<char*>(Y) + static_cast<int64_t>(m) * ldy + 4 * n) =
            make_float4(ftz(v.x), ftz(v.y), ftz(v.z), ftz(v.w));
      } else {
        const float y4[4] = {v.x, v.y, v.z, v.w};
        store_out4(Y, static_cast<int64_t>(m) * ldy, n, tl.out, y4, tl.out_scale);
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, int KS, int S>
hipError_t go_tile(const MfmaArgs& a, hipStream_t s) {
  static_assert(static_cast<size_t>(S) * (BM + BN) * KS <= 163840, "stage ring exceeds 160 KiB of LDS");
  const int mt = (a.M + BM - 1) / BM, nt = (a.N + BN - 1) / BN;
  TileTail tl{};
  for (int i = 0; i < a.nseg; ++i) {
    tl.W[i] = a.seg[i].W;
    tl.K[i] = a.seg[i].K;
    tl.koff[i] = a.seg[i].koff;
  }
  tl.nseg = a.nseg;
  tl.bias = a.epi.bias;
  tl.scol_per_tensor = a.epi.scol_per_tensor;
  tl.act = a.epi.act;
  tl.out = a.epi.out;
  tl.out_scale = a.epi.out_scale;
  // QM_ROWCOL with fp32 output and neither bias nor activation (every K split): the general
  // epilogue's code compiled out, as in the GEMV kernels
  const RowColEpilogue& e = a.epi;
  const bool simple = e.srow && !e.scol_per_tensor && !e.bias && e.act == 0 && e.out == 0;
  const int8_t* A = a.A + a.seg[0].koff;
  const int lda = static_cast<int>(a.lda), ldy = static_cast<int>(a.ldy);
  const dim3 grid(mt * nt), block(64 * WM * WN);
#define TARS_TILE(SIMPLE, KSPLIT)                                                                                      \
  hipLaunchKernelGGL((mfma_tile_kernel<BM, BN, WM, WN, KS, S, SIMPLE, KSPLIT>), grid, block, 0, s, A, a.seg[0].W,      \
                     e.scol, e.srow, lda, a.seg[0].K, a.M, a.N, mt, ldy, a.Y, tl)
  if (a.nseg > 1) {
    if (simple) TARS_TILE(true, true);
    else TARS_TILE(false, true);
  } else {
    if (simple) TARS_TILE(true, false);
    else TARS_TILE(false, false);
  }
#undef TARS_TILE
  return hipGetLastError();
}

// ------------------------------------------------------------------------------------ panels
// 64 x 48 prompt-row tiles with the whole K (256 KQ bytes) resident in LDS. The tile's 112 rows are
// loaded in three phases, each wave issuing its loads in phase order: the 64 A rows with the first
// 16 weight rows, then the next 16 weight rows, then the last 16. The output's three 16-column
// blocks are computed and put through the epilogue as their weight rows land, and the first
// blocks' stores overlap the later loads. (Through a ring over K every output waits for the last
// stage, and the whole tile's stores leave together after it.) LDS layout, swizzle and load shape
// are mfma_tile_kernel's: 16-row groups of KQ blocks of 16 rows x 256 bytes, each global -> LDS
// load 4 rows x 256 bytes. Wave w owns output rows 16 w .. 16 w + 15 and keeps its A operands in
// registers across the three blocks.
//
// vmcnt counts stores as well as loads, so a wait for the last phase's loads also waits for every
// store issued before it to complete. Block 1's store is therefore issued after that wait (issued
// before it, the wait took ~0.2 us longer). Block 0's store goes out before block 1's work and has
// usually completed by then (deferring it past the wait as well measured the same).
// The epilogue operands are loaded after the first phase's loads, so the wait for that phase covers
// them and they do not delay its first loads.
template <int KQ, bool SIMPLE>
__global__ __launch_bounds__(256) void mfma_panel_kernel(const int8_t* A, const int8_t* W, const float* scol,
                                                        const float* srow, int lda, int K, int M, int N, int mt,
                                                        int ldy, void* Y, TileTail tl) {
  constexpr int GA = 4, GB = 3, NKB = 4 * KQ, GRP = 4096 * KQ;  // A / W 16-row groups, 64-k steps
  static_assert(KQ >= 1 && 7 * KQ < 64 && (GA + GB) * GRP <= 163840, "panel shape");
  __shared__ __align__(16) int8_t lds[(GA + GB) * GRP];
  const v4i zero = {0, 0, 0, 0};
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, lg = lane >> 4;
  // the tile order of mfma_tile_kernel: each XCD a contiguous range of tiles, M tiles fastest
  const int G8 = mt * ((N + 47) / 48);
  const int b = blockIdx.x;
  const int t = (G8 % 8 == 0) ? (b % 8) * (G8 / 8) + b / 8 : b;
  const int m0 = (t % mt) * 64, n0 = (t / mt) * 48;
  const int m = m0 + 16 * wave + li;  // this lane's output row

  // This wave's load u: 16-row group u / KQ (A groups first), K block u % KQ, rows 4 wave .. + 3
  // of the group (lane: row 4 wave + lg, 16-byte chunk li ^ row), landing at LDS byte
  // 1024 (4 u + wave). Rows past the matrix are clamped to its last row: they feed only outputs
  // that are not stored.
  auto load = [&](int u) {
    const int g = u / KQ, kq = u % KQ, r = 4 * wave + lg;
    const int8_t* row = g < GA ? A + static_cast<int64_t>(min(m0 + 16 * g + r, M - 1)) * lda
                               : W + static_cast<int64_t>(min(n0 + 16 * (g - GA) + r, N - 1)) * K;
    stage16(row + 256 * kq + 16 * (li ^ r), lds + 1024 * (4 * u + wave));
  };
#pragma unroll
  for (int u = 0; u < (GA + 1) * KQ; ++u) load(u);
  issue_fence();
  // Epilogue operands of this lane's outputs (row m, columns n0 + 16 j + 4 lg .. + 3); a 16-column
  // block past N reads the last block (its outputs are not stored).
  float sc[GB][4], bi[GB][4];
#pragma unroll
  for (int j = 0; j < GB; ++j) {
    const int nb = min(n0 + 16 * j, N - 16) + 4 * lg;
    float4 c4, b4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (SIMPLE || !tl.scol_per_tensor) c4 = *reinterpret_cast<const float4*>(scol + nb);
    else c4 = make_float4(scol[0], scol[0], scol[0], scol[0]);
    if (!SIMPLE && tl.bias) b4 = *reinterpret_cast<const float4*>(tl.bias + nb);
    sc[j][0] = c4.x, sc[j][1] = c4.y, sc[j][2] = c4.z, sc[j][3] = c4.w;
    bi[j][0] = b4.x, bi[j][1] = b4.y, bi[j][2] = b4.z, bi[j][3] = b4.w;
  }
  const float sr = *(srow ? srow + min(m, M - 1) : scol);
  issue_fence();
#pragma unroll
  for (int u = (GA + 1) * KQ; u < (GA + GB) * KQ; ++u) load(u);

  auto store = [&](int j, const float (&y)[4]) {
    const int n = n0 + 16 * j + 4 * lg;
    if (m < M && n < N) {
      if constexpr (SIMPLE) {
        *reinterpret_cast<float4*>(static_cast<char*>(Y) + static_cast<int64_t>(m) * ldy + 4 * n) =
            make_float4(ftz(y[0]), ftz(y[1]), ftz(y[2]), ftz(y[3]));
      } else {
        store_out4(Y, static_cast<int64_t>(m) * ldy, n, tl.out, y, tl.out_scale);
      }
    }
  };
  const int8_t* const rd = lds + 256 * li;
  // phase 0: at most the last two groups' loads of this wave outstanding, then every wave's
  wait_vmcnt<2 * KQ>();
  __builtin_amdgcn_s_barrier();
  v4i fa[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
    fa[kb] = *reinterpret_cast<const v4i*>(rd + GRP * wave + 4096 * (kb / 4) + 16 * ((4 * (kb % 4) + lg) ^ li));
  float y1[4];
#pragma unroll
  for (int j = 0; j < GB; ++j) {
    if (j == 1) {
      // the last group's loads may still be outstanding, and block 0's store issued after them
      // (loads complete in issue order, so at most KQ outstanding covers both cases)
      wait_vmcnt<KQ>();
      __builtin_amdgcn_s_barrier();
    } else if (j == 2) {
      wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();
      store(1, y1);
    }
    // two exact int32 chains over alternate k steps (integer adds are order-free)
    v4i acc0 = zero, acc1 = zero;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const v4i fw = *reinterpret_cast<const v4i*>(rd + GRP * (GA + j) + 4096 * (kb / 4) +
                                                   16 * ((4 * (kb % 4) + lg) ^ li));
      if (kb & 1) acc1 = mfma(fw, fa[kb], acc1);
      else acc0 = mfma(fw, fa[kb], acc0);
    }
    const v4i acc = acc0 + acc1;
    // W is the MFMA's first operand, so lane l holds columns 4 lg .. 4 lg + 3 of row li
    float y[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if constexpr (SIMPLE) {
        y[v] = fmul(fmul(i2f(acc[v]), sr), sc[j][v]);
      } else {
        float z = i2f(acc[v]);
        if (srow) z = fmul(z, sr);
        z = fmul(z, sc[j][v]);
        if (tl.bias) z = fadd(z, bi[j][v]);
        y[v] = act_fn(z, tl.act);
      }
    }
    if (j == 1) {
#pragma unroll
      for (int v = 0; v < 4; ++v) y1[v] = y[v];
    } else {
      store(j, y);
    }
  }
}

template <int KQ>
hipError_t go_panel(const MfmaArgs& a, hipStream_t s) {
  const int mt = (a.M + 63) / 64, nt = (a.N + 47) / 48;
  TileTail tl{};
  tl.nseg = 1;
  tl.bias = a.epi.bias;
  tl.scol_per_tensor = a.epi.scol_per_tensor;
  tl.act = a.epi.act;
  tl.out = a.epi.out;
  tl.out_scale = a.epi.out_scale;
  const RowColEpilogue& e = a.epi;
  const bool simple = e.srow && !e.scol_per_tensor && !e.bias && e.act == 0 && e.out == 0;
  const int lda = static_cast<int>(a.lda), ldy = static_cast<int>(a.ldy);
  const dim3 grid(mt * nt), block(256);
  if (simple)
    hipLaunchKernelGGL((mfma_panel_kernel<KQ, true>), grid, block, 0, s, a.A + a.seg[0].koff, a.seg[0].W, e.scol,
                       e.srow, lda, a.seg[0].K, a.M, a.N, mt, ldy, a.Y, tl);
  else
    hipLaunchKernelGGL((mfma_panel_kernel<KQ, false>), grid, block, 0, s, a.A + a.seg[0].koff, a.seg[0].W, e.scol,
                       e.srow, lda, a.seg[0].K, a.M, a.N, mt, ldy, a.Y, tl);
  return hipGetLastError();
}

// ------------------------------------------------------------------------------------ chunk rows
// Chunk rows (M <= 16) on one 16 x 16 output tile per workgroup, the tile's 16 weight rows and up
// to 16 activation rows staged in LDS by global -> LDS loads of 4 rows x 256 bytes (the layout and
// swizzle of mfma_tile_kernel's 16-row blocks), K split over the KW waves in 256-byte blocks. A
// wave stages and reads only its own blocks, so it waits on its own loads and needs no workgroup
// barrier until its int32 partial tile meets the others in LDS; wave 0 then forms the epilogue.
// A K split (KSPLIT) runs its blocks one after another, each block's fp32 partial added in block
// order (llm.py:303-321).
template <int KW, int DB, bool SIMPLE, bool KSPLIT>
__global__ __launch_bounds__(64 * KW) void mfma_chunk_kernel(const int8_t* A, const int8_t* W, const float* scol,
                                                            const float* srow, int lda, int K, int M, int N, int ldy,
                                                            void* Y, TileTail tl) {
  constexpr int SLOT = DB * 8192;    // DB blocks: weights 4 KiB + activations 4 KiB each
  constexpr int RP = 20;             // int32 pitch of a partial tile's row in LDS
  __shared__ __align__(16) int8_t lds[KW * SLOT];
  __shared__ __align__(16) int32_t red[KW][16][RP];
  const v4i zero = {0, 0, 0, 0};
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int nt = N >> 4, b = blockIdx.x;
  const int n0 = 16 * ((nt % 8 == 0) ? (b % 8) * (nt / 8) + b / 8 : b);
  // wave 0's epilogue operands: thread t < 64 owns row t >> 2, columns n0 + 4 (t & 3) .. + 3
  const int er = lane >> 2, ec = n0 + 4 * (lane & 3);
  float sr = 0.0f, sc[4], bi[4] = {0.0f, 0.0f, 0.0f, 0.0f}, chain[4];
  if (wave == 0) {
    float4 c4 = (SIMPLE || !tl.scol_per_tensor) ? *reinterpret_cast<const float4*>(scol + ec)
                                                : make_float4(scol[0], scol[0], scol[0], scol[0]);
    sc[0] = c4.x, sc[1] = c4.y, sc[2] = c4.z, sc[3] = c4.w;
    if (!SIMPLE && tl.bias) {
      const float4 b4 = *reinterpret_cast<const float4*>(tl.bias + ec);
      bi[0] = b4.x, bi[1] = b4.y, bi[2] = b4.z, bi[3] = b4.w;
    }
    sr = *(srow ? srow + min(er, M - 1) : scol);
  }
  issue_fence();
  const int aq = (M + 3) >> 2;       // activation row quads holding live rows
  int8_t* const slot = lds + SLOT * wave;
  const int nseg = KSPLIT ? tl.nseg : 1;
  for (int sgi = 0; sgi < nseg; ++sgi) {
    const int8_t* const Wg = (KSPLIT && sgi) ? tl.W[sgi] : W;
    const int Kg = (KSPLIT && sgi) ? tl.K[sgi] : K;
    const int8_t* const Ag = A + ((KSPLIT && sgi) ? tl.koff[sgi] : 0);
    const int nb = Kg >> 8, b0 = nb * wave / KW, b1 = nb * (wave + 1) / KW;
    v4i acc0 = zero, acc1 = zero;
    for (int bb = b0; bb < b1; bb += DB) {
      const int nbb = min(DB, b1 - bb);
      // the previous batch's operand reads are done before its slot is refilled
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        if (d >= nbb) break;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = 4 * q + lg, k = 256 * (bb + d) + 16 * (li ^ r);
          stage16(Wg + static_cast<int64_t>(n0 + r) * Kg + k, slot + 8192 * d + 1024 * q);
          if (q < aq) stage16(Ag + static_cast<int64_t>(min(r, M - 1)) * lda + k, slot + 8192 * d + 4096 + 1024 * q);
        }
      }
      wait_vmcnt<0>();
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        if (d >= nbb) break;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int off = 8192 * d + 256 * li + 16 * ((4 * kk + lg) ^ li);
          const v4i fw = *reinterpret_cast<const v4i*>(slot + off);
          const v4i fa = *reinterpret_cast<const v4i*>(slot + off + 4096);
          if (kk & 1) acc1 = mfma(fw, fa, acc1);
          else acc0 = mfma(fw, fa, acc0);
        }
      }
    }
    // W is the MFMA's first operand: lane l holds columns 4 lg .. 4 lg + 3 of row li
    if (KSPLIT && sgi) __syncthreads();  // wave 0 has read the previous block's partial tiles
    *reinterpret_cast<v4i*>(&red[wave][li][4 * lg]) = acc0 + acc1;
    __syncthreads();
    if (wave == 0) {
      v4i sum = *reinterpret_cast<const v4i*>(&red[0][er][4 * (lane & 3)]);
#pragma unroll
      for (int w = 1; w < KW; ++w) sum += *reinterpret_cast<const v4i*>(&red[w][er][4 * (lane & 3)]);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float y;
        if constexpr (SIMPLE) {
          y = fmul(fmul(i2f(sum[v]), sr), sc[v]);
        } else {
          y = i2f(sum[v]);
          if (srow) y = fmul(y, sr);
          y = fmul(y, sc[v]);
          if (tl.bias) y = fadd(y, bi[v]);
          y = act_fn(y, tl.act);
        }
        chain[v] = sgi == 0 ? y : fadd(chain[v], y);
      }
    }
  }
  if (wave != 0 || er >= M) return;
  if constexpr (SIMPLE) {
    *reinterpret_cast<float4*>(static_cast<char*>(Y) + static_cast<int64_t>(er) * ldy + 4 * ec) =
        make_float4(ftz(chain[0]), ftz(chain[1]), ftz(chain[2]), ftz(chain[3]));
  } else {
    store_out4(Y, static_cast<int64_t>(er) * ldy, ec, tl.out, chain, tl.out_scale);
  }
}

template <int KW, int DB = 2>
hipError_t go_chunk(const MfmaArgs& a, hipStream_t s) {
  TileTail tl{};
  for (int i = 0; i < a.nseg; ++i) {
    tl.W[i] = a.seg[i].W;
    tl.K[i] = a.seg[i].K;
    tl.koff[i] = a.seg[i].koff;
  }
  tl.nseg = a.nseg;
  tl.bias = a.epi.bias;
  tl.scol_per_tensor = a.epi.scol_per_tensor;
  tl.act = a.epi.act;
  tl.out = a.epi.out;
  tl.out_scale = a.epi.out_scale;
  const RowColEpilogue& e = a.epi;
  const bool simple = e.srow && !e.scol_per_tensor && !e.bias && e.act == 0 && e.out == 0;
  const int lda = static_cast<int>(a.lda), ldy = static_cast<int>(a.ldy);
  const dim3 grid(a.N / 16), block(64 * KW);
  const int8_t* A = a.A + a.seg[0].koff;
#define TARS_CHUNK(SIMPLE, KSPLIT)                                                                                 \
  hipLaunchKernelGGL((mfma_chunk_kernel<KW, DB, SIMPLE, KSPLIT>), grid, block, 0, s, A, a.seg[0].W, e.scol, e.srow, \
                     lda, a.seg[0].K, a.M, a.N, ldy, a.Y, tl)
  if (a.nseg > 1) {
    if (simple) TARS_CHUNK(true, true);
    else TARS_CHUNK(false, true);
  } else {
    if (simple) TARS_CHUNK(true, false);
    else TARS_CHUNK(false, false);
  }
#undef TARS_CHUNK
  return hipGetLastError();
}

// ------------------------------------------------------------------------------------ dispatch
// Chunk rows (M <= 16): one 16-column tile per workgroup (the weights have no reuse, so the most
// workgroups), on the LDS-staged chunk kernel when K is one block of whole 256-byte blocks (4
// waves up to K = 1024, else 8, two blocks staged per batch; 16 waves, one block per batch, and 2
// to 8 waves measured the same or slower): M = 4 K = 1024 N = 3072 / K = 3072 N = 1024 4.26 / 5.87
// -> 2.92 / 3.62 us, M = 16 4.48 / 6.61 -> 3.10 / 4.16 us against the direct kernel (its 16-row x
// 64-byte register loads touch twice the cache lines per instruction); the direct kernel with 8
// waves over K otherwise.
// Prompt rows, when every K block is a whole number of stages (K a multiple of 256): the LDS tile
// kernel, its tile chosen by measurement on MI355X with the weights cold, bit-identical across
// tiles; the direct kernel's 32 x 32 tiles with 4 waves over K otherwise.
//  * 64 x 48 tiles (4 waves of 16 x 48, 256-byte stages, 3 slots) when they give one to 1.25
//    workgroups per CU: M=256 K=1024 N=3072 7.5 -> 5.5 us (the 64 x 64 / 16-row-load tiles before;
//    4 / 5 slots 5.70 / 5.89 us against 5.40, 512-byte stages in 2 slots 5.41 us); with one K block
//    of at most 1280 the panel form of the same tiles instead: K = 1024 5.41 -> 4.71 us (5.04 us
//    with block 1's store issued before the last wait and the epilogue operands before the first
//    loads; block 2 in two K halves 4.86 us), K = 256 / 512 / 768 / 1280 at N = 3072: 3.91 / 4.45 /
//    4.92 / 5.89 -> 3.63 / 3.96 / 4.27 / 5.26 us;
//  * 64 x 64 tiles (4 waves of 32 x 32, 256-byte stages, 3 slots) when they give 512 or more:
//    M=1024 K=1024 N=3072 16.5 -> 15.8 us;
//  * 32 x 32 tiles (4 waves of 16 x 16) with 512-byte stages in 3 slots when K is a multiple of
//    1024 and they give at most 1.25 workgroups per CU: M=256 K=3072 N=1024 8.6 -> 5.9 us with
//    1024-byte stages in 2 slots, 5.76 us with these (K = 1024 / 2048 / 4096 at N = 1024: 4.04 /
//    4.86 / 6.72 -> 3.77 / 4.77 / 6.68 us; 512-byte stages in 4 slots 0.1 - 0.3 us slower);
//  * 32 x 32 tiles with 256-byte stages in 3 slots otherwise: M=64 K=1024 N=3072 5.2 -> 3.8 us.
bool whole_stages(const MfmaArgs& a, int ks) {
  for (int i = 0; i < a.nseg; ++i)
    if (a.seg[i].K % ks) return false;
  return true;
}

int64_t tiles(const MfmaArgs& a, int bm, int bn) {
  return static_cast<int64_t>((a.M + bm - 1) / bm) * ((a.N + bn - 1) / bn);
}

hipError_t run(const MfmaArgs& a, hipStream_t s) {
  if (a.M <= 16) {
    if (whole_stages(a, 256) && a.lda <= INT32_MAX && a.ldy <= INT32_MAX) {
      int ktot = 0;
      for (int i = 0; i < a.nseg; ++i) ktot += a.seg[i].K;
      return ktot <= 1024 ? go_chunk<4, 2>(a, s) : go_chunk<8, 2>(a, s);
    }
    return go_direct<1, 1, 8, 1>(a, s);
  }
  // the LDS tile kernels take 32-bit row strides; the direct kernel any
  if (!whole_stages(a, 256) || a.lda > INT32_MAX || a.ldy > INT32_MAX) return go_direct<2, 2, 4, 1>(a, s);
  const int64_t t48 = tiles(a, 64, 48), t32 = tiles(a, 32, 32);
  if (t48 >= 192 && t48 <= 320) {
    if (a.nseg == 1 && a.seg[0].K <= 1280) {
      switch (a.seg[0].K / 256) {
        case 1: return go_panel<1>(a, s);
        case 2: return go_panel<2>(a, s);
        case 3: return go_panel<3>(a, s);
        case 4: return go_panel<4>(a, s);
        default: return go_panel<5>(a, s);
      }
    }
    return go_tile<64, 48, 4, 1, 256, 3>(a, s);
  }
  if (tiles(a, 64, 64) >= 512) return go_tile<64, 64, 2, 2, 256, 3>(a, s);
  if (t32 <= 320 && whole_stages(a, 1024)) return go_tile<32, 32, 2, 2, 512, 3>(a, s);
  return go_tile<32, 32, 2, 2, 256, 3>(a, s);
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
