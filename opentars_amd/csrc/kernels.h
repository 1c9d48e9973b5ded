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

// Direct global -> LDS loads (global_load_lds_dwordx4): 64 lanes x 16 bytes land in a 1 KiB LDS
// block in lane order with no VGPR round trip (lane l's bytes at dst + 16 l; dst is wave-uniform).
// The loads count in vmcnt like any other vector load; wait_vmcnt<N> waits until at most N of this
// wave's vector loads are outstanding.
#define TARS_LDS(p) ((__attribute__((address_space(3))) void*)(p))

__device__ __forceinline__ void stage16(const void* src, void* dst) {
  __builtin_amdgcn_global_load_lds(src, TARS_LDS(dst), 16, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit count");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Waits until at most L * ahead of this wave's vector loads are outstanding: a ring of stages of L
// loads each, `ahead` (uniform, 0..A) of them issued after the one about to be read.
template <int L, int A>
__device__ __forceinline__ void wait_stages_ahead(int ahead) {
  if constexpr (A > 0) {
    if (ahead >= A) {
      wait_vmcnt<L * A>();
      return;
    }
    wait_stages_ahead<L, A - 1>(ahead);
  } else {
    wait_vmcnt<0>();
  }
}

// Forces a uniform value (a kernel argument) into SGPRs at this point, so its scalar load is issued
// here, beside the vector loads already in flight, rather than at its first use.
template <class T>
__device__ __forceinline__ void pin_sgpr(const T& v) {
  __asm__ volatile("" : : "s"(v));
}

// Workgroup ids are dealt round-robin over the 8 XCDs (id % 8). Block index of workgroup x of n
// such that the workgroups of one XCD take consecutive blocks: the blocks' outputs then share
// cache lines inside one XCD's L2 instead of across XCDs. A bijection on [0, n).
__device__ __forceinline__ int xcd_block(int x, int n) {
  const int r = x & 7, k = x >> 3, per = n >> 3, rem = n & 7;
  return r * per + min(r, rem) + k;
}

// Kernel-argument preloading (the library is built with -amdgpu-kernarg-preload-count): gfx950
// places the leading scalar kernel arguments in SGPRs at wave launch, so a kernel whose first
// loads need only those issues them without a kernel-argument round trip. Kernels on the latency
// path take what their first loads need as leading scalars and the rest as a struct after them.
// A field of that struct is read through the kernel-argument segment with kload: a volatile scalar
// load that is issued where it stands (not sunk to its first use), so its latency overlaps the
// streams already in flight.
typedef const __attribute__((address_space(4))) char* KArg;
template <class T>
__device__ __forceinline__ T kload(KArg p) {
  return *reinterpret_cast<const volatile __attribute__((address_space(4))) T*>(p);
}
__device__ __forceinline__ KArg kernarg_at(size_t offset) {
  return (KArg)__builtin_amdgcn_kernarg_segment_ptr() + offset;
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
constexpr int kMaxGroups = 4;   // matrices per call
constexpr int kMaxPieces = 8;   // equal row pieces they may be cut into (one grid z slice each)
struct GemvGroup {
  const int8_t* W;       // [N, K] dense
  RowColEpilogue epi;    // srow unused: the row scale comes from the fused quantizer
  void* Y;
  int64_t ldy;
  int N;
};

// Optional residual add and norm in front of the fused quantizer (the executor's fusion of ELT ADD
// -> LayerNorm / RMSNorm / L2Norm -> ROW_QUANT -> GEMMs; quant_gemv_norm_supported(K); one row, so
// the strides are unused): the kernel's x row is the ELT's A row (the norm's input row when B is
// null). Every workgroup forms ftz(A + B) and its norm in registers and quantizes the norm's fp32
// output values; the first workgroup also stores the sum (at sum) and the norm's output (at y).
struct NormPrologue {
  int fn;               // a RowFn norm (ROWFN_LAYERNORM / RMSNORM / L2NORM); 0: no prologue
  const float* B;       // rows added to x (nullptr: the norm reads x itself)
  int64_t ldb;
  float* sum;           // with B: the sum's rows (fp32)
  int64_t ldsum;
  const float* gamma;   // [K]
  const float* beta;    // [K] or nullptr
  float eps;
  float* y;             // the norm's output rows (fp32)
  int64_t ldy;
};

struct QuantGemvArgs {
  const float* x;        // [M, K] fp32 rows at stride lda bytes
  int64_t lda;
  int8_t* q;             // optional: the quantized rows (stride ldq) and row scales, as quant_rows
  int64_t ldq;
  float* s;
  int M, K;
  GemvGroup g[kMaxPieces];
  int ngroups;  // matrix (piece) g runs as grid z = g
  // Optional gated product (an MLP's act(gate) * up): with ngroups == 2 and equal N, rows n of
  // matrix 0 and matrix 1 are computed by the same lane and fmul(y0[n], y1[n]) (the contract's
  // ELT MUL of the two fp32 outputs) is also stored to prod[m * ldprod / 4 + n]. prod may be g[0].Y
  // (in place: then only the product is stored there); fp32 outputs only.
  float* prod;
  int64_t ldprod;
  NormPrologue pro;  // pro.fn != 0: the residual add and norm in front of the quantizer
};

// Row functions, elementwise ops, rotary embedding and fp32 dot products (rowops.hip). Row strides
// are in bytes; fp32 and fp16 elements are read with element loads, so 4- / 2-byte alignment
// suffices.
enum RowFn { ROWFN_SOFTMAX = 0, ROWFN_LAYERNORM = 1, ROWFN_RMSNORM = 2, ROWFN_L2NORM = 3 };
struct RowArgs {
  const void* x;           // [M, N] fp32 rows
  int64_t lda;
  int fn;
  const float* gamma;      // [N] (norms)
  const float* beta;       // [N] or nullptr
  float eps;
  int causal_k;            // softmax: > 0 -> row m sees min(N, causal_k + m) elements
  const int32_t* valid;    // softmax: per-row valid counts (overrides causal_k) or nullptr
  void* y;
  int64_t ldy;
  int out;
  float out_scale;
  int M, N;
};

enum EltOp { ELTOP_MUL = 0, ELTOP_ADD = 1, ELTOP_MULADD = 2, ELTOP_SUB = 3 };
enum BMode { BMODE_DENSE = 0, BMODE_ROW = 1, BMODE_COL = 2, BMODE_SCALAR = 3 };
struct EltArgs {
  const void* A;           // fp32 or fp16 rows (a_fp16); a_row: one row broadcast to all M
  int64_t lda;
  int a_fp16, a_row;
  const float* B;          // dense rows at ldb, or N / M / 1 values
  int64_t ldb;
  int bmode;
  const void* C;           // MULADD addend rows, in the output's float format
  int64_t ldc;
  int op, act;
  void* Y;
  int64_t ldy;
  int out;
  float out_scale;
  int M, N;
};

struct RopeArgs {
  const void* x;
  int64_t lda;
  const float* tab;        // rows of [cos(0..rot/2-1), sin(0..rot/2-1)]
  int rows_per_pos, rot;
  void* y;
  int64_t ldy;
  int out;
  float out_scale;
  int M, N;
};

struct ReluArgs {
  const void* x;
  int64_t lda;
  int act;
  void* y;
  int64_t ldy;
  int out;
  float out_scale;
  int M, N;
};

struct FdotArgs {
  const void* A;           // [M, K] fp32
  int64_t lda;
  const void* B;           // NT: [N, K] fp32; NN: [K, N] fp32 or fp16 (b_fp16)
  int64_t ldb;
  int nn, b_fp16;
  void* Y;
  int64_t ldy;
  int out;
  float out_scale;
  int M, N, K;
};

// Decode attention of up to kAttnMaxHeads query heads in one launch, the fusion of the reference's
// per-head FDOT_NT (scores) -> ROW_SOFTMAX (causal) -> FDOT_NN (P V) triple
// (tars_mini/llm.py:736-746), bit-identical to running the three ops per head in order: every
// head's scores, probabilities and outputs are the golden's, and the scores and probabilities of
// the last head are written to sc / pr (the buffers all heads share).
constexpr int kAttnMaxHeads = 32, kAttnMaxKeys = 4080;  // 4080 keys: the scores row and the V ring fit 64 KiB of LDS
// A norm (RowFn LayerNorm / RMSNorm / L2Norm, fp32 output) and the full-width RoPE (rot == hd) of
// its output rows, run inside the split scores kernel (AttnArgs::rope): one row per query head, or
// per K / V head group.
struct AttnNormRope {
  const float* x;        // the norm's input rows (row r: query head r, or K / V head group r)
  int64_t ldx;
  const float* gamma;    // [hd]
  const float* beta;     // [hd] or nullptr
  float eps;
  int fn;
  float* n;              // the norm's output rows
  int64_t ldn;
  const float* tab;      // RoPE table rows [cos(0..hd/2-1), sin(0..hd/2-1)]; row r / rows_per_pos
  int rows_per_pos;
};

struct AttnArgs {
  const float* q[kAttnMaxHeads];   // head h: query rows [M, hd] at ldq
  const float* k[kAttnMaxHeads];   // K rows [nk, hd] at ldk (fp32)
  const void* v[kAttnMaxHeads];    // V rows [nk, hd] at ldv (fp32, or fp16 when v_fp16)
  void* att[kAttnMaxHeads];        // output rows [M, hd] at ldatt, format out
  int64_t ldq, ldk, ldv, ldatt;
  float* sc;                       // [M, nk] at ldsc: the last head's scores (fp32)
  int64_t ldsc;
  float* pr;                       // [M, nk] at ldpr: the last head's probabilities (fp32)
  int64_t ldpr;
  int heads, M, nk, hd, causal_k, v_fp16, out;
  float out_scale;
  // The split form (two launches over many workgroups) when scratch is not null and the shape fits
  // (attention_split_fits); otherwise one workgroup per head. scratch: device memory of
  // scratch_floats floats holding the scores of every head and query row between the launches.
  float* scratch;
  int64_t scratch_floats;
  // set by launch_attention for the split kernels: scratch row stride (floats), query heads per
  // K / V head group, keys per scores workgroup
  int64_t ld_scratch;
  int group, keys_per_wg;
  // rope > 0 (query heads per K / V head; one query row per head, the split form, hd a multiple
  // of 32, rq.fn == rk.fn): the scores kernel first runs the q and k norm + RoPE (the executor's fusion of a
  // decoder's q and k norm and rotation with its attention). Head h's query row q[h] is the RoPE of
  // the norm of row h of rq.x; key row rope_key of head h's keys (k[h]) is that of row h / rope of
  // rk.x, which the workgroups whose keys include it form in registers, use, and store (several
  // store the same values when a workgroup's group holds fewer heads than a K / V head serves). The
  // workgroups of the first key chunk store the query rows (norm outputs and q rows), the new key's
  // workgroups its norm output.
  int rope, rope_key;  // rope_key: the key row the k RoPE writes
  AttnNormRope rq, rk;
};
bool attention_supported(int hd, int nk);
// Split form limits: query rows per head group (heads sharing K / V times M) and probabilities a
// P V workgroup holds in LDS; output columns per P V workgroup.
constexpr int kAttnSplitMaxQ = 4, kAttnSplitProbs = 4096, kAttnSplitCols = 32;
bool attention_split_fits(int heads, int M, int nk, int64_t scratch_floats);
// The split form's scratch of stream `s` on the current device: kAttnScratchFloats floats allocated
// at the stream's first call (not while `s` is capturing a graph), kept until the process ends;
// each stream its own (up to 64 per device), so calls on different streams never share one; null
// when none.
constexpr int64_t kAttnScratchFloats = int64_t{1} << 18;
float* attention_workspace(hipStream_t s);
// The same size of scratch as a file-scope device array on the current device (no allocation;
// its address looked up once per device); null when the lookup fails.
float* attention_static_scratch();

// Embedding rows: dst row i = fp32(table row ids[i]) (times the fp32 scale when scaled).
constexpr int kEmbedMaxIds = 64;
struct EmbedArgs {
  const uint16_t* table;  // bf16 [rows, cols] at ld_table bytes
  int64_t ld_table;
  float* dst;             // fp32 [n, cols] at ldd bytes
  int64_t ldd;
  int cols, n, scaled;
  uint32_t scale_bits;
  int32_t ids[kEmbedMaxIds];
};
hipError_t launch_embed_rows(const EmbedArgs& a, hipStream_t s);
hipError_t launch_attention(const AttnArgs& a, hipStream_t s);

hipError_t launch_row(const RowArgs& a, hipStream_t s);
// An ELT ADD (dense fp32 rows, fp32 output, no activation) and the LayerNorm / RMSNorm / L2Norm of
// its output in one launch: the ELT's output is written, then normalized as launch_row would.
bool add_norm_supported(int M, int N);
hipError_t launch_add_norm(const EltArgs& e, const RowArgs& r, hipStream_t s);
// A LayerNorm / RMSNorm / L2Norm with an fp32 output and the RoPE (fp32 output) of its output rows
// in one launch (rows within add_norm_supported's bounds): the norm's output is written, then rotated.
hipError_t launch_norm_rope(const RowArgs& r, const RopeArgs& p, hipStream_t s);
// Two independent (norm, RoPE) jobs in one launch (r0.M + r1.M workgroups).
hipError_t launch_norm_rope2(const RowArgs& r0, const RopeArgs& p0, const RowArgs& r1, const RopeArgs& p1, hipStream_t s);
hipError_t launch_elt(const EltArgs& a, hipStream_t s);
hipError_t launch_rope(const RopeArgs& a, hipStream_t s);
hipError_t launch_relu(const ReluArgs& a, hipStream_t s);
hipError_t launch_fdot(const FdotArgs& a, hipStream_t s);

hipError_t launch_quant_rows(const QuantArgs& a, hipStream_t s);
hipError_t launch_gemv_w8a8(const W8A8Args& a, hipStream_t s);
hipError_t launch_quant_gemv_w8a8(QuantGemvArgs& a, hipStream_t s);
bool quant_gemv_pairs_supported(int K);  // whether a.prod (the gated product) can run at this K
bool quant_gemv_norm_supported(int K);   // whether a.pro (a norm prologue) can run at this K
hipError_t launch_gemm_w8a8_mfma(const W8A8Args& a, hipStream_t s);
hipError_t launch_gemv_w8a8_ksplit(const KSplitArgs& a, hipStream_t s);
hipError_t launch_gemm_w8a8_ksplit_mfma(const KSplitArgs& a, hipStream_t s);
hipError_t launch_align_w4(const AlignArgs& a, hipStream_t s);
hipError_t launch_gemv_w4a16(const W4Args& a, hipStream_t s);

}  // namespace tars
