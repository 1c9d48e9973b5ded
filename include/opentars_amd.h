/*
 * opentars_amd: the openTARS golden model's quantized matrix path on MI355X (gfx950).
 *
 * C ABI of libopentars_amd.so. Plain pointers and sizes only. Every pointer is a device
 * pointer (hipMalloc'd or a torch CUDA/HIP tensor's data_ptr) except where noted; `stream` is a
 * hipStream_t (NULL = the null stream). Work is enqueued on `stream` and is stream-ordered with
 * whatever else the caller puts there; nothing synchronizes the host. No entry point allocates,
 * except that tars_attention and the attention in tars_run_queue allocate a 1 MiB scores scratch
 * per (device, stream) at a stream's first use there, and tars_run_queue one per launch plan that
 * runs attention (tars_attention_noalloc never does).
 *
 * Every entry point validates its arguments on the host before it launches anything and returns
 * a status. On a non-zero status nothing was launched and nothing was written, mirroring the
 * golden model's "every check before any write" rule (tars_mini/golden.py:450-472).
 *
 * Results are bit-exact against the golden model's arithmetic (tars_mini/golden.py,
 * tars_mini/numerics.py): exact int32 dot products, then the fp32 epilogue one rounded step at a
 * time (round-to-nearest-even, subnormals flushed on the way in and out, canonical NaN, no FMA).
 * Results never depend on launch geometry.
 */
#ifndef OPENTARS_AMD_H
#define OPENTARS_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: 0, or minus the contract's error code (tars_mini/contract.py:107-111) ---- */
#define TARS_OK           0
#define TARS_E_FIELD     (-6)   /* a field value the contract rejects (act/out code, K > 65535, ...) */
#define TARS_E_ALIGN     (-7)   /* shape / alignment / stride rule (N % 16, K % 16, 16-byte offsets) */
#define TARS_E_RANGE     (-8)   /* a size that cannot be addressed (overflowing extents)              */
#define TARS_E_OVERLAP   (-9)   /* an output overlaps an input: the golden's ContractError            */
#define TARS_E_ARG       (-10)  /* a NULL pointer where data is required, or a bad block list        */
#define TARS_E_DEVICE    (-11)  /* the HIP runtime refused the launch (no device, bad stream, ...)   */

/* ---- epilogue codes (tars_mini/contract.py:96-101) ---- */
#define TARS_ACT_NONE     0
#define TARS_ACT_RELU     1
#define TARS_ACT_RELU6    2
#define TARS_ACT_GELU     3
#define TARS_ACT_SILU     4
#define TARS_ACT_SIGMOID  5
#define TARS_ACT_SOFTPLUS 6
#define TARS_ACT_EXP      7
#define TARS_OUT_FP32     0
#define TARS_OUT_BF16     1
#define TARS_OUT_INT8     2     /* q8(y, out_scale): out_scale_bits is its fp32 encoding */
#define TARS_OUT_FP16     3     /* binary16, RNE, gradual underflow, NaN 0x7E00 (ELT only) */

/* ---- W4A16 activation dtypes (tars_mini/contract.py:92) ---- */
#define TARS_DT_BF16      0
#define TARS_DT_FP32      4

/*
 * Per-token INT8 quantization of fp32 rows.
 * Replaces numerics.quant_rows (tars_mini/numerics.py:383-390) as run by the ROW_QUANT descriptor
 * (tars_mini/golden.py:369-372, emitted by Dev.quant, tars_mini/llm.py:97-104).
 *   x  fp32 [M, K], row stride lda bytes      q  int8 [M, K], row stride ldq bytes
 *   s  fp32 [M] row scales (amax * fp32(1/127))
 * Rules: M >= 1, K >= 16, K % 16 == 0, lda/ldq multiples of 16 holding a row, 16-byte aligned
 * pointers; q and s must not overlap x or each other.
 */
int tars_quant_rows(const float* x, int64_t lda, int8_t* q, int64_t ldq, float* s,
                    int32_t M, int32_t K, void* stream);

/*
 * W8A8 GEMM / GEMV with the golden epilogue:
 *   y[m,n] = convert(act(((i2f(sum_k A[m,k] W[n,k]) * srow[m]) * scol[n]) + bias[n]))
 * Replaces Machine._gemm (tars_mini/golden.py:326-349) for OP_GEMM with QM_ROWCOL (srow given),
 * QM_CHANNEL (srow NULL, scol_count == N) and QM_TENSOR (srow NULL, scol_count == 1); emitted by
 * Dev.gemm_rc (tars_mini/llm.py:111-118).
 *   A     int8 [M, K], row stride lda bytes      W     int8 [N, K] dense row-major
 *   srow  fp32 [M] or NULL                        scol  fp32 [scol_count]
 *   bias  fp32 [N] or NULL                        Y     [M, N] of the output format, stride ldy
 * Small M runs the HBM-streaming GEMV family (packed int8 dot products, up to 4 activation rows
 * per weight read); larger M runs INT8 MFMA tiles (see tars_set_w8a8_path for the rule).
 * Rules: N % 16 == 0, K % 16 == 0, 16 <= K <= 65535, act in 0..7, out in {FP32, BF16, INT8},
 * out_scale_bits == 0 unless out == INT8, 16-byte aligned pointers and strides.
 */
int tars_gemm_w8a8(const int8_t* A, int64_t lda, const float* srow,
                   const int8_t* W, const float* scol, int32_t scol_count, const float* bias,
                   void* Y, int64_t ldy, int32_t M, int32_t N, int32_t K,
                   int32_t act, int32_t out, uint32_t out_scale_bits, void* stream);

/* One weight matrix fed by a shared quantized activation (tars_quant_gemm_w8a8). */
typedef struct tars_w8a8_out {
  const int8_t* W;          /* int8 [N, K] dense row-major, 16-byte aligned */
  const float* scol;        /* fp32 [N] per-channel scales */
  const float* bias;        /* fp32 [N] or NULL */
  void* Y;                  /* [M, N] of the output format, row stride ldy bytes */
  int64_t ldy;
  int32_t N;
  int32_t act;
  int32_t out;
  uint32_t out_scale_bits;
} tars_w8a8_out;

/*
 * Fused per-token quantization + W8A8 GEMV/GEMM for up to 4 weight matrices sharing it:
 *   (q, s) = quant_rows(x);  Y_i = convert_i(act_i(((i2f(q W_i^T) * s) * scol_i) + bias_i))
 * Replaces one ROW_QUANT descriptor and the QM_ROWCOL GEMM descriptors that read its output, as
 * QwenLowering emits them for q/k/v and gate/up (tars_mini/llm.py:711-731, 620-623; the
 * descriptors at tars_mini/golden.py:369-372 and 326-349). Bit-identical to quant_rows followed
 * by tars_gemm_w8a8 per matrix.
 *   x  fp32 [M, K] (stride lda);  q/ldq/s: optional outputs (both NULL or both given) receiving
 *   the quantized rows and row scales exactly as tars_quant_rows writes them.
 *   outs: HOST array of nouts (1..4) descriptors. Rules: those of tars_quant_rows and
 *   tars_gemm_w8a8 (per matrix, scol per channel); no output may overlap an input or another output.
 */
int tars_quant_gemm_w8a8(const float* x, int64_t lda, int8_t* q, int64_t ldq, float* s,
                         int32_t M, int32_t K, const tars_w8a8_out* outs, int32_t nouts,
                         void* stream);

/*
 * W8A8 with K split into blocks that share one quantized activation row block and one
 * per-channel scale vector: block i covers columns [c_i, c_i + K_i) of A (c_0 = 0) with its own
 * dense weights W_i [N, K_i]; each block's partial is a full W8A8 result in fp32 and the partials
 * add in block order, y = ((y_0 + y_1) + y_2) + ...  fp32 output only.
 * Replaces QwenLowering.lin_k + the ELT_ADD loop (tars_mini/llm.py:303-321, 627-635, 753-761;
 * tars_mini/golden.py:411-412).
 *   W_blocks, K_blocks: HOST arrays of nblocks device pointers / block widths (1 <= nblocks <= 8,
 *   every K_i % 16 == 0, 16 <= K_i <= 65535).
 */
int tars_gemm_w8a8_ksplit(const int8_t* A, int64_t lda, const float* srow,
                          const int8_t* const* W_blocks, const int32_t* K_blocks, int32_t nblocks,
                          const float* scol, float* Y, int64_t ldy, int32_t M, int32_t N,
                          void* stream);

/*
 * Block-FP alignment of W4A16 activations: fp32 or bf16 [M, K] -> int16 mantissas [M, K] and one
 * fp32 scale per 128-wide group [M, K/128].
 * Replaces numerics.align_w4_groups (tars_mini/numerics.py:55-98).
 *   x: a_dtype TARS_DT_FP32 or TARS_DT_BF16, row stride lda bytes; q row stride ldq bytes;
 *   scales row stride lds bytes (multiple of 4). Rules: K % 128 == 0, K >= 128.
 */
int tars_align_w4(const void* x, int64_t lda, int32_t a_dtype, int16_t* q, int64_t ldq,
                  float* scales, int64_t lds, int32_t M, int32_t K, void* stream);

/*
 * W4A16 group-128 GEMV/GEMM with fp16 group scales and block-FP activations:
 *   per group g: term = (i2f(dot_g) * ws[n,g]) * xs[m,g]; four fp32 banks add terms g % 4 in g
 *   order from +0; y = (b0 + b1) + (b2 + b3); then bias, act, convert.
 * Replaces Machine._gemm_w4 (tars_mini/golden.py:295-324), emitted by Dev.gemm_w4
 * (tars_mini/llm.py:120-132).
 *   x   fp32 / bf16 [M, K], stride lda       Wp  uint8 [N, K/2] nibbles (low = even k), 128-B aligned
 *   ws  uint16 [N, K/128] binary16 bits      bias fp32 [N] or NULL; Y as tars_gemm_w8a8
 * Rules: K % 256 == 0, 256 <= K <= 8192, N % 16 == 0 (tars_mini/golden.py:96-99, 140-147).
 */
int tars_gemm_w4a16(const void* x, int64_t lda, int32_t a_dtype,
                    const uint8_t* Wp, const uint16_t* ws, const float* bias,
                    void* Y, int64_t ldy, int32_t M, int32_t N, int32_t K,
                    int32_t act, int32_t out, uint32_t out_scale_bits, void* stream);

/* ---- fp32 row functions, elementwise ops, rotary embedding, fp32 dot products ----
 * The golden model's v0.3/v0.4 row-engine ops (tars_mini/golden.py:351-436), bit-exact in the same
 * contract: every fp32 multiply or add one rounded step, subnormals flushed, canonical NaN, row sums
 * in the 16-lane order (tars_mini/numerics.py:306-316). Shared rules: M, N (and K) >= 1; fp32 data
 * 4-byte aligned, fp16 data 2-byte aligned, the output aligned to its element; a stride of 0 means
 * dense, else it is a multiple of the element size holding a row; act 0..7; out FP32 / BF16 / INT8
 * (ELT also FP16); out_scale_bits only with INT8; an output overlapping an input is refused
 * (TARS_E_OVERLAP) except ELT's in-place forms. */
#define TARS_ROW_SOFTMAX   0
#define TARS_ROW_LAYERNORM 1
#define TARS_ROW_RMSNORM   2
#define TARS_ROW_L2NORM    3

/*
 * Row functions of fp32 rows.
 * Replaces Machine._row (tars_mini/golden.py:358-380) for softmax, causal softmax, LayerNorm,
 * RMSNorm and L2Norm: numerics.softmax_rows, softmax_rows_causal, layernorm_rows, rmsnorm_rows,
 * l2norm_rows (tars_mini/numerics.py:328-380).
 *   x fp32 [M, N] at lda bytes; y [M, N] at ldy bytes in format out.
 *   SOFTMAX: gamma, beta, eps_bits 0. Causal when causal_k > 0 (row m sees its first
 *     min(N, causal_k + m) elements, the descriptor's K rule) or when valid (device int32 [M],
 *     each in 1..N; values outside are clamped) is given; the rest of a causal row is +0.
 *   LAYERNORM / RMSNORM / L2NORM: gamma fp32 [N], beta fp32 [N] or NULL, eps_bits the fp32
 *     encoding of eps; causal_k 0, valid NULL.
 */
int tars_row_op(const float* x, int64_t lda, int32_t fn, const float* gamma, const float* beta,
                uint32_t eps_bits, int32_t causal_k, const int32_t* valid, void* y, int64_t ldy,
                int32_t out, uint32_t out_scale_bits, int32_t M, int32_t N, void* stream);

#define TARS_ELT_MUL       0
#define TARS_ELT_ADD       1
#define TARS_ELT_MULADD    2
#define TARS_ELT_SUB       3
#define TARS_BM_DENSE      0    /* B(m, n) = B[m][n] at ldb */
#define TARS_BM_ROW        1    /* B[n]                     */
#define TARS_BM_COL        2    /* B[m]                     */
#define TARS_BM_SCALAR     3    /* B[0]                     */

/*
 * Elementwise y = act(A) * B, act(A) + B, act(A) + -B or C + act(A) * B, each step rounded once.
 * Replaces Machine._elt (tars_mini/golden.py:393-418); its in-place rule is golden.py:440-448.
 *   A [M, N] fp32 (a_fp16 = 1: binary16 bits) at lda bytes; a_row = 1: A is one row used for every m.
 *   B fp32 per bmode; C (MULADD only, else NULL) [M, N] at ldc in the output's float format
 *   (fp32, or fp16 when out = FP16); MULADD needs out FP32 or FP16.
 *   Y [M, N] at ldy in format out. Y may be A itself (same format and stride, not a broadcast row)
 *   or C itself (same stride).
 */
int tars_elt(const void* A, int64_t lda, int32_t a_fp16, int32_t a_row, const float* B, int64_t ldb,
             int32_t bmode, const void* C, int64_t ldc, int32_t op, int32_t act, void* Y, int64_t ldy,
             int32_t out, uint32_t out_scale_bits, int32_t M, int32_t N, void* stream);

/*
 * Rotary embedding of the first rot elements of each fp32 row; the rest copied.
 * Replaces Machine._rope (tars_mini/golden.py:420-424) / numerics.rope_rows (numerics.py:412-424).
 *   tab fp32 rows of rot values [cos(0..rot/2-1), sin(0..rot/2-1)], dense; row m uses table row
 *   m / rows_per_pos. Rules: rot even, 2 <= rot <= N, rows_per_pos >= 1.
 */
int tars_rope(const float* x, int64_t lda, const float* tab, int32_t rows_per_pos, int32_t rot,
              void* y, int64_t ldy, int32_t out, uint32_t out_scale_bits, int32_t M, int32_t N,
              void* stream);

/*
 * Activation of fp32 rows, converted to the output format.
 * Replaces Machine._relu (tars_mini/golden.py:351-356).
 */
int tars_relu(const float* x, int64_t lda, int32_t act, void* y, int64_t ldy, int32_t out,
              uint32_t out_scale_bits, int32_t M, int32_t N, void* stream);

/*
 * Token rows of a bf16 embedding table, looked up on the device: dst row i (at dst + i * ldd) =
 * table row ids[i] widened to fp32 (the 16 bits moved to the top half, exact), times the fp32
 * scale scale_bits when `scaled` (one multiply, rounded to nearest even, subnormals kept).
 * Replaces the board runtime's host lookup of the input embedding and Gemma 4's per-layer
 * embedding rows (deploy/kv260/sw/tars_board.py:298-314, Qwen._put), so a step sends token ids.
 *   table [rows, cols] at ld_table bytes (>= 2 cols, even); ids: host array of n indexes in
 *   [0, rows), any n >= 1; dst fp32 at ldd bytes (>= 4 cols, a multiple of 4); dst must not
 *   overlap the table's extent (its row gaps included).
 * The ids travel as kernel arguments, 64 per launch. Every check runs before the first launch;
 * the one exception to "nothing written on a non-zero status" is TARS_E_DEVICE from the runtime
 * refusing a later launch, which leaves the rows of the launches before it written.
 */
int tars_embed_rows(const uint16_t* table, int64_t ld_table, int64_t rows, int32_t cols,
                    const int32_t* ids, int32_t n, int32_t scaled, uint32_t scale_bits, float* dst,
                    int64_t ldd, void* stream);

/*
 * fp32 dot products y[m][n] = sum_k A[m][k] * B(k, n).
 * Replaces Machine._fdot (tars_mini/golden.py:426-436): nn = 0, B [N, K] fp32 (numerics.fdot_nt,
 * the 16-lane sum, numerics.py:393-399); nn = 1, B [K, N] fp32 or binary16 (b_fp16), each output
 * one sequential chain over k (numerics.fdot_nn, numerics.py:402-409).
 */
int tars_fdot(const float* A, int64_t lda, const void* B, int64_t ldb, int32_t nn, int32_t b_fp16,
              void* Y, int64_t ldy, int32_t out, uint32_t out_scale_bits, int32_t M, int32_t N,
              int32_t K, void* stream);

/*
 * Attention of `heads` query heads in one call: per head h the triple the reference lowers
 * attention to (tars_mini/llm.py:736-746), FDOT_NT of q[h]'s rows with the K rows (the scores,
 * Machine._fdot, golden.py:426-436), ROW_SOFTMAX with the causal rule (Machine._row,
 * golden.py:358-380), FDOT_NN of the probabilities with the V rows into att[h]. Every output bit
 * is what the three ops leave run head after head: att[h] for every head, and the shared score
 * rows sc and probability rows pr holding the last head's (either may be NULL to skip it).
 *   q, k, v, att: HOST arrays of `heads` device pointers. q[h] fp32 [M, hd] at ldq; k[h] fp32
 *   [nk, hd] at ldk; v[h] [nk, hd] at ldv, fp32 or binary16 (v_fp16); att[h] [M, hd] at ldatt
 *   in format out (FP32, BF16, or INT8 with out_scale_bits); sc, pr fp32 [M, nk] at ldsc / ldpr.
 *   causal_k > 0: query row m sees its first min(nk, causal_k + m) keys (the descriptor's K
 *   rule); 0: all nk. hd 64, 128 or 256; 1 <= nk <= 4080; 1 <= heads <= 32; M >= 1; pointers
 *   and strides (0 = dense) multiples of 16 bytes. No output may overlap another output or any
 *   head's q, K or V rows (the heads run concurrently): TARS_E_OVERLAP.
 * Consecutive heads with equal k and v pointers (2 or 4 query heads per K / V head) are run
 * together. When such a group has at most 4 query rows in all (heads in the group times M) and
 * the scores fit, the work is split over many workgroups through a 1 MiB device scratch buffer
 * of the call's stream, which the library allocates at the stream's first use on the device and
 * keeps until the process ends (each stream has its own, up to 64 streams per device, so calls on
 * different streams may overlap in time; a graph captured from a stream keeps that stream's
 * scratch, so replay it ordered with the stream's other attention calls); otherwise (more streams,
 * or a stream capturing a graph before its first use), one workgroup per head. The bits are the
 * same.
 */
int tars_attention(const float* const* q, int64_t ldq, const float* const* k, int64_t ldk,
                   const void* const* v, int64_t ldv, int32_t v_fp16, void* const* att, int64_t ldatt,
                   int32_t out, uint32_t out_scale_bits, float* sc, int64_t ldsc, float* pr, int64_t ldpr,
                   int32_t heads, int32_t M, int32_t nk, int32_t hd, int32_t causal_k, void* stream);

/*
 * tars_attention without any allocation, for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc); it has no counterpart
 * in the reference. Same arguments, checks and results as tars_attention; the split form's scores
 * go to a static device array of 262144 floats (1 MiB) that each GPU holds from the library's load
 * until the process ends, instead of a workspace the library allocates. heads * M * nk (nk rounded
 * up to a multiple of 4) above 262144 is refused with TARS_E_RANGE. Every call on a GPU shares that
 * GPU's array: calls that overlap in time on one GPU race.
 */
int tars_attention_noalloc(const float* const* q, int64_t ldq, const float* const* k, int64_t ldk,
                           const void* const* v, int64_t ldv, int32_t v_fp16, void* const* att,
                           int64_t ldatt, int32_t out, uint32_t out_scale_bits, float* sc, int64_t ldsc,
                           float* pr, int64_t ldpr, int32_t heads, int32_t M, int32_t nk, int32_t hd,
                           int32_t causal_k, void* stream);

/* Library version string ("opentars_amd <semver> gfx950"). Host only, never fails. */
const char* tars_version(void);

/* Text of the last non-zero status on the calling thread ("" if none). Host only. */
const char* tars_last_error(void);

/*
 * Kernel-family selection for W8A8 (test and benchmark control, not part of the reference's
 * interface): 0 = automatic, by measurement (the dot-product GEMV family for M <= 2; with
 * K % 256 == 0 for M <= 4 unless K >= 4096 and N >= 4096, for M <= 8 while N < 4096 and for
 * M <= 16 while N < 2048; with other K for M <= 16 unless M >= 9, N >= 3072 and K >= 256, or
 * M >= 5 and N * K >= 12 MiB; INT8 MFMA family otherwise; for tars_gemm_w8a8_ksplit the GEMV family for M <= 2, for
 * M <= 4 when a block is not whole 256-byte blocks, else for M = 3 under 12 MiB of weights and
 * M <= 8 under 6 MiB), 1 = force the GEMV family for every M, 2 = force the MFMA family
 * for every M. Results are identical either way. Returns the previous setting. Process-wide.
 */
int tars_set_w8a8_path(int path);

/* ---------------------------------------------------------------- descriptor queue executor
 * Replaces tars_mini/golden.py:450-492 (Machine.run_queue) for a DDR image that lives in device
 * memory; the descriptor layout, CRC and check order are contract.py:14-38,154-181 and
 * golden.py:59-169 (validate), :172-258 (strides, segments, extra_out), :260-267 and :440-448
 * (overlap rules).
 */

/* The end state of a queue run (golden.py:23-30 Status) plus the hand-off flag. */
typedef struct tars_queue_status {
  int32_t done;     /* 1: all n descriptors ran */
  int32_t err_code; /* the contract's ERR_CODE: 0 OK, 1 E_MAGIC, 2 E_VERSION, 3 E_CRC, 4 E_VALID,
                       5 E_OPCODE, 6 E_FIELD, 7 E_ALIGN, 8 E_RANGE */
  int32_t op_idx;   /* the descriptor that stopped the queue (CUR_OP_IDX); n when done */
  int32_t host_op;  /* 1: stopped at a valid descriptor this library does not run on the GPU
                       (ops other than the W8A8 / W4A16 GEMM and ROW_QUANT, or an image address
                       that misses the kernels' 16 / 128-byte alignment); nothing of it ran */
} tars_queue_status;

/*
 * Runs the n descriptors at image + queue_addr, in order, on `stream`. `image` is the device
 * address of the DDR image (image_len bytes); every descriptor address is an offset into it.
 * host_queue NULL: the descriptors are read from the image (the call waits for the stream's
 * earlier work to do so); otherwise host_queue is the caller's HOST copy of the same 64 * n bytes
 * and the call does not wait (a descriptor whose output lands on a later descriptor of the queue
 * still makes it wait and re-read those from the image). The descriptors are checked on the host
 * in the contract's order; the GPU-run ones are enqueued on `stream` and have not necessarily
 * finished when the call returns. Returns TARS_OK with *st describing the
 * outcome (a contract error stops the queue at its descriptor, keeping earlier writes), or
 * TARS_E_OVERLAP when a descriptor's output overlaps one of its inputs (the golden's
 * ContractError; st->op_idx names it, nothing of it ran), TARS_E_ARG, or TARS_E_DEVICE.
 * core_id: the executing core's id (CORE_ID must match); gemv_only: the KV260 profile (a conv or
 * a GEMM with K > 4096 is E_OPCODE), golden.py:48-50.
 * Fused attention uses the split form's scores scratch of `stream` (as tars_attention) when the
 * queue runs op by op, and the launch plan's own scratch when it replays as a graph, so queues on
 * different images may run on different streams at once. Each plan that runs attention holds
 * 1 MiB of device memory; evicting a plan (more than 8 cached) frees it, which waits for the device.
 */
int tars_run_queue(uint8_t* image, uint64_t image_len, uint64_t queue_addr, int32_t n,
                   const uint8_t* host_queue, int32_t core_id, int32_t gemv_only,
                   tars_queue_status* st, void* stream);

/*
 * The full check of one 64-byte descriptor (host memory) against an image of image_len bytes:
 * *err_code = its ERR_CODE (E_RANGE included, golden.py:462-468); *gpu (if not NULL) = 1 when
 * it is valid and tars_run_queue would run it on the GPU. Returns TARS_E_OVERLAP for a valid
 * descriptor whose output overlaps an input (golden.py:473-479), else TARS_OK. Host only.
 */
int tars_check_descriptor(const uint8_t* desc, uint64_t image_len, int32_t core_id,
                          int32_t gemv_only, int32_t* err_code, int32_t* gpu);

/* The 23 fields of a 64-byte descriptor in layout order (MAGIC, VERSION, CORE_ID, HDR_RSV,
 * OPCODE, CTRL, GROUP_SIZE, EPI, BASE_ADDR, A_OFF, W_OFF, Y_OFF, SCALE_OFF, BIAS_OFF, M, N, K,
 * LDA16, OUT_SCALE, CRC32, VALID, LDY16, DEP_SIG), contract.py:170-172. Host only. */
int tars_decode_descriptor(const uint8_t* desc, uint64_t* fields);

/* The CRC-32 a descriptor's CRC32 field must hold: zlib's crc32 over the 64 bytes with bytes
 * 4..7 read as zero (contract.py:154-181). Host only. */
uint32_t tars_descriptor_crc(const uint8_t* desc);

/* Writes the 64-byte descriptor holding the 23 fields (layout order as tars_decode_descriptor);
 * with fix_crc the CRC32 field is replaced by the descriptor's CRC (contract.py:154-167 encode).
 * TARS_E_ARG if a value does not fit its field. Host only. */
int tars_encode_descriptor(const uint64_t* fields, int32_t fix_crc, uint8_t* desc);

/* Peephole fusion in tars_run_queue (benchmark and test control, not part of the reference's
 * interface): 1 (default) runs a decode-row ROW_QUANT and the QM_ROWCOL GEMMs that read its output
 * as one fused launch, 0 runs every descriptor on its own. Results are identical either way.
 * Returns the previous setting. Process-wide. */
int tars_set_queue_fusion(int on);

/* Fused launches tars_run_queue has run (diagnostics for tests and benchmarks, not part of the
 * reference's interface), counted per kind since the last reset: counts[0] decode-row quantizer +
 * GEMMs, counts[1] attention (per-head FDOT / softmax / FDOT triples), counts[2] residual ELT ADD +
 * norm, counts[3] (norm, RoPE) pairs, counts[4] an MLP's gated product (the ELT MUL of a gate and
 * an up GEMM folded into their quantizer + GEMMs launch, which counts[0] also counts), counts[5]
 * launches that ran two adjacent independent (norm, RoPE) pairs, such as a decoder layer's q and
 * k (counts[3] counts both pairs), counts[6] quantizer + GEMMs launches that also ran the norm in
 * front of the quantizer and the residual ELT ADD before it (which counts[0] also counts),
 * counts[7] attention launches whose scores kernel also ran the layer's q and k norm + RoPE pairs
 * (counted in counts[1] and, as two pairs, in counts[3]). A replayed launch plan counts its fused
 * launches again. The first ncounts (up to 8) are written to counts, which may be NULL; reset != 0
 * zeroes the counts after reading them. Process-wide. */
int tars_queue_fusion_counts(int64_t* counts, int32_t ncounts, int32_t reset);

/* Launch plans in tars_run_queue (benchmark and test control): 1 (default) keeps, for up to 8
 * queues, the launches of a queue that ran to the end without a hand-off or an output over its own
 * descriptors; when the same descriptor bytes run again on the same image with the same settings,
 * they are captured once into a HIP graph and every later run is one graph launch. 0 disables
 * and drops the plans. Results are identical either way. Returns the previous setting. */
int tars_set_queue_graphs(int on);

#ifdef __cplusplus
}
#endif

#endif /* OPENTARS_AMD_H */
