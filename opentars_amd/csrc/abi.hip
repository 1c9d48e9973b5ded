// The C ABI of libopentars_amd.so (include/opentars_amd.h): argument checks, then dispatch.
//
// Checks follow the golden model's order for a GEMM descriptor (tars_mini/golden.py:59-169):
// field values (E_FIELD) before shapes and alignment (E_ALIGN) before extents (E_RANGE), then
// the output-overlaps-input refusal (golden.py:473-479, a ContractError there). All checks run on
// the host before anything is enqueued, so a failing call writes nothing.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/opentars_amd.h"
#include "kernels.h"

namespace {

thread_local std::string g_last_error;
int g_w8a8_path = 0;  // 0 auto, 1 GEMV family, 2 MFMA family

// Automatic family for a W8A8 product of M rows, N output channels and K: the dot-product GEMV
// family (weights read once per 4 rows), or the INT8 MFMA family. Measured on MI355X with the
// weights cold, over M = 2 - 16 and 26 (K, N) pairs from 128 x 2048 to 1024 x 151936:
//  * M <= 2: the GEMV family everywhere;
//  * K whole 256-byte blocks (the LDS-staged chunk-row MFMA kernel): at M = 3 - 4 the MFMA family
//    from K = 4096 and N = 4096 (4096 x 4096: 6.2 -> 5.2 us; 3072 x 8192 stays: 7.0 against 8.0 us,
//    and so does every Qwen3-0.6B chunk shape, the head's 1024 x 151936 28.7 against 42.5 us); at
//    M = 5 - 8, where two GEMV row blocks read the weights twice, from N = 4096 (1024 x 6144, M = 6:
//    4.3 -> 3.6 us; N = 3072 ties); at M = 9 - 16 from N = 2048 (1024 x 3072, M = 12: 3.4 -> 3.0 us);
//  * other K (the direct MFMA kernel): the MFMA family at M = 9 - 16 from N = 3072 and K = 256
//    (1040 x 3072, M = 16: 5.8 -> 5.3 us) and at M = 5 - 16 from 12 MiB of weights (4112 x 4096,
//    M = 5: 11.5 -> 9.2 us); the GEMV family otherwise (128 x 4096, M = 16: 2.4 against 4.1 us);
//  * M > 16: the MFMA family.
bool use_gemv(int M, int N, int K) {
  if (g_w8a8_path != 0) return g_w8a8_path == 1;
  if (M <= 2) return true;
  if (K % 256 == 0) {
    if (M <= 4) return !(K >= 4096 && N >= 4096);
    if (M <= 8) return N < 4096;
    return M <= 16 && N < 2048;
  }
  if (M > 16) return false;
  const int64_t nk = static_cast<int64_t>(N) * K;
  return !((M >= 9 && N >= 3072 && K >= 256) || (M >= 5 && nk >= (12 << 20)));
}

// Automatic family for a K split of M rows, N output channels and ktot in all. Measured on MI355X
// with the weights cold at 4096 + 2816 and 3456 + 3456 (N = 1152), 4096 + 4096 (N = 2048) and
// 2048 + 2048 (N = 1024), M = 2 - 16: the GEMV family (weights read once per row block) at M <= 2;
// with every block whole 256-byte blocks, the chunk-row MFMA kernel at M = 3 from 12M weight bytes
// (4096 + 4096: 9.5 -> 7.6 us), at M = 4 - 8 from 6M (4096 + 2816, M = 4: 7.3 -> 6.7 us; M = 8:
// 11.8 -> 7.3 us) and at every M >= 9; otherwise the direct MFMA kernel from M = 5 (3456 + 3456:
// M = 4 7.4 against 10.4 us, M = 8 11.8 against 10.8 us).
bool use_gemv_ksplit(int M, int N, int ktot, bool chunk) {
  if (M <= 2) return true;
  if (!chunk) return M <= 4;
  const int64_t nk = static_cast<int64_t>(N) * ktot;
  if (M <= 3) return nk < (12 << 20);
  if (M <= 8) return nk < (6 << 20);
  return false;
}

int fail(int code, const char* what) {
  g_last_error = what;
  return code;
}

struct Span {
  uintptr_t lo, hi;  // [lo, hi)
};

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Row segments of a strided matrix: rows of `row_bytes` every `ld` bytes.
std::vector<Span> rows(const void* base, int64_t ld, int64_t nrows, int64_t row_bytes) {
  std::vector<Span> v;
  v.reserve(static_cast<size_t>(nrows));
  const uintptr_t b = reinterpret_cast<uintptr_t>(base);
  for (int64_t r = 0; r < nrows; ++r) v.push_back({b + static_cast<uintptr_t>(r * ld), b + static_cast<uintptr_t>(r * ld + row_bytes)});
  return v;
}

std::vector<Span> one(const void* base, int64_t bytes) {
  const uintptr_t b = reinterpret_cast<uintptr_t>(base);
  return {{b, b + static_cast<uintptr_t>(bytes)}};
}

// Whether any input segment intersects any output segment (outputs ascending and disjoint).
bool overlaps(const std::vector<Span>& in, const std::vector<Span>& out) {
  for (const Span& s : in) {
    auto it = std::upper_bound(out.begin(), out.end(), s.lo,
                               [](uintptr_t lo, const Span& o) { return lo < o.hi; });
    if (it != out.end() && it->lo < s.hi) return true;
  }
  return false;
}

// Extent check: ld * (rows - 1) + row_bytes stays inside the address space.
bool extent_ok(const void* base, int64_t ld, int64_t nrows, int64_t row_bytes) {
  if (nrows <= 0) return true;
  const unsigned __int128 end = static_cast<unsigned __int128>(reinterpret_cast<uintptr_t>(base)) +
                                static_cast<unsigned __int128>(ld) * static_cast<unsigned __int128>(nrows - 1) +
                                static_cast<unsigned __int128>(row_bytes);
  return end <= static_cast<unsigned __int128>(UINTPTR_MAX);
}

int esize(int out) { return out == TARS_OUT_FP32 ? 4 : (out == TARS_OUT_BF16 || out == TARS_OUT_FP16) ? 2 : 1; }

int check_epilogue(int act, int out, uint32_t out_scale_bits) {
  if (act < 0 || act > 7) return fail(TARS_E_FIELD, "act must be 0..7");
  if (out != TARS_OUT_FP32 && out != TARS_OUT_BF16 && out != TARS_OUT_INT8)
    return fail(TARS_E_FIELD, "out must be FP32, BF16 or INT8 (FP16 is not a GEMM output)");
  if (out != TARS_OUT_INT8 && out_scale_bits != 0)
    return fail(TARS_E_FIELD, "out_scale is only meaningful for INT8 output");
  return TARS_OK;
}

int launched(hipError_t e) {
  if (e != hipSuccess) {
    g_last_error = std::string("HIP launch failed: ") + hipGetErrorString(e);
    return TARS_E_DEVICE;
  }
  return TARS_OK;
}

float f32_of(uint32_t b) {
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}

}  // namespace

namespace tars {
// The calling thread's last-error text, shared by every entry point of the library.
void set_last_error(const std::string& what) { g_last_error = what; }
// The W8A8 kernel-family switch (tars_set_w8a8_path).
int w8a8_path() { return g_w8a8_path; }

// tars_quant_gemm_w8a8's checks and launch, with the gated product (QuantGemvArgs::prod) for the
// queue executor's MLP fusion: prod rows must not overlap an input, the quantized rows or Y1, and
// either are Y0's rows exactly (in place) or overlap no output. With pro (the executor's fusion of a
// residual ELT ADD and a norm in front of the quantizer): x is the ELT's A rows (the norm's input
// rows without B), pro's rows and vectors join the inputs and its sum and norm rows the outputs,
// and no output may overlap an input or another output (so no ELT in place).
int quant_gemm_w8a8_checked(const float* x, int64_t lda, int8_t* q, int64_t ldq, float* s, int32_t M, int32_t K,
                            const tars_w8a8_out* outs, int32_t nouts, float* prod, int64_t ldprod, void* stream,
                            const NormPrologue* pro) {
  g_last_error.clear();
  if (!x || !outs) return fail(TARS_E_ARG, "NULL pointer");
  if ((q == nullptr) != (s == nullptr)) return fail(TARS_E_ARG, "q and s are both given or both NULL");
  if (nouts < 1 || nouts > tars::kMaxGroups) return fail(TARS_E_ARG, "1 <= nouts <= 4");
  for (int i = 0; i < nouts; ++i) {
    const tars_w8a8_out& o = outs[i];
    if (!o.W || !o.scol || !o.Y) return fail(TARS_E_ARG, "NULL pointer in an output descriptor");
    if (int rc = check_epilogue(o.act, o.out, o.out_scale_bits)) return rc;
  }
  if (K > 65535) return fail(TARS_E_FIELD, "K must fit the 16-bit field (|acc| < 2^31)");
  if (M <= 0 || K <= 0 || K % 16) return fail(TARS_E_ALIGN, "M >= 1, K >= 16 and K % 16 == 0");
  if (lda == 0) lda = 4LL * K;
  if (q && ldq == 0) ldq = K;
  if (lda < 4LL * K || lda % 16 || (q && (ldq < K || ldq % 16)))
    return fail(TARS_E_ALIGN, "strides must be multiples of 16 holding a row");
  if (!aligned(x, 16) || (q && (!aligned(q, 16) || !aligned(s, 16)))) return fail(TARS_E_ALIGN, "pointers must be 16-byte aligned");
  std::vector<std::vector<Span>> yout(nouts);
  std::vector<int64_t> ldys(nouts);
  for (int i = 0; i < nouts; ++i) {
    const tars_w8a8_out& o = outs[i];
    const int64_t yrow = static_cast<int64_t>(o.N) * esize(o.out);
    ldys[i] = o.ldy == 0 ? yrow : o.ldy;
    if (o.N <= 0 || o.N % 16) return fail(TARS_E_ALIGN, "N >= 16 and N % 16 == 0");
    if (ldys[i] < yrow || ldys[i] % 16) return fail(TARS_E_ALIGN, "output stride must be a multiple of 16 holding a row");
    if (!aligned(o.W, 16) || !aligned(o.scol, 16) || !aligned(o.Y, 16) || (o.bias && !aligned(o.bias, 16)))
      return fail(TARS_E_ALIGN, "pointers must be 16-byte aligned");
    if (!extent_ok(o.W, K, o.N, K) || !extent_ok(o.Y, ldys[i], M, yrow)) return fail(TARS_E_RANGE, "extent overflows");
    yout[i] = rows(o.Y, ldys[i], M, yrow);
  }
  if (!extent_ok(x, lda, M, 4LL * K) || (q && !extent_ok(q, ldq, M, K))) return fail(TARS_E_RANGE, "extent overflows");
  // inputs: x and every matrix's W / scol / bias; outputs: q, s and every Y
  std::vector<Span> inputs = rows(x, lda, M, 4LL * K);
  for (int i = 0; i < nouts; ++i) {
    const tars_w8a8_out& o = outs[i];
    auto w = one(o.W, static_cast<int64_t>(o.N) * K), sc = one(o.scol, 4LL * o.N);
    inputs.insert(inputs.end(), w.begin(), w.end());
    inputs.insert(inputs.end(), sc.begin(), sc.end());
    if (o.bias) inputs.push_back(one(o.bias, 4LL * o.N)[0]);
  }
  std::vector<std::vector<Span>> outputs = yout;
  bool prod_in_place = false;
  if (prod) {  // the gated product: two fp32 matrices of one height, stored at prod (or in place over Y0)
    if (nouts != 2 || outs[0].N != outs[1].N || outs[0].out != 0 || outs[1].out != 0)
      return fail(TARS_E_ARG, "the gated product takes two fp32 outputs of one height");
    if (!tars::quant_gemv_pairs_supported(K)) return fail(TARS_E_FIELD, "the gated product is not available at this K");
    const int64_t prow = 4LL * outs[0].N;
    if (ldprod == 0) ldprod = prow;
    if (!aligned(prod, 16) || ldprod < prow || ldprod % 16) return fail(TARS_E_ALIGN, "product: 16-byte aligned rows");
    if (!extent_ok(prod, ldprod, M, prow)) return fail(TARS_E_RANGE, "extent overflows");
    prod_in_place = prod == outs[0].Y && (M == 1 || ldprod == ldys[0]);  // one row: the strides never apply
    if (!prod_in_place) outputs.push_back(rows(prod, ldprod, M, prow));
  }
  if (q) {
    outputs.push_back(rows(q, ldq, M, K));
    outputs.push_back(one(s, 4LL * M));
  }
  NormPrologue p{};
  if (pro) {
    p = *pro;
    if (p.fn != ROWFN_LAYERNORM && p.fn != ROWFN_RMSNORM && p.fn != ROWFN_L2NORM)
      return fail(TARS_E_FIELD, "the norm prologue takes a LayerNorm, RMSNorm or L2Norm");
    if (!tars::quant_gemv_norm_supported(K)) return fail(TARS_E_FIELD, "the norm prologue is not available at this K");
    if (M != 1) return fail(TARS_E_FIELD, "the norm prologue takes one row");
    if (!p.gamma || !p.y || (p.B != nullptr) != (p.sum != nullptr))
      return fail(TARS_E_ARG, "norm prologue: gamma and y, and B and sum together");
    const int64_t row = 4LL * K;
    if (p.ldb == 0) p.ldb = row;
    if (p.ldsum == 0) p.ldsum = row;
    if (p.ldy == 0) p.ldy = row;
    if ((p.B && (p.ldb < row || p.ldb % 16 || p.ldsum < row || p.ldsum % 16)) || p.ldy < row || p.ldy % 16)
      return fail(TARS_E_ALIGN, "norm prologue: strides must be multiples of 16 holding a row");
    if (!aligned(p.gamma, 16) || (p.beta && !aligned(p.beta, 16)) || !aligned(p.y, 16) ||
        (p.B && (!aligned(p.B, 16) || !aligned(p.sum, 16))))
      return fail(TARS_E_ALIGN, "norm prologue: pointers must be 16-byte aligned");
    if (!extent_ok(p.y, p.ldy, M, row) || (p.B && (!extent_ok(p.B, p.ldb, M, row) || !extent_ok(p.sum, p.ldsum, M, row))))
      return fail(TARS_E_RANGE, "extent overflows");
    inputs.push_back(one(p.gamma, row)[0]);
    if (p.beta) inputs.push_back(one(p.beta, row)[0]);
    if (p.B) {
      const auto b = rows(p.B, p.ldb, M, row);
      inputs.insert(inputs.end(), b.begin(), b.end());
      outputs.push_back(rows(p.sum, p.ldsum, M, row));
    }
    outputs.push_back(rows(p.y, p.ldy, M, row));
  }
  for (size_t i = 0; i < outputs.size(); ++i) {
    if (overlaps(inputs, outputs[i])) return fail(TARS_E_OVERLAP, "an output overlaps an input");
    for (size_t j = 0; j < i; ++j)
      if (overlaps(outputs[j], outputs[i])) return fail(TARS_E_OVERLAP, "two outputs overlap");
  }
  tars::QuantGemvArgs a{};
  a.x = x;
  a.lda = lda;
  a.q = q;
  a.ldq = ldq;
  a.s = s;
  a.M = M;
  a.K = K;
  a.ngroups = nouts;
  a.prod = prod;
  a.ldprod = ldprod;
  a.pro = p;
  for (int i = 0; i < nouts; ++i) {
    const tars_w8a8_out& o = outs[i];
    a.g[i].W = o.W;
    a.g[i].epi = tars::RowColEpilogue{nullptr, o.scol, 0, o.bias, o.act, o.out, f32_of(o.out_scale_bits)};
    a.g[i].Y = o.Y;
    a.g[i].ldy = ldys[i];
    a.g[i].N = o.N;
  }
  return launched(tars::launch_quant_gemv_w8a8(a, static_cast<hipStream_t>(stream)));
}

}  // namespace tars

extern "C" {

const char* tars_version(void) { return "opentars_amd 0.1.0 gfx950"; }

const char* tars_last_error(void) { return g_last_error.c_str(); }

int tars_set_w8a8_path(int path) {
  const int prev = g_w8a8_path;
  g_w8a8_path = (path >= 0 && path <= 2) ? path : 0;
  return prev;
}

int tars_quant_rows(const float* x, int64_t lda, int8_t* q, int64_t ldq, float* s, int32_t M,
                    int32_t K, void* stream) {
  g_last_error.clear();
  if (!x || !q || !s) return fail(TARS_E_ARG, "NULL pointer");
  if (M <= 0 || K <= 0 || K % 16) return fail(TARS_E_ALIGN, "M >= 1, K >= 16 and K % 16 == 0");
  if (lda == 0) lda = 4LL * K;
  if (ldq == 0) ldq = K;
  if (lda < 4LL * K || lda % 16 || ldq < K || ldq % 16)
    return fail(TARS_E_ALIGN, "strides must be multiples of 16 holding a row");
  if (!aligned(x, 16) || !aligned(q, 16) || !aligned(s, 16)) return fail(TARS_E_ALIGN, "pointers must be 16-byte aligned");
  if (!extent_ok(x, lda, M, 4LL * K) || !extent_ok(q, ldq, M, K)) return fail(TARS_E_RANGE, "extent overflows");
  const auto xin = rows(x, lda, M, 4LL * K);
  const auto qout = rows(q, ldq, M, K);
  const auto sout = one(s, 4LL * M);
  if (overlaps(xin, qout) || overlaps(xin, sout) || overlaps(sout, qout))
    return fail(TARS_E_OVERLAP, "an output overlaps an input");
  tars::QuantArgs a{x, lda, q, ldq, s, M, K};
  return launched(tars::launch_quant_rows(a, static_cast<hipStream_t>(stream)));
}

int tars_gemm_w8a8(const int8_t* A, int64_t lda, const float* srow, const int8_t* W,
                   const float* scol, int32_t scol_count, const float* bias, void* Y, int64_t ldy,
                   int32_t M, int32_t N, int32_t K, int32_t act, int32_t out,
                   uint32_t out_scale_bits, void* stream) {
  g_last_error.clear();
  if (!A || !W || !scol || !Y) return fail(TARS_E_ARG, "NULL pointer");
  if (int rc = check_epilogue(act, out, out_scale_bits)) return rc;
  if (scol_count != N && !(scol_count == 1 && srow == nullptr))
    return fail(TARS_E_FIELD, "scol_count must be N (or 1 without row scales)");
  if (K > 65535) return fail(TARS_E_FIELD, "K must fit the 16-bit field (|acc| < 2^31)");
  if (M <= 0 || N <= 0 || N % 16 || K <= 0 || K % 16) return fail(TARS_E_ALIGN, "M, N, K >= 1; N % 16 == 0; K % 16 == 0");
  const int64_t yrow = static_cast<int64_t>(N) * esize(out);
  if (lda == 0) lda = K;
  if (ldy == 0) ldy = yrow;
  if (lda < K || lda % 16 || ldy < yrow || ldy % 16) return fail(TARS_E_ALIGN, "strides must be multiples of 16 holding a row");
  if (!aligned(A, 16) || !aligned(W, 16) || !aligned(scol, 16) || !aligned(Y, 16) ||
      (srow && !aligned(srow, 16)) || (bias && !aligned(bias, 16)))
    return fail(TARS_E_ALIGN, "pointers must be 16-byte aligned");
  if (!extent_ok(A, lda, M, K) || !extent_ok(W, K, N, K) || !extent_ok(Y, ldy, M, yrow))
    return fail(TARS_E_RANGE, "extent overflows");
  const auto yout = rows(Y, ldy, M, yrow);
  if (overlaps(rows(A, lda, M, K), yout) || overlaps(one(W, static_cast<int64_t>(N) * K), yout) ||
      overlaps(one(scol, 4LL * scol_count), yout) || (srow && overlaps(one(srow, 4LL * M), yout)) ||
      (bias && overlaps(one(bias, 4LL * N), yout)))
    return fail(TARS_E_OVERLAP, "the output overlaps an input");
  tars::W8A8Args a{};
  a.A = A;
  a.lda = lda;
  a.W = W;
  a.epi = tars::RowColEpilogue{srow, scol, scol_count == 1 && N != 1 ? 1 : 0, bias, act, out,
                               f32_of(out_scale_bits)};
  a.Y = Y;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  const bool gemv = use_gemv(M, N, K);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return launched(gemv ? tars::launch_gemv_w8a8(a, s) : tars::launch_gemm_w8a8_mfma(a, s));
}

int tars_quant_gemm_w8a8(const float* x, int64_t lda, int8_t* q, int64_t ldq, float* s,
                         int32_t M, int32_t K, const tars_w8a8_out* outs, int32_t nouts,
                         void* stream) {
  return tars::quant_gemm_w8a8_checked(x, lda, q, ldq, s, M, K, outs, nouts, nullptr, 0, stream, nullptr);
}

int tars_gemm_w8a8_ksplit(const int8_t* A, int64_t lda, const float* srow,
                          const int8_t* const* W_blocks, const int32_t* K_blocks, int32_t nblocks,
                          const float* scol, float* Y, int64_t ldy, int32_t M, int32_t N,
                          void* stream) {
  g_last_error.clear();
  if (!A || !scol || !Y || !W_blocks || !K_blocks) return fail(TARS_E_ARG, "NULL pointer");
  if (nblocks < 1 || nblocks > tars::kMaxBlocks) return fail(TARS_E_ARG, "1 <= nblocks <= 8");
  int64_t ktot = 0;
  for (int i = 0; i < nblocks; ++i) {
    if (!W_blocks[i]) return fail(TARS_E_ARG, "NULL weight block");
    if (K_blocks[i] > 65535) return fail(TARS_E_FIELD, "block K must fit the 16-bit field");
    if (K_blocks[i] <= 0 || K_blocks[i] % 16) return fail(TARS_E_ALIGN, "block K >= 16 and % 16 == 0");
    if (!aligned(W_blocks[i], 16)) return fail(TARS_E_ALIGN, "weight blocks must be 16-byte aligned");
    ktot += K_blocks[i];
  }
  if (M <= 0 || N <= 0 || N % 16) return fail(TARS_E_ALIGN, "M, N >= 1; N % 16 == 0");
  if (lda == 0) lda = ktot;
  if (ldy == 0) ldy = 4LL * N;
  if (lda < ktot || lda % 16 || ldy < 4LL * N || ldy % 16) return fail(TARS_E_ALIGN, "strides must be multiples of 16 holding a row");
  if (!aligned(A, 16) || !aligned(scol, 16) || !aligned(Y, 16) || (srow && !aligned(srow, 16)))
    return fail(TARS_E_ALIGN, "pointers must be 16-byte aligned");
  if (!extent_ok(A, lda, M, ktot) || !extent_ok(Y, ldy, M, 4LL * N)) return fail(TARS_E_RANGE, "extent overflows");
  const auto yout = rows(Y, ldy, M, 4LL * N);
  bool ov = overlaps(rows(A, lda, M, ktot), yout) || overlaps(one(scol, 4LL * N), yout) ||
            (srow && overlaps(one(srow, 4LL * M), yout));
  for (int i = 0; i < nblocks && !ov; ++i) ov = overlaps(one(W_blocks[i], static_cast<int64_t>(N) * K_blocks[i]), yout);
  if (ov) return fail(TARS_E_OVERLAP, "the output overlaps an input");
  tars::KSplitArgs a{};
  a.A = A;
  a.lda = lda;
  a.srow = srow;
  a.scol = scol;
  int koff = 0;
  for (int i = 0; i < nblocks; ++i) {
    a.W[i] = W_blocks[i];
    a.K[i] = K_blocks[i];
    a.koff[i] = koff;
    koff += K_blocks[i];
  }
  a.nblocks = nblocks;
  a.Y = Y;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  bool chunk = true;  // every block a whole number of 256-byte blocks: the MFMA family's chunk-row kernel
  for (int i = 0; i < nblocks; ++i) chunk = chunk && K_blocks[i] % 256 == 0;
  const bool gemv = g_w8a8_path == 1 || (g_w8a8_path == 0 && use_gemv_ksplit(M, N, ktot, chunk));
  hipStream_t s = static_cast<hipStream_t>(stream);
  return launched(gemv ? tars::launch_gemv_w8a8_ksplit(a, s) : tars::launch_gemm_w8a8_ksplit_mfma(a, s));
}

int tars_align_w4(const void* x, int64_t lda, int32_t a_dtype, int16_t* q, int64_t ldq,
                  float* scales, int64_t lds, int32_t M, int32_t K, void* stream) {
  g_last_error.clear();
  if (!x || !q || !scales) return fail(TARS_E_ARG, "NULL pointer");
  if (a_dtype != TARS_DT_FP32 && a_dtype != TARS_DT_BF16) return fail(TARS_E_FIELD, "a_dtype must be FP32 or BF16");
  if (M <= 0 || K <= 0 || K % 128) return fail(TARS_E_ALIGN, "M >= 1 and K a nonzero multiple of 128");
  const int64_t xrow = static_cast<int64_t>(K) * (a_dtype == TARS_DT_FP32 ? 4 : 2);
  const int64_t srow_bytes = 4LL * (K / 128);
  if (lda == 0) lda = xrow;
  if (ldq == 0) ldq = 2LL * K;
  if (lds == 0) lds = srow_bytes;
  if (lda < xrow || lda % 16 || ldq < 2LL * K || ldq % 16 || lds < srow_bytes || lds % 4)
    return fail(TARS_E_ALIGN, "strides must hold a row (x and q multiples of 16, scales of 4)");
  if (!aligned(x, 16) || !aligned(q, 16) || !aligned(scales, 4)) return fail(TARS_E_ALIGN, "pointer alignment");
  if (!extent_ok(x, lda, M, xrow) || !extent_ok(q, ldq, M, 2LL * K) || !extent_ok(scales, lds, M, srow_bytes))
    return fail(TARS_E_RANGE, "extent overflows");
  const auto xin = rows(x, lda, M, xrow);
  const auto qout = rows(q, ldq, M, 2LL * K);
  const auto sout = rows(scales, lds, M, srow_bytes);
  if (overlaps(xin, qout) || overlaps(xin, sout) || overlaps(sout, qout))
    return fail(TARS_E_OVERLAP, "an output overlaps an input");
  tars::AlignArgs a{x, lda, a_dtype == TARS_DT_BF16 ? 1 : 0, q, ldq, scales, lds, M, K};
  return launched(tars::launch_align_w4(a, static_cast<hipStream_t>(stream)));
}

int tars_gemm_w4a16(const void* x, int64_t lda, int32_t a_dtype, const uint8_t* Wp,
                    const uint16_t* ws, const float* bias, void* Y, int64_t ldy, int32_t M,
                    int32_t N, int32_t K, int32_t act, int32_t out, uint32_t out_scale_bits,
                    void* stream) {
  g_last_error.clear();
  if (!x || !Wp || !ws || !Y) return fail(TARS_E_ARG, "NULL pointer");
  if (a_dtype != TARS_DT_FP32 && a_dtype != TARS_DT_BF16) return fail(TARS_E_FIELD, "a_dtype must be FP32 or BF16");
  if (int rc = check_epilogue(act, out, out_scale_bits)) return rc;
  if (M <= 0 || N <= 0 || N % 16 || K <= 0 || K % 16) return fail(TARS_E_ALIGN, "M, N, K >= 1; N % 16 == 0; K % 16 == 0");
  if (K < 256 || K % 256 || K > 8192 || !aligned(Wp, 128))
    return fail(TARS_E_ALIGN, "W4A16: K % 256 == 0, 256 <= K <= 8192, weights 128-byte aligned");
  const int64_t xrow = static_cast<int64_t>(K) * (a_dtype == TARS_DT_FP32 ? 4 : 2);
  const int64_t yrow = static_cast<int64_t>(N) * esize(out);
  if (lda == 0) lda = xrow;
  if (ldy == 0) ldy = yrow;
  if (lda < xrow || lda % 16 || ldy < yrow || ldy % 16) return fail(TARS_E_ALIGN, "strides must be multiples of 16 holding a row");
  if (!aligned(x, 16) || !aligned(ws, 16) || !aligned(Y, 16) || (bias && !aligned(bias, 16)))
    return fail(TARS_E_ALIGN, "pointers must be 16-byte aligned");
  if (!extent_ok(x, lda, M, xrow) || !extent_ok(Y, ldy, M, yrow)) return fail(TARS_E_RANGE, "extent overflows");
  const auto yout = rows(Y, ldy, M, yrow);
  if (overlaps(rows(x, lda, M, xrow), yout) || overlaps(one(Wp, static_cast<int64_t>(N) * K / 2), yout) ||
      overlaps(one(ws, 2LL * N * (K / 128)), yout) || (bias && overlaps(one(bias, 4LL * N), yout)))
    return fail(TARS_E_OVERLAP, "the output overlaps an input");
  tars::W4Args a{};
  a.x = x;
  a.lda = lda;
  a.bf16 = a_dtype == TARS_DT_BF16 ? 1 : 0;
  a.Wp = Wp;
  a.ws = ws;
  a.bias = bias;
  a.act = act;
  a.out = out;
  a.out_scale = f32_of(out_scale_bits);
  a.Y = Y;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  return launched(tars::launch_gemv_w4a16(a, static_cast<hipStream_t>(stream)));
}

// ------------------------------------------------------------------ fp32 row / elementwise / dot ops
// Shared rules: M, N (and K) >= 1; fp32 data 4-byte aligned, fp16 data 2-byte aligned, the output
// aligned to its element; strides 0 (dense) or multiples of the element size holding a row; act
// 0..7; out FP32 / BF16 / INT8 (and FP16 for ELT); out_scale only with INT8.
}  // extern "C"

namespace {

int check_out(int out, uint32_t out_scale_bits, bool fp16_ok) {
  if (out < 0 || out > 3 || (out == TARS_OUT_FP16 && !fp16_ok))
    return fail(TARS_E_FIELD, fp16_ok ? "out must be FP32, BF16, INT8 or FP16" : "out must be FP32, BF16 or INT8");
  if (out != TARS_OUT_INT8 && out_scale_bits != 0) return fail(TARS_E_FIELD, "out_scale is only meaningful for INT8 output");
  return TARS_OK;
}

// A row stride: 0 -> dense; else a multiple of the element size holding a row.
bool stride_ok(int64_t& ld, int64_t row_bytes, int elem) {
  if (ld == 0) ld = row_bytes;
  return ld >= row_bytes && ld % elem == 0;
}

// Whether the spans (any order) are pairwise disjoint; sorts them by start.
bool disjoint(std::vector<Span>& v) {
  std::sort(v.begin(), v.end(), [](const Span& x, const Span& y) { return x.lo < y.lo; });
  for (size_t i = 1; i < v.size(); ++i)
    if (v[i].lo < v[i - 1].hi) return false;
  return true;
}

// The checks of tars_attention, in the order of the other entry points (NULLs, fields, shapes and
// alignment, extents, overlaps), and its kernel arguments.
int attention_args(const float* const* q, int64_t ldq, const float* const* k, int64_t ldk, const void* const* v,
                   int64_t ldv, int32_t v_fp16, void* const* att, int64_t ldatt, int32_t out, uint32_t out_scale_bits,
                   float* sc, int64_t ldsc, float* pr, int64_t ldpr, int32_t heads, int32_t M, int32_t nk, int32_t hd,
                   int32_t causal_k, tars::AttnArgs& a) {
  g_last_error.clear();
  if (!q || !k || !v || !att) return fail(TARS_E_ARG, "NULL pointer array");
  if (heads < 1 || heads > tars::kAttnMaxHeads) return fail(TARS_E_ARG, "heads must be 1..32");
  for (int32_t h = 0; h < heads; ++h)
    if (!q[h] || !k[h] || !v[h] || !att[h]) return fail(TARS_E_ARG, "NULL pointer");
  if (v_fp16 != 0 && v_fp16 != 1) return fail(TARS_E_FIELD, "v_fp16 is 0 or 1");
  if (int rc = check_out(out, out_scale_bits, false)) return rc;
  if (causal_k < 0) return fail(TARS_E_FIELD, "causal_k >= 0");
  if (M < 1 || nk < 1) return fail(TARS_E_ALIGN, "M, nk >= 1");
  if (!tars::attention_supported(hd, nk)) return fail(TARS_E_ARG, "head size 64, 128 or 256 and at most 4080 keys");
  const int ve = v_fp16 ? 2 : 4, oe = esize(out);
  const int64_t qrow = 4LL * hd, vrow = static_cast<int64_t>(ve) * hd, arow = static_cast<int64_t>(oe) * hd,
                srow = 4LL * nk;
  if (!stride_ok(ldq, qrow, 16) || !stride_ok(ldk, qrow, 16) || !stride_ok(ldv, vrow, 16) ||
      !stride_ok(ldatt, arow, 16) || !stride_ok(ldsc, srow, 16) || !stride_ok(ldpr, srow, 16))
    return fail(TARS_E_ALIGN, "strides must hold a row and be multiples of 16 bytes");
  if (!aligned(sc, 16) || !aligned(pr, 16)) return fail(TARS_E_ALIGN, "pointers must be 16-byte aligned");
  std::vector<Span> ins, outs;
  for (int32_t h = 0; h < heads; ++h) {
    if (!aligned(q[h], 16) || !aligned(k[h], 16) || !aligned(v[h], 16) || !aligned(att[h], 16))
      return fail(TARS_E_ALIGN, "pointers must be 16-byte aligned");
    if (!extent_ok(q[h], ldq, M, qrow) || !extent_ok(k[h], ldk, nk, qrow) || !extent_ok(v[h], ldv, nk, vrow) ||
        !extent_ok(att[h], ldatt, M, arow))
      return fail(TARS_E_RANGE, "extent overflows");
    auto add = [](std::vector<Span>& to, std::vector<Span> from) { to.insert(to.end(), from.begin(), from.end()); };
    add(ins, rows(q[h], ldq, M, qrow));
    if (h == 0 || k[h] != k[h - 1]) add(ins, rows(k[h], ldk, nk, qrow));  // heads sharing K / V: their rows once
    if (h == 0 || v[h] != v[h - 1]) add(ins, rows(v[h], ldv, nk, vrow));
    add(outs, rows(att[h], ldatt, M, arow));
  }
  if ((sc && !extent_ok(sc, ldsc, M, srow)) || (pr && !extent_ok(pr, ldpr, M, srow)))
    return fail(TARS_E_RANGE, "extent overflows");
  if (sc) {
    const auto r = rows(sc, ldsc, M, srow);
    outs.insert(outs.end(), r.begin(), r.end());
  }
  if (pr) {
    const auto r = rows(pr, ldpr, M, srow);
    outs.insert(outs.end(), r.begin(), r.end());
  }
  if (!disjoint(outs) || overlaps(ins, outs)) return fail(TARS_E_OVERLAP, "an output overlaps another output or an input");
  for (int32_t h = 0; h < heads; ++h) {
    a.q[h] = q[h];
    a.k[h] = k[h];
    a.v[h] = v[h];
    a.att[h] = att[h];
  }
  a.ldq = ldq;
  a.ldk = ldk;
  a.ldv = ldv;
  a.ldatt = ldatt;
  a.sc = sc;
  a.ldsc = ldsc;
  a.pr = pr;
  a.ldpr = ldpr;
  a.heads = heads;
  a.M = M;
  a.nk = nk;
  a.hd = hd;
  a.causal_k = causal_k;
  a.v_fp16 = v_fp16;
  a.out = out;
  a.out_scale = f32_of(out_scale_bits);
  return TARS_OK;
}

}  // namespace

extern "C" {

int tars_row_op(const float* x, int64_t lda, int32_t fn, const float* gamma, const float* beta, uint32_t eps_bits,
                int32_t causal_k, const int32_t* valid, void* y, int64_t ldy, int32_t out, uint32_t out_scale_bits,
                int32_t M, int32_t N, void* stream) {
  g_last_error.clear();
  if (!x || !y) return fail(TARS_E_ARG, "NULL pointer");
  if (fn < TARS_ROW_SOFTMAX || fn > TARS_ROW_L2NORM) return fail(TARS_E_FIELD, "fn must be SOFTMAX, LAYERNORM, RMSNORM or L2NORM");
  if (int rc = check_out(out, out_scale_bits, false)) return rc;
  const bool softmax = fn == TARS_ROW_SOFTMAX;
  if (softmax && (gamma || beta || eps_bits)) return fail(TARS_E_FIELD, "softmax takes no gamma, beta or eps");
  if (!softmax && (causal_k || valid)) return fail(TARS_E_FIELD, "only softmax is causal");
  if (!softmax && !gamma) return fail(TARS_E_ARG, "the norms need gamma");
  if (causal_k < 0) return fail(TARS_E_FIELD, "causal_k must be >= 0");
  if (M <= 0 || N <= 0) return fail(TARS_E_ALIGN, "M, N >= 1");
  const int64_t xrow = 4LL * N, yrow = static_cast<int64_t>(N) * esize(out);
  if (!stride_ok(lda, xrow, 4) || !stride_ok(ldy, yrow, esize(out))) return fail(TARS_E_ALIGN, "strides must hold a row");
  if (!aligned(x, 4) || !aligned(y, esize(out)) || (gamma && !aligned(gamma, 4)) || (beta && !aligned(beta, 4)) ||
      (valid && !aligned(valid, 4)))
    return fail(TARS_E_ALIGN, "pointer alignment");
  if (!extent_ok(x, lda, M, xrow) || !extent_ok(y, ldy, M, yrow)) return fail(TARS_E_RANGE, "extent overflows");
  const auto yout = rows(y, ldy, M, yrow);
  if (overlaps(rows(x, lda, M, xrow), yout) || (gamma && overlaps(one(gamma, xrow), yout)) ||
      (beta && overlaps(one(beta, xrow), yout)) || (valid && overlaps(one(valid, 4LL * M), yout)))
    return fail(TARS_E_OVERLAP, "the output overlaps an input");
  tars::RowArgs a{x, lda, fn, gamma, beta, f32_of(eps_bits), causal_k, valid, y, ldy, out, f32_of(out_scale_bits), M, N};
  return launched(tars::launch_row(a, static_cast<hipStream_t>(stream)));
}

int tars_elt(const void* A, int64_t lda, int32_t a_fp16, int32_t a_row, const float* B, int64_t ldb, int32_t bmode,
             const void* C, int64_t ldc, int32_t op, int32_t act, void* Y, int64_t ldy, int32_t out,
             uint32_t out_scale_bits, int32_t M, int32_t N, void* stream) {
  g_last_error.clear();
  if (!A || !B || !Y || (op == TARS_ELT_MULADD && !C)) return fail(TARS_E_ARG, "NULL pointer");
  if (op < TARS_ELT_MUL || op > TARS_ELT_SUB) return fail(TARS_E_FIELD, "op must be MUL, ADD, MULADD or SUB");
  if (bmode < TARS_BM_DENSE || bmode > TARS_BM_SCALAR) return fail(TARS_E_FIELD, "bmode must be DENSE, ROW, COL or SCALAR");
  if (act < 0 || act > 7) return fail(TARS_E_FIELD, "act must be 0..7");
  if ((a_fp16 != 0 && a_fp16 != 1) || (a_row != 0 && a_row != 1)) return fail(TARS_E_FIELD, "a_fp16 and a_row are 0 or 1");
  if (int rc = check_out(out, out_scale_bits, true)) return rc;
  if (op == TARS_ELT_MULADD && out != TARS_OUT_FP32 && out != TARS_OUT_FP16)
    return fail(TARS_E_FIELD, "MULADD adds C in the output format: out must be FP32 or FP16");
  if (op != TARS_ELT_MULADD && C) return fail(TARS_E_FIELD, "C is only read by MULADD");
  if (M <= 0 || N <= 0) return fail(TARS_E_ALIGN, "M, N >= 1");
  const int ae = a_fp16 ? 2 : 4, ye = esize(out), ce = out == TARS_OUT_FP16 ? 2 : 4;
  const int64_t arow = static_cast<int64_t>(ae) * N, yrow = static_cast<int64_t>(ye) * N, crow = static_cast<int64_t>(ce) * N;
  if (!stride_ok(lda, arow, ae) || !stride_ok(ldy, yrow, ye) || (op == TARS_ELT_MULADD && !stride_ok(ldc, crow, ce)) ||
      (bmode == TARS_BM_DENSE && !stride_ok(ldb, 4LL * N, 4)))
    return fail(TARS_E_ALIGN, "strides must hold a row");
  if (!aligned(A, ae) || !aligned(B, 4) || !aligned(Y, ye) || (C && !aligned(C, ce))) return fail(TARS_E_ALIGN, "pointer alignment");
  const int64_t am = a_row ? 1 : M;
  const int64_t bbytes = bmode == TARS_BM_ROW ? 4LL * N : bmode == TARS_BM_COL ? 4LL * M : 4;
  if (!extent_ok(A, lda, am, arow) || !extent_ok(Y, ldy, M, yrow) || (C && !extent_ok(C, ldc, M, crow)) ||
      (bmode == TARS_BM_DENSE && !extent_ok(B, ldb, M, 4LL * N)))
    return fail(TARS_E_RANGE, "extent overflows");
  // In place (golden.py:440-448): Y may be A itself (same format and stride, not a broadcast row)
  // or C itself (same stride); any other overlap of an input with Y is refused.
  const bool a_inplace = A == Y && !a_row && lda == ldy &&
                         (a_fp16 ? out == TARS_OUT_FP16 : out == TARS_OUT_FP32);
  const bool c_inplace = C && C == Y && ldc == ldy;
  const auto yout = rows(Y, ldy, M, yrow);
  if ((!a_inplace && overlaps(rows(A, lda, am, arow), yout)) ||
      (bmode == TARS_BM_DENSE ? overlaps(rows(B, ldb, M, 4LL * N), yout) : overlaps(one(B, bbytes), yout)) ||
      (C && !c_inplace && overlaps(rows(C, ldc, M, crow), yout)))
    return fail(TARS_E_OVERLAP, "the output overlaps an input");
  tars::EltArgs a{A, lda, a_fp16, a_row, B, ldb, bmode, C, ldc, op, act, Y, ldy, out, f32_of(out_scale_bits), M, N};
  return launched(tars::launch_elt(a, static_cast<hipStream_t>(stream)));
}

int tars_rope(const float* x, int64_t lda, const float* tab, int32_t rows_per_pos, int32_t rot, void* y, int64_t ldy,
              int32_t out, uint32_t out_scale_bits, int32_t M, int32_t N, void* stream) {
  g_last_error.clear();
  if (!x || !tab || !y) return fail(TARS_E_ARG, "NULL pointer");
  if (int rc = check_out(out, out_scale_bits, false)) return rc;
  if (M <= 0 || N <= 0 || rows_per_pos <= 0 || rot <= 0 || rot % 2 || rot > N)
    return fail(TARS_E_ALIGN, "M, N >= 1; rows_per_pos >= 1; rot even, 2 <= rot <= N");
  const int64_t xrow = 4LL * N, yrow = static_cast<int64_t>(N) * esize(out);
  const int64_t tab_bytes = 4LL * rot * ((M - 1) / rows_per_pos + 1);
  if (!stride_ok(lda, xrow, 4) || !stride_ok(ldy, yrow, esize(out))) return fail(TARS_E_ALIGN, "strides must hold a row");
  if (!aligned(x, 4) || !aligned(tab, 4) || !aligned(y, esize(out))) return fail(TARS_E_ALIGN, "pointer alignment");
  if (!extent_ok(x, lda, M, xrow) || !extent_ok(y, ldy, M, yrow) || !extent_ok(tab, tab_bytes, 1, tab_bytes))
    return fail(TARS_E_RANGE, "extent overflows");
  const auto yout = rows(y, ldy, M, yrow);
  if (overlaps(rows(x, lda, M, xrow), yout) || overlaps(one(tab, tab_bytes), yout))
    return fail(TARS_E_OVERLAP, "the output overlaps an input");
  tars::RopeArgs a{x, lda, tab, rows_per_pos, rot, y, ldy, out, f32_of(out_scale_bits), M, N};
  return launched(tars::launch_rope(a, static_cast<hipStream_t>(stream)));
}

int tars_relu(const float* x, int64_t lda, int32_t act, void* y, int64_t ldy, int32_t out, uint32_t out_scale_bits,
              int32_t M, int32_t N, void* stream) {
  g_last_error.clear();
  if (!x || !y) return fail(TARS_E_ARG, "NULL pointer");
  if (act < 0 || act > 7) return fail(TARS_E_FIELD, "act must be 0..7");
  if (int rc = check_out(out, out_scale_bits, false)) return rc;
  if (M <= 0 || N <= 0) return fail(TARS_E_ALIGN, "M, N >= 1");
  const int64_t xrow = 4LL * N, yrow = static_cast<int64_t>(N) * esize(out);
  if (!stride_ok(lda, xrow, 4) || !stride_ok(ldy, yrow, esize(out))) return fail(TARS_E_ALIGN, "strides must hold a row");
  if (!aligned(x, 4) || !aligned(y, esize(out))) return fail(TARS_E_ALIGN, "pointer alignment");
  if (!extent_ok(x, lda, M, xrow) || !extent_ok(y, ldy, M, yrow)) return fail(TARS_E_RANGE, "extent overflows");
  if (overlaps(rows(x, lda, M, xrow), rows(y, ldy, M, yrow))) return fail(TARS_E_OVERLAP, "the output overlaps an input");
  tars::ReluArgs a{x, lda, act, y, ldy, out, f32_of(out_scale_bits), M, N};
  return launched(tars::launch_relu(a, static_cast<hipStream_t>(stream)));
}

int tars_fdot(const float* A, int64_t lda, const void* B, int64_t ldb, int32_t nn, int32_t b_fp16, void* Y, int64_t ldy,
              int32_t out, uint32_t out_scale_bits, int32_t M, int32_t N, int32_t K, void* stream) {
  g_last_error.clear();
  if (!A || !B || !Y) return fail(TARS_E_ARG, "NULL pointer");
  if ((nn != 0 && nn != 1) || (b_fp16 != 0 && b_fp16 != 1)) return fail(TARS_E_FIELD, "nn and b_fp16 are 0 or 1");
  if (b_fp16 && !nn) return fail(TARS_E_FIELD, "an fp16 B is read only by the NN form");
  if (int rc = check_out(out, out_scale_bits, false)) return rc;
  if (M <= 0 || N <= 0 || K <= 0) return fail(TARS_E_ALIGN, "M, N, K >= 1");
  const int be = b_fp16 ? 2 : 4;
  const int64_t arow = 4LL * K, brow = static_cast<int64_t>(be) * (nn ? N : K), bn = nn ? K : N;
  const int64_t yrow = static_cast<int64_t>(N) * esize(out);
  if (!stride_ok(lda, arow, 4) || !stride_ok(ldb, brow, be) || !stride_ok(ldy, yrow, esize(out)))
    return fail(TARS_E_ALIGN, "strides must hold a row");
  if (!aligned(A, 4) || !aligned(B, be) || !aligned(Y, esize(out))) return fail(TARS_E_ALIGN, "pointer alignment");
  if (!extent_ok(A, lda, M, arow) || !extent_ok(B, ldb, bn, brow) || !extent_ok(Y, ldy, M, yrow))
    return fail(TARS_E_RANGE, "extent overflows");
  const auto yout = rows(Y, ldy, M, yrow);
  if (overlaps(rows(A, lda, M, arow), yout) || overlaps(rows(B, ldb, bn, brow), yout))
    return fail(TARS_E_OVERLAP, "the output overlaps an input");
  tars::FdotArgs a{A, lda, B, ldb, nn, b_fp16, Y, ldy, out, f32_of(out_scale_bits), M, N, K};
  return launched(tars::launch_fdot(a, static_cast<hipStream_t>(stream)));
}

int tars_attention(const float* const* q, int64_t ldq, const float* const* k, int64_t ldk, const void* const* v,
                   int64_t ldv, int32_t v_fp16, void* const* att, int64_t ldatt, int32_t out, uint32_t out_scale_bits,
                   float* sc, int64_t ldsc, float* pr, int64_t ldpr, int32_t heads, int32_t M, int32_t nk, int32_t hd,
                   int32_t causal_k, void* stream) {
  tars::AttnArgs a{};
  if (int rc = attention_args(q, ldq, k, ldk, v, ldv, v_fp16, att, ldatt, out, out_scale_bits, sc, ldsc, pr, ldpr, heads,
                              M, nk, hd, causal_k, a))
    return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  a.scratch = tars::attention_workspace(s);
  a.scratch_floats = a.scratch ? tars::kAttnScratchFloats : 0;
  return launched(tars::launch_attention(a, s));
}

int tars_attention_noalloc(const float* const* q, int64_t ldq, const float* const* k, int64_t ldk, const void* const* v,
                           int64_t ldv, int32_t v_fp16, void* const* att, int64_t ldatt, int32_t out,
                           uint32_t out_scale_bits, float* sc, int64_t ldsc, float* pr, int64_t ldpr, int32_t heads,
                           int32_t M, int32_t nk, int32_t hd, int32_t causal_k, void* stream) {
  tars::AttnArgs a{};
  if (int rc = attention_args(q, ldq, k, ldk, v, ldv, v_fp16, att, ldatt, out, out_scale_bits, sc, ldsc, pr, ldpr, heads,
                              M, nk, hd, causal_k, a))
    return rc;
  const int64_t need = static_cast<int64_t>(heads) * M * ((nk + 3) / 4 * 4);
  if (need > tars::kAttnScratchFloats)
    return fail(TARS_E_RANGE, "heads * M * nk (nk rounded up to 4) exceeds the 262144 floats of the static scratch");
  a.scratch = tars::attention_static_scratch();
  if (!a.scratch) return fail(TARS_E_DEVICE, "the static scratch has no device address on this device");
  a.scratch_floats = tars::kAttnScratchFloats;
  return launched(tars::launch_attention(a, static_cast<hipStream_t>(stream)));
}

int tars_embed_rows(const uint16_t* table, int64_t ld_table, int64_t table_rows, int32_t cols, const int32_t* ids,
                    int32_t n, int32_t scaled, uint32_t scale_bits, float* dst, int64_t ldd, void* stream) {
  g_last_error.clear();
  if (!table || !ids || !dst) return fail(TARS_E_ARG, "NULL pointer");
  if (scaled != 0 && scaled != 1) return fail(TARS_E_FIELD, "scaled is 0 or 1");
  if (table_rows <= 0 || cols <= 0 || n <= 0) return fail(TARS_E_ALIGN, "rows, cols, n >= 1");
  if (!stride_ok(ld_table, 2LL * cols, 2) || !stride_ok(ldd, 4LL * cols, 4)) return fail(TARS_E_ALIGN, "strides must hold a row");
  if (!aligned(table, 2) || !aligned(dst, 4)) return fail(TARS_E_ALIGN, "pointer alignment");
  for (int32_t i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= table_rows) return fail(TARS_E_RANGE, "a token id lies outside the table");
  if (!extent_ok(table, ld_table, table_rows, 2LL * cols) || !extent_ok(dst, ldd, n, 4LL * cols))
    return fail(TARS_E_RANGE, "extent overflows");
  // the table as one span (its row gaps included): a per-row list would cost a host pass over
  // every vocabulary row per call
  if (overlaps(one(table, ld_table * (table_rows - 1) + 2LL * cols), rows(dst, ldd, n, 4LL * cols)))
    return fail(TARS_E_OVERLAP, "the output overlaps the table");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  for (int32_t i0 = 0; i0 < n; i0 += tars::kEmbedMaxIds) {
    tars::EmbedArgs a{};
    a.table = table;
    a.ld_table = ld_table;
    a.n = std::min<int32_t>(tars::kEmbedMaxIds, n - i0);
    a.dst = reinterpret_cast<float*>(reinterpret_cast<char*>(dst) + static_cast<int64_t>(i0) * ldd);
    a.ldd = ldd;
    a.cols = cols;
    a.scaled = scaled;
    a.scale_bits = scale_bits;
    for (int32_t j = 0; j < a.n; ++j) a.ids[j] = ids[i0 + j];
    if (int rc = launched(tars::launch_embed_rows(a, s))) return rc;
  }
  return TARS_OK;
}

}  // extern "C"
