// Descriptor-queue executor over a DDR image held in device memory (tars_mini/golden.py:450-492
// run_queue, with golden.py:59-169 validate, :172-258 strides / segments / extra_out and
// :260-267 / :440-448 the overlap rules; tars_mini/contract.py:14-38 the 512-bit layout and
// :154-181 encode / decode / CRC).
//
// Host side: the descriptors are read from the image once (one device-to-host copy; or taken from
// the caller's host copy of the same bytes), decoded,
// CRC-checked and validated in the contract's order, their byte segments range- and overlap-
// checked; every descriptor the GPU runs (W8A8 GEMM in QM_TENSOR / QM_CHANNEL / QM_ROWCOL, the
// W4A16 group GEMM, ROW_QUANT) is then enqueued on the caller's stream with pointers into the
// image, in queue order, so each one sees every earlier write (stream order). The queue stops at
// the first invalid descriptor (its ERR_CODE and index, earlier writes kept), at an output that
// overlaps an input (the golden's ContractError), or at a valid descriptor of another kind, which
// is handed back to the caller (host_op = 1). A descriptor whose output lands on a later
// descriptor of the same queue makes the executor wait for it and re-read the rest of the queue.
// A decode-row ROW_QUANT and the QM_ROWCOL GEMMs that read it run as one fused launch (peephole
// fusion, bit-identical to the one-by-one order; see fuse_group).
#include <algorithm>
#include <atomic>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "../../include/opentars_amd.h"
#include "kernels.h"

namespace {

typedef unsigned __int128 u128;

// ---------------------------------------------------------------------------- descriptor fields
// Field order and (low bit, width) of the 512-bit descriptor, byte i holding bits 8i+7..8i.
enum Field {
  F_MAGIC, F_VERSION, F_CORE_ID, F_HDR_RSV, F_OPCODE, F_CTRL, F_GROUP_SIZE, F_EPI, F_BASE_ADDR,
  F_A_OFF, F_W_OFF, F_Y_OFF, F_SCALE_OFF, F_BIAS_OFF, F_M, F_N, F_K, F_LDA16, F_OUT_SCALE,
  F_CRC32, F_VALID, F_LDY16, F_DEP_SIG, kFields
};
struct BitRange {
  int lo, width;
};
constexpr BitRange kBits[kFields] = {
    {496, 16}, {480, 16}, {472, 8},  {448, 24}, {432, 16}, {416, 16}, {400, 16}, {384, 16},
    {320, 64}, {288, 32}, {256, 32}, {224, 32}, {192, 32}, {160, 32}, {144, 16}, {128, 16},
    {112, 16}, {96, 16},  {64, 32},  {32, 32},  {31, 1},   {16, 15},  {0, 16}};

constexpr uint32_t kMagic = 0xAA55, kVersion = 0x0002;
constexpr uint64_t kDescBytes = 64;
enum Op { OP_CONV = 1, OP_GEMM = 2, OP_RELU = 3, OP_ROW = 4, OP_CONV_ACT = 5, OP_ELT = 6, OP_ROPE = 7, OP_FDOT = 8 };
enum Qm { QM_NONE = 0, QM_TENSOR = 1, QM_CHANNEL = 2, QM_ROWCOL = 3 };  // QM_ROWCOL doubles as the W4 group mode
enum Dt { DT_BF16 = 0, DT_INT8 = 1, DT_INT4 = 2, DT_FP8 = 3, DT_FP32 = 4 };
enum Out { OUT_FP32 = 0, OUT_BF16 = 1, OUT_INT8 = 2, OUT_FP16 = 3 };
enum RowFn { ROW_SOFTMAX = 0, ROW_LAYERNORM = 1, ROW_RMSNORM = 2, ROW_L2NORM = 3, ROW_QUANT = 4 };
enum EltOp { ELT_MUL = 0, ELT_ADD = 1, ELT_MULADD = 2, ELT_SUB = 3 };
enum Bcast { BM_DENSE = 0, BM_ROW = 1, BM_COL = 2, BM_SCALAR = 3 };
constexpr uint64_t kStateFp16 = 1u << 3;
constexpr uint64_t kW4Group = 128;
enum Err { E_OK = 0, E_MAGIC, E_VERSION, E_CRC, E_VALID, E_OPCODE, E_FIELD, E_ALIGN, E_RANGE };

struct Desc {
  uint64_t f[kFields];
  uint64_t operator[](Field i) const { return f[i]; }
};

uint64_t field_bits(const uint8_t* raw, BitRange r) {
  u128 acc = 0;
  const int b0 = r.lo / 8, b1 = (r.lo + r.width - 1) / 8;
  for (int b = b1; b >= b0; --b) acc = (acc << 8) | raw[b];
  acc >>= (r.lo % 8);
  const u128 mask = (r.width >= 64) ? ~static_cast<u128>(0) >> 64 : ((static_cast<u128>(1) << r.width) - 1);
  return static_cast<uint64_t>(acc & mask);
}

Desc decode(const uint8_t* raw) {
  Desc d;
  for (int i = 0; i < kFields; ++i) d.f[i] = field_bits(raw, kBits[i]);
  return d;
}

// CRC-32/ISO-HDLC (reflected polynomial 0xEDB88320, initial and final xor 0xFFFFFFFF), the zlib
// crc32, over the 64 bytes with the CRC field (bytes 4..7) read as zero.
uint32_t crc32_desc(const uint8_t* raw) {
  static uint32_t table[256];
  static bool ready = false;
  if (!ready) {
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int k = 0; k < 8; ++k) c = (c & 1) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
      table[i] = c;
    }
    ready = true;
  }
  uint32_t c = 0xFFFFFFFFu;
  for (uint64_t i = 0; i < kDescBytes; ++i) {
    const uint8_t byte = (i >= 4 && i < 8) ? 0 : raw[i];
    c = table[(c ^ byte) & 0xFF] ^ (c >> 8);
  }
  return c ^ 0xFFFFFFFFu;
}

// ---------------------------------------------------------------------------- derived values
uint32_t act_code(uint64_t epi) { return static_cast<uint32_t>((epi & 3) | ((epi >> 5) & 1) << 2); }
uint32_t out_code(uint64_t epi) { return static_cast<uint32_t>((epi >> 2) & 3); }
bool has_bias(uint64_t epi) { return (epi >> 4) & 1; }
uint64_t out_esize(uint32_t out) { return out == OUT_FP32 ? 4 : out == OUT_INT8 ? 1 : 2; }
bool is_conv(uint64_t op) { return op == OP_CONV || op == OP_CONV_ACT; }
bool is_v04(uint64_t op) { return op == OP_ELT || op == OP_ROPE || op == OP_FDOT; }
bool is_w4(const Desc& d) {
  return d[F_OPCODE] == OP_GEMM && (d[F_CTRL] & 7) == QM_ROWCOL && ((d[F_CTRL] >> 8) & 15) == DT_INT4;
}

int64_t floor_div(int64_t a, int64_t b) {
  int64_t q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
  return q;
}

// Implicit-GEMM geometry of a conv descriptor: HDR_RSV = H[23:12] | KH[11:8] | KW[7:4] |
// (STRIDE-1)[3:2] | PAD[1:0], GROUP_SIZE = W (contract.py:58-72).
struct ConvGeom {
  int64_t H, W, KH, KW, S, P, Cin, OH, OW;
};
ConvGeom conv_geom(const Desc& d) {
  const uint64_t g = d[F_HDR_RSV];
  ConvGeom c;
  c.H = static_cast<int64_t>(g >> 12);
  c.KH = static_cast<int64_t>((g >> 8) & 15);
  c.KW = static_cast<int64_t>((g >> 4) & 15);
  c.S = static_cast<int64_t>((g >> 2) & 3) + 1;
  c.P = static_cast<int64_t>(g & 3);
  c.W = static_cast<int64_t>(d[F_GROUP_SIZE]);
  c.Cin = (c.KH && c.KW) ? static_cast<int64_t>(d[F_K]) / (c.KH * c.KW) : 0;
  c.OH = floor_div(c.H + 2 * c.P - c.KH, c.S) + 1;
  c.OW = floor_div(c.W + 2 * c.P - c.KW, c.S) + 1;
  return c;
}

struct Strides {
  uint64_t lda, ldy, arow, yrow;
};
Strides strides(const Desc& d) {
  const uint64_t op = d[F_OPCODE], N = d[F_N], K = d[F_K];
  uint64_t arow;
  if (is_w4(d)) {
    arow = (((d[F_CTRL] >> 4) & 15) == DT_FP32 ? 4 : 2) * K;
  } else if (op == OP_GEMM) {
    arow = K;
  } else if (is_conv(op)) {
    arow = static_cast<uint64_t>(conv_geom(d).Cin);
  } else if (op == OP_FDOT) {
    arow = 4 * K;
  } else {
    arow = ((op == OP_ELT && (d[F_HDR_RSV] & kStateFp16)) ? 2 : 4) * N;
  }
  const uint64_t yrow = N * out_esize(out_code(d[F_EPI]));
  return {d[F_LDA16] ? 16 * d[F_LDA16] : arow, d[F_LDY16] ? 16 * d[F_LDY16] : yrow, arow, yrow};
}

// (row stride, row bytes) of the second operand of ELT (dense B) and FDOT.
std::pair<uint64_t, uint64_t> b_stride(const Desc& d) {
  uint64_t brow;
  if (d[F_OPCODE] == OP_FDOT) {
    brow = ((d[F_HDR_RSV] & kStateFp16) ? 2 : 4) * ((d[F_CTRL] & 1) ? d[F_N] : d[F_K]);
  } else {
    brow = (d[F_HDR_RSV] & 3) == BM_DENSE ? 4 * d[F_N] : 0;
  }
  return {d[F_GROUP_SIZE] ? 16 * d[F_GROUP_SIZE] : brow, brow};
}

// ---------------------------------------------------------------------------- validation
// The contract's checks in its order; the first failing class wins (golden.py:59-169).
int field_rules(const Desc& d, int core_id) {
  const uint64_t op = d[F_OPCODE], c = d[F_CTRL], e = d[F_EPI];
  const uint64_t qmode = c & 7, sym = (c >> 3) & 1, adt = (c >> 4) & 15, wdt = (c >> 8) & 15, fus = (c >> 12) & 1;
  const uint32_t act = act_code(e), out = out_code(e);
  const bool bias = has_bias(e), conv = is_conv(op), w4 = is_w4(d);
  const uint64_t hdr = d[F_HDR_RSV];
  const bool hdr_ok = conv || (op == OP_GEMM && qmode == QM_ROWCOL && !w4) || (op == OP_ELT && hdr < 16) ||
                      (op == OP_FDOT && (c & 1) && hdr == kStateFp16);
  const bool grp_ok = conv || is_v04(op) || w4;
  if (d[F_CORE_ID] != static_cast<uint64_t>(core_id) || d[F_DEP_SIG] || (hdr && !hdr_ok) ||
      (d[F_GROUP_SIZE] && !grp_ok))
    return E_FIELD;
  if ((c >> 13) || (e >> 6) || (out == OUT_FP16 && op != OP_ELT)) return E_FIELD;
  if (out != OUT_INT8 && d[F_OUT_SCALE]) return E_FIELD;
  if (op == OP_GEMM || conv) {
    if (w4) {
      if (sym != 1 || (adt != DT_FP32 && adt != DT_BF16) || hdr != 0 || d[F_GROUP_SIZE] != kW4Group) return E_FIELD;
    } else if ((qmode != QM_TENSOR && qmode != QM_CHANNEL && qmode != QM_ROWCOL) || sym != 1 || adt != DT_INT8 ||
               wdt != DT_INT8 || (conv && qmode == QM_ROWCOL)) {
      return E_FIELD;
    }
    if ((act != 0) != (fus == 1)) return E_FIELD;
    if (op == OP_CONV_ACT && act == 0) return E_FIELD;
    if (conv) {
      const ConvGeom g = conv_geom(d);
      if (!(g.H && g.W && g.KH && g.KW) || g.OH < 1 || g.OW < 1 || static_cast<int64_t>(d[F_M]) != g.OH * g.OW)
        return E_FIELD;
    }
  } else if (op == OP_RELU) {
    if (c != 0 || bias || d[F_K] || d[F_W_OFF] || d[F_SCALE_OFF] || d[F_BIAS_OFF] || act == 0) return E_FIELD;
  } else if (op == OP_ROW) {
    const uint64_t fn = c & 7;
    if ((c >> 3) || fn > ROW_QUANT || act != 0 || (d[F_K] && fn != ROW_SOFTMAX)) return E_FIELD;
    if (fn == ROW_SOFTMAX && (bias || d[F_W_OFF] || d[F_SCALE_OFF] || d[F_BIAS_OFF])) return E_FIELD;
    if (fn == ROW_QUANT && (bias || d[F_W_OFF] || d[F_BIAS_OFF] || out != OUT_INT8 || d[F_OUT_SCALE]))
      return E_FIELD;
    if (!bias && d[F_BIAS_OFF]) return E_FIELD;
  } else if (op == OP_ELT) {
    const uint64_t eop = c & 3;
    if ((c >> 2) || d[F_K] || d[F_SCALE_OFF] || bias != (eop == ELT_MULADD) ||
        (eop == ELT_MULADD && out != OUT_FP32 && out != OUT_FP16) || (!bias && d[F_BIAS_OFF]))
      return E_FIELD;
  } else if (op == OP_ROPE) {
    if (c || act != 0 || bias || d[F_SCALE_OFF] || d[F_BIAS_OFF] || d[F_GROUP_SIZE] == 0) return E_FIELD;
  } else {  // OP_FDOT
    if ((c >> 1) || act != 0 || bias || d[F_SCALE_OFF] || d[F_BIAS_OFF]) return E_FIELD;
  }
  return E_OK;
}

int align_rules(const Desc& d) {
  const uint64_t op = d[F_OPCODE], M = d[F_M], N = d[F_N], K = d[F_K];
  const bool conv = is_conv(op), gemm = op == OP_GEMM || conv;
  if (M == 0 || N == 0 || N % 16 || ((gemm || op == OP_FDOT) && (K == 0 || K % 16))) return E_ALIGN;
  if (is_w4(d) && (K < 2 * kW4Group || K % (2 * kW4Group) || K > 64 * kW4Group || d[F_W_OFF] % 128)) return E_ALIGN;
  if (op == OP_ROPE && (K == 0 || K % 32 || K > N)) return E_ALIGN;
  if (conv) {
    const ConvGeom g = conv_geom(d);
    if (K % static_cast<uint64_t>(g.KH * g.KW) || g.Cin % 16) return E_ALIGN;
  }
  const Field offs[5] = {F_A_OFF, F_Y_OFF, F_SCALE_OFF, F_BIAS_OFF, F_W_OFF};
  const int noffs = op == OP_ROW ? 4 : 5;
  for (int i = 0; i < noffs; ++i) {
    const uint64_t bm = d[F_HDR_RSV] & 3;
    const uint64_t al = (offs[i] == F_W_OFF && op == OP_ELT && (bm == BM_COL || bm == BM_SCALAR)) ? 4 : 16;
    if (d[offs[i]] % al) return E_ALIGN;
  }
  const Strides s = strides(d);
  if (s.lda < s.arow || s.ldy < s.yrow) return E_ALIGN;
  if (op == OP_ELT || op == OP_FDOT) {
    const auto b = b_stride(d);
    if (b.first < b.second) return E_ALIGN;
  }
  return E_OK;
}

int validate(const uint8_t* raw, const Desc& d, int core_id, bool gemv_only) {
  if (d[F_MAGIC] != kMagic) return E_MAGIC;
  if (d[F_VERSION] != kVersion) return E_VERSION;
  if (crc32_desc(raw) != d[F_CRC32]) return E_CRC;
  if (d[F_VALID] != 1) return E_VALID;
  const uint64_t op = d[F_OPCODE];
  if (op < OP_CONV || op > OP_FDOT) return E_OPCODE;
  if (gemv_only && (is_conv(op) || (op == OP_GEMM && d[F_K] > 4096))) return E_OPCODE;
  if (int e = field_rules(d, core_id)) return e;
  return align_rules(d);
}

// ---------------------------------------------------------------------------- byte segments
// A tensor's bytes in closed form: `rows` rows of `rb` bytes, `ld` apart, i.e. the segments
// [base + r ld, base + r ld + rb) for r < rows. A K or V cache of thousands of rows is one entry,
// and whether two tensors share a byte is answered without listing their rows.
struct Span {
  u128 base, ld, rb;
  uint64_t rows;
  bool empty() const { return rows == 0 || rb == 0; }
  u128 lo() const { return base; }
  u128 hi() const { return empty() ? base : base + ld * (rows - 1) + rb; }
};
using Segs = std::vector<Span>;

Span interval(u128 lo, u128 hi) { return hi > lo ? Span{lo, hi - lo, hi - lo, 1} : Span{lo, 1, 0, 0}; }

// Rows that touch or overlap (ld <= row bytes) are one interval, their union.
Span strided_span(u128 base, uint64_t ld, uint64_t nrows, uint64_t row_bytes) {
  if (nrows == 0 || row_bytes == 0) return Span{base, 1, 0, 0};
  if (nrows == 1 || ld <= row_bytes) return interval(base, base + static_cast<u128>(ld) * (nrows - 1) + row_bytes);
  return Span{base, ld, row_bytes, nrows};
}

Segs strided(u128 base, uint64_t ld, uint64_t nrows, uint64_t row_bytes) {
  return {strided_span(base, ld, nrows, row_bytes)};
}

// Whether [lo, hi) meets a row of s: the rows from the first that ends past lo to the last that
// starts before hi.
bool meets(const Span& s, u128 lo, u128 hi) {
  if (s.empty() || lo >= hi || hi <= s.lo() || lo >= s.hi()) return false;
  if (s.rows == 1) return true;
  const u128 r0 = lo < s.base + s.rb ? 0 : (lo - s.base - s.rb) / s.ld + 1;
  const u128 r1 = std::min<u128>(s.rows - 1, (hi - 1 - s.base) / s.ld);
  return r0 <= r1;
}

// Whether any row of a meets any row of b: the rows of the span with fewer rows, from the first
// that ends past the other's start, each tested in closed form.
bool meets(const Span& a, const Span& b) {
  if (a.empty() || b.empty() || a.hi() <= b.lo() || b.hi() <= a.lo()) return false;
  const Span& x = a.rows <= b.rows ? a : b;
  const Span& y = a.rows <= b.rows ? b : a;
  const u128 r0 = x.base + x.rb > y.lo() ? 0 : (y.lo() - x.base - x.rb) / x.ld + 1;
  for (u128 r = r0; r < x.rows; ++r) {
    const u128 lo = x.base + x.ld * r;
    if (lo >= y.hi()) break;
    if (meets(y, lo, lo + x.rb)) return true;
  }
  return false;
}

// The tensors a valid descriptor reads (each a list of segments) and the rows it writes
// (ascending and disjoint since ldy >= row bytes), as in golden.py:183-248.
void segments(const Desc& d, std::vector<Segs>& reads, Segs& y) {
  const u128 B = d[F_BASE_ADDR];
  const uint64_t M = d[F_M], N = d[F_N], K = d[F_K], op = d[F_OPCODE];
  const Strides s = strides(d);
  reads.clear();
  y = strided(B + d[F_Y_OFF], s.ldy, M, s.yrow);
  if (is_v04(op)) {
    if (op == OP_ELT && ((d[F_HDR_RSV] >> 2) & 1)) {
      reads.push_back({interval(B + d[F_A_OFF], B + d[F_A_OFF] + s.arow)});
    } else {
      reads.push_back(strided(B + d[F_A_OFF], s.lda, M, s.arow));
    }
    const u128 w0 = B + d[F_W_OFF];
    if (op == OP_ELT) {
      const uint64_t bm = d[F_HDR_RSV] & 3;
      if (bm == BM_DENSE) {
        reads.push_back(strided(w0, b_stride(d).first, M, 4 * N));
      } else {
        const uint64_t nb = bm == BM_ROW ? 4 * N : bm == BM_COL ? 4 * M : 4;
        reads.push_back({interval(w0, w0 + nb)});
      }
      if ((d[F_CTRL] & 3) == ELT_MULADD) reads.push_back(strided(B + d[F_BIAS_OFF], s.ldy, M, s.yrow));
    } else if (op == OP_ROPE) {
      const uint64_t tab_rows = (M - 1) / d[F_GROUP_SIZE] + 1;
      reads.push_back({interval(w0, w0 + static_cast<u128>(4 * K) * tab_rows)});
    } else {
      const auto b = b_stride(d);
      reads.push_back(strided(w0, b.first, (d[F_CTRL] & 1) ? K : N, b.second));
    }
    return;
  }
  if (is_conv(op)) {
    const ConvGeom g = conv_geom(d);
    const uint64_t npx = static_cast<uint64_t>(g.H * g.W);
    const u128 a0 = B + d[F_A_OFF];
    if (s.lda == s.arow) {
      reads.push_back({interval(a0, a0 + static_cast<u128>(npx) * s.arow)});
    } else {
      reads.push_back(strided(a0, s.lda, npx, s.arow));
    }
  } else {
    reads.push_back(strided(B + d[F_A_OFF], s.lda, M, s.arow));
  }
  if (op == OP_GEMM || is_conv(op)) {
    const bool w4 = is_w4(d);
    const uint64_t ns = (d[F_CTRL] & 7) == QM_TENSOR ? 1 : N;
    reads.push_back({interval(B + d[F_W_OFF], B + d[F_W_OFF] + static_cast<u128>(N) * K / (w4 ? 2 : 1))});
    reads.push_back({interval(B + d[F_SCALE_OFF],
                              B + d[F_SCALE_OFF] + (w4 ? static_cast<u128>(2 * N) * (K / kW4Group) : static_cast<u128>(4 * ns)))});
    if (has_bias(d[F_EPI])) reads.push_back({interval(B + d[F_BIAS_OFF], B + d[F_BIAS_OFF] + 4 * N)});
    if ((d[F_CTRL] & 7) == QM_ROWCOL && !w4) {
      const u128 r0 = B + static_cast<u128>(16) * d[F_HDR_RSV];
      reads.push_back({interval(r0, r0 + 4 * M)});
    }
  } else if (op == OP_ROW) {
    const uint64_t fn = d[F_CTRL] & 7;
    if (fn == ROW_LAYERNORM || fn == ROW_RMSNORM || fn == ROW_L2NORM) {
      reads.push_back({interval(B + d[F_SCALE_OFF], B + d[F_SCALE_OFF] + 4 * N)});
      if (has_bias(d[F_EPI])) reads.push_back({interval(B + d[F_BIAS_OFF], B + d[F_BIAS_OFF] + 4 * N)});
    }
  }
}

// ROW_QUANT's second output, the row scales (golden.py:250-256).
Segs extra_out(const Desc& d) {
  if (d[F_OPCODE] == OP_ROW && (d[F_CTRL] & 7) == ROW_QUANT) {
    const u128 a = static_cast<u128>(d[F_BASE_ADDR]) + d[F_SCALE_OFF];
    return {interval(a, a + 4 * d[F_M])};
  }
  return {};
}

// Whether any row of any tensor in a meets any row of any tensor in b.
bool overlaps(const Segs& a, const Segs& b) {
  for (const Span& x : a)
    for (const Span& y : b)
      if (meets(x, y)) return true;
  return false;
}

// ELT may read its own output rows in place: A (read 0) or C (read 2), fp32/fp16 (golden.py:440-448).
bool in_place(const Desc& d, size_t i) {
  const uint32_t out = out_code(d[F_EPI]);
  if (d[F_OPCODE] != OP_ELT || (out != OUT_FP32 && out != OUT_FP16)) return false;
  const Strides s = strides(d);
  if (i == 0) {
    const uint32_t afmt = (d[F_HDR_RSV] & kStateFp16) ? OUT_FP16 : OUT_FP32;
    return afmt == out && !((d[F_HDR_RSV] >> 2) & 1) && d[F_A_OFF] == d[F_Y_OFF] && s.lda == s.ldy;
  }
  return i == 2 && d[F_BIAS_OFF] == d[F_Y_OFF];
}

u128 max_hi(const Segs& v) {
  u128 m = 0;
  for (const Span& s : v) m = std::max(m, s.hi());
  return m;
}

// The full check of one descriptor: contract code (E_RANGE against an image of `len` bytes
// included) or TARS_E_OVERLAP for an output that overlaps an input.
struct Checked {
  int err;       // contract ERR_CODE
  bool overlap;  // valid, but an output overlaps an input (the golden's ContractError)
  Desc d;
  std::vector<Segs> reads;
  Segs y, extra;
};

Checked check(const uint8_t* raw, uint64_t len, int core_id, bool gemv_only) {
  Checked c{};
  c.d = decode(raw);
  c.err = validate(raw, c.d, core_id, gemv_only);
  if (c.err != E_OK) return c;
  segments(c.d, c.reads, c.y);
  c.extra = extra_out(c.d);
  u128 hi = std::max(max_hi(c.y), max_hi(c.extra));
  for (const Segs& s : c.reads) hi = std::max(hi, max_hi(s));
  if (hi > static_cast<u128>(len)) {
    c.err = E_RANGE;
    return c;
  }
  for (size_t j = 0; j < c.reads.size(); ++j) {
    if (overlaps(c.reads[j], c.y) && !in_place(c.d, j)) c.overlap = true;
    if (!c.extra.empty() && overlaps(c.reads[j], c.extra)) c.overlap = true;
  }
  if (!c.extra.empty() && overlaps(c.extra, c.y)) c.overlap = true;
  return c;
}

// Whether this library runs the descriptor on the GPU: W8A8 GEMM (QM_TENSOR / QM_CHANNEL /
// QM_ROWCOL), the W4A16 group GEMM, ROW_QUANT.
// Every valid descriptor but a convolution runs on the GPU.
bool gpu_kind(const Desc& d) { return d[F_OPCODE] != OP_CONV && d[F_OPCODE] != OP_CONV_ACT; }

// Enqueues a valid, GPU-kind descriptor with pointers into the image; returns a TARS_ status.
// `needs_host` is set instead when the image addresses miss the kernels' alignment (a base
// address that is not a multiple of 16, or W4 weights off a 128-byte boundary).
int launch(uint8_t* image, const Desc& d, hipStream_t stream, bool& needs_host) {
  uint8_t* B = image + d[F_BASE_ADDR];
  const Strides s = strides(d);
  const int M = static_cast<int>(d[F_M]), N = static_cast<int>(d[F_N]), K = static_cast<int>(d[F_K]);
  const uint32_t act = act_code(d[F_EPI]), out = out_code(d[F_EPI]);
  const uintptr_t b = reinterpret_cast<uintptr_t>(B);
  needs_host = b % 16 != 0 || (is_w4(d) && (b + d[F_W_OFF]) % 128 != 0);
  if (needs_host) return TARS_OK;
  const float* bias = has_bias(d[F_EPI]) ? reinterpret_cast<const float*>(B + d[F_BIAS_OFF]) : nullptr;
  const uint32_t osc = static_cast<uint32_t>(d[F_OUT_SCALE]);
  const uint64_t op = d[F_OPCODE];
  const auto f32p = [&](Field off) { return reinterpret_cast<const float*>(B + d[off]); };
  const int64_t lda = static_cast<int64_t>(s.lda), ldy = static_cast<int64_t>(s.ldy);
  if (op == OP_ROW) {  // golden.py:358-380
    const uint64_t fn = d[F_CTRL] & 7;
    if (fn == ROW_QUANT)
      return tars_quant_rows(f32p(F_A_OFF), lda, reinterpret_cast<int8_t*>(B + d[F_Y_OFF]), ldy,
                             reinterpret_cast<float*>(B + d[F_SCALE_OFF]), M, N, stream);
    if (fn == ROW_SOFTMAX)
      return tars_row_op(f32p(F_A_OFF), lda, TARS_ROW_SOFTMAX, nullptr, nullptr, 0, K, nullptr, B + d[F_Y_OFF], ldy,
                         static_cast<int>(out), osc, M, N, stream);
    return tars_row_op(f32p(F_A_OFF), lda, static_cast<int32_t>(fn), f32p(F_SCALE_OFF), bias,
                       static_cast<uint32_t>(d[F_W_OFF]), 0, nullptr, B + d[F_Y_OFF], ldy, static_cast<int>(out), osc, M,
                       N, stream);
  }
  if (op == OP_RELU)  // golden.py:351-356
    return tars_relu(f32p(F_A_OFF), lda, static_cast<int>(act), B + d[F_Y_OFF], ldy, static_cast<int>(out), osc, M, N,
                     stream);
  if (op == OP_ELT) {  // golden.py:393-418
    const uint64_t hr = d[F_HDR_RSV], eop = d[F_CTRL] & 3, bm = hr & 3;
    return tars_elt(B + d[F_A_OFF], lda, (hr & kStateFp16) ? 1 : 0, static_cast<int32_t>((hr >> 2) & 1), f32p(F_W_OFF),
                    bm == BM_DENSE ? static_cast<int64_t>(b_stride(d).first) : 0, static_cast<int32_t>(bm),
                    eop == ELT_MULADD ? B + d[F_BIAS_OFF] : nullptr, eop == ELT_MULADD ? ldy : 0,
                    static_cast<int32_t>(eop), static_cast<int>(act), B + d[F_Y_OFF], ldy, static_cast<int>(out), osc, M,
                    N, stream);
  }
  if (op == OP_ROPE)  // golden.py:420-424
    return tars_rope(f32p(F_A_OFF), lda, f32p(F_W_OFF), static_cast<int32_t>(d[F_GROUP_SIZE]), K, B + d[F_Y_OFF], ldy,
                     static_cast<int>(out), osc, M, N, stream);
  if (op == OP_FDOT)  // golden.py:426-436
    return tars_fdot(f32p(F_A_OFF), lda, B + d[F_W_OFF], static_cast<int64_t>(b_stride(d).first),
                     static_cast<int32_t>(d[F_CTRL] & 1), (d[F_HDR_RSV] & kStateFp16) ? 1 : 0, B + d[F_Y_OFF], ldy,
                     static_cast<int>(out), osc, M, N, K, stream);
  if (is_w4(d)) {
    const int adt = ((d[F_CTRL] >> 4) & 15) == DT_FP32 ? TARS_DT_FP32 : TARS_DT_BF16;
    return tars_gemm_w4a16(B + d[F_A_OFF], static_cast<int64_t>(s.lda), adt, B + d[F_W_OFF],
                           reinterpret_cast<const uint16_t*>(B + d[F_SCALE_OFF]), bias, B + d[F_Y_OFF],
                           static_cast<int64_t>(s.ldy), M, N, K, static_cast<int>(act), static_cast<int>(out), osc, stream);
  }
  const uint64_t qmode = d[F_CTRL] & 7;
  const float* srow = qmode == QM_ROWCOL ? reinterpret_cast<const float*>(B + 16 * d[F_HDR_RSV]) : nullptr;
  return tars_gemm_w8a8(reinterpret_cast<const int8_t*>(B + d[F_A_OFF]), static_cast<int64_t>(s.lda), srow,
                        reinterpret_cast<const int8_t*>(B + d[F_W_OFF]), reinterpret_cast<const float*>(B + d[F_SCALE_OFF]),
                        qmode == QM_TENSOR ? 1 : N, bias, B + d[F_Y_OFF], static_cast<int64_t>(s.ldy), M, N, K,
                        static_cast<int>(act), static_cast<int>(out), osc, stream);
}

}  // namespace

namespace tars {
void set_last_error(const std::string& what);
int w8a8_path();
int quant_gemm_w8a8_checked(const float* x, int64_t lda, int8_t* q, int64_t ldq, float* s, int32_t M, int32_t K,
                            const tars_w8a8_out* outs, int32_t nouts, float* prod, int64_t ldprod, void* stream,
                            const NormPrologue* pro);
}  // namespace tars

namespace {

bool g_fusion = true;

float f32_bits(uint64_t v) {
  const uint32_t b = static_cast<uint32_t>(v);
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}

u128 addr(const Desc& d, Field off) { return static_cast<u128>(d[F_BASE_ADDR]) + d[off]; }

// Peephole fusion for decode rows: a ROW_QUANT with M = 1 followed by up to 4 QM_ROWCOL W8A8
// GEMMs (each valid on its own) whose A row is exactly the quantizer's int8 output and whose row
// scale is its scale runs as one tars_quant_gemm_w8a8 launch, which also writes the quantizer's
// outputs: bit-identical to running them one by one (the GEMMs read the same int8 values and
// scale the kernel computes). No fusion when an output of the group lands on a later descriptor
// of the queue; when the group's outputs overlap each other or any input of the group, the fused
// call refuses before launching and the descriptors run one by one. `fused` = GEMMs folded in.
// One ROW_QUANT (M = 1) and the GEMMs reading its output, as one tars_quant_gemm_w8a8 call.
// With `elt` (a gated group): the two GEMMs' ELT MUL runs in the same launch (the product of the
// fp32 outputs stored at the ELT's output, see fuse_group). With `norm` (and `add`): the norm whose
// output the quantizer reads (and the residual ELT ADD whose output the norm reads) run in the
// same launch as its prologue (see fuse_norm_group).
int launch_fused(uint8_t* image, const Desc& dq, const std::vector<Desc>& members, hipStream_t s,
                 const Desc* elt = nullptr, const Desc* add = nullptr, const Desc* norm = nullptr) {
  tars_w8a8_out outs[4];
  for (size_t k = 0; k < members.size(); ++k) {
    const Desc& d = members[k];
    uint8_t* B = image + d[F_BASE_ADDR];
    outs[k].W = reinterpret_cast<const int8_t*>(B + d[F_W_OFF]);
    outs[k].scol = reinterpret_cast<const float*>(B + d[F_SCALE_OFF]);
    outs[k].bias = has_bias(d[F_EPI]) ? reinterpret_cast<const float*>(B + d[F_BIAS_OFF]) : nullptr;
    outs[k].Y = B + d[F_Y_OFF];
    outs[k].ldy = static_cast<int64_t>(strides(d).ldy);
    outs[k].N = static_cast<int32_t>(d[F_N]);
    outs[k].act = static_cast<int32_t>(act_code(d[F_EPI]));
    outs[k].out = static_cast<int32_t>(out_code(d[F_EPI]));
    outs[k].out_scale_bits = static_cast<uint32_t>(d[F_OUT_SCALE]);
  }
  uint8_t* B = image + dq[F_BASE_ADDR];
  const Strides sq = strides(dq);
  float* prod = elt ? reinterpret_cast<float*>(image + (*elt)[F_BASE_ADDR] + (*elt)[F_Y_OFF]) : nullptr;
  const float* x = reinterpret_cast<const float*>(B + dq[F_A_OFF]);
  int64_t lda = static_cast<int64_t>(sq.lda);
  tars::NormPrologue pro{};
  if (norm) {  // one row: the strides never apply
    const Desc& r = *norm;
    uint8_t* RB = image + r[F_BASE_ADDR];
    pro.fn = static_cast<int>(r[F_CTRL] & 7);
    pro.gamma = reinterpret_cast<const float*>(RB + r[F_SCALE_OFF]);
    pro.beta = has_bias(r[F_EPI]) ? reinterpret_cast<const float*>(RB + r[F_BIAS_OFF]) : nullptr;
    pro.eps = f32_bits(r[F_W_OFF]);
    pro.y = reinterpret_cast<float*>(RB + r[F_Y_OFF]);
    x = reinterpret_cast<const float*>(RB + r[F_A_OFF]);
    lda = 0;
    if (add) {
      const Desc& e = *add;
      uint8_t* EB = image + e[F_BASE_ADDR];
      x = reinterpret_cast<const float*>(EB + e[F_A_OFF]);
      pro.B = reinterpret_cast<const float*>(EB + e[F_W_OFF]);
      pro.sum = reinterpret_cast<float*>(EB + e[F_Y_OFF]);
    }
  }
  return tars::quant_gemm_w8a8_checked(x, lda, reinterpret_cast<int8_t*>(B + dq[F_Y_OFF]), static_cast<int64_t>(sq.ldy),
                                       reinterpret_cast<float*>(B + dq[F_SCALE_OFF]), 1, static_cast<int32_t>(dq[F_N]),
                                       outs, static_cast<int32_t>(members.size()), prod,
                                       elt ? static_cast<int64_t>(strides(*elt).ldy) : 0, s, norm ? &pro : nullptr);
}

// An MLP's gated product after a two-GEMM group (tars_mini/llm.py:620-624: the gate GEMM with its
// activation, the up GEMM, then ELT MUL of their outputs): a dense fp32 ELT MUL with no activation
// over one row whose A operand is exactly the first GEMM's output and whose B operand is exactly
// the second's, both GEMMs storing fp32. The fused launch stores the second output, the product at
// the ELT's output and, unless that is the first output itself (in place), the first output:
// the same bytes as the three descriptors one by one (the ELT multiplies the stored fp32 values,
// which are the kernel's flushed epilogue values).
bool gated_elt(const Checked& e, const Desc& g0, const Desc& g1, uintptr_t image) {
  const Desc& d = e.d;
  return e.err == E_OK && !e.overlap && d[F_OPCODE] == OP_ELT && (d[F_CTRL] & 3) == ELT_MUL &&
         act_code(d[F_EPI]) == 0 && out_code(d[F_EPI]) == OUT_FP32 && (d[F_HDR_RSV] & (3 | 4 | kStateFp16)) == BM_DENSE &&
         d[F_M] == 1 && d[F_N] == g0[F_N] && d[F_N] == g1[F_N] && out_code(g0[F_EPI]) == OUT_FP32 &&
         out_code(g1[F_EPI]) == OUT_FP32 && addr(d, F_A_OFF) == addr(g0, F_Y_OFF) && addr(d, F_W_OFF) == addr(g1, F_Y_OFF) &&
         (image + d[F_BASE_ADDR] + d[F_Y_OFF]) % 16 == 0 && tars::quant_gemv_pairs_supported(static_cast<int>(g0[F_K]));
}

// With `norm` (and `add`), the prologue fuse_norm_group checked runs in the same launch.
int fuse_group(uint8_t* image, const Checked& quant, const std::vector<uint8_t>& q, int32_t i, uint64_t in_image,
               int32_t n, u128 rest_lo, u128 rest_hi, uint64_t image_len, int core_id, bool gemv_only, hipStream_t s,
               int& fused, std::vector<Desc>& group, Desc& elt, bool& gated, const Desc* add = nullptr,
               const Desc* norm = nullptr) {
  fused = 0;
  group.clear();
  gated = false;
  const Desc& dq = quant.d;
  if (!g_fusion || quant.err != E_OK || quant.overlap || dq[F_OPCODE] != OP_ROW || (dq[F_CTRL] & 7) != ROW_QUANT ||
      dq[F_M] != 1 || (reinterpret_cast<uintptr_t>(image) + dq[F_BASE_ADDR]) % 16)
    return TARS_OK;
  std::vector<Checked> members;
  for (int32_t j = i + 1; j < n && static_cast<uint64_t>(j) < in_image && members.size() < 4; ++j) {
    Checked c = check(q.data() + static_cast<size_t>(j) * kDescBytes, image_len, core_id, gemv_only);
    const Desc& d = c.d;
    if (c.err != E_OK || c.overlap || d[F_OPCODE] != OP_GEMM || is_w4(d) || (d[F_CTRL] & 7) != QM_ROWCOL ||
        d[F_M] != 1 || d[F_K] != dq[F_N] || addr(d, F_A_OFF) != addr(dq, F_Y_OFF) ||
        static_cast<u128>(d[F_BASE_ADDR]) + 16 * static_cast<u128>(d[F_HDR_RSV]) != addr(dq, F_SCALE_OFF) ||
        (reinterpret_cast<uintptr_t>(image) + d[F_BASE_ADDR]) % 16)
      break;
    members.push_back(std::move(c));
  }
  if (members.empty()) return TARS_OK;
  const Segs rest = {interval(rest_lo, rest_hi)};
  if (rest_lo < rest_hi) {
    if (overlaps(rest, quant.y) || overlaps(rest, quant.extra)) return TARS_OK;
    for (const Checked& c : members)
      if (overlaps(rest, c.y)) return TARS_OK;
  }
  for (const Checked& c : members) group.push_back(c.d);
  const int32_t je = i + 3;  // the gated product's ELT MUL, right after a two-GEMM group
  if (members.size() == 2 && je < n && static_cast<uint64_t>(je) < in_image) {
    const Checked e = check(q.data() + static_cast<size_t>(je) * kDescBytes, image_len, core_id, gemv_only);
    if (gated_elt(e, members[0].d, members[1].d, reinterpret_cast<uintptr_t>(image)) &&
        !(rest_lo < rest_hi && overlaps(rest, e.y))) {
      const int rc = launch_fused(image, dq, group, s, &e.d, add, norm);
      if (rc == TARS_OK) {
        fused = 3;
        elt = e.d;
        gated = true;
        return rc;
      }
      if (rc != TARS_E_OVERLAP) return rc;
      tars::set_last_error("");  // the product overlaps an operand: the ELT runs on its own
    }
  }
  const int rc = launch_fused(image, dq, group, s, nullptr, add, norm);
  if (rc == TARS_E_OVERLAP) {
    tars::set_last_error("");
    group.clear();
    return TARS_OK;
  }
  if (rc == TARS_OK) fused = static_cast<int>(members.size());
  return rc;
}

// Attention fusion: a run of per-head triples FDOT_NT (scores) -> ROW_SOFTMAX -> FDOT_NN (P V), the
// reference's decode/prefill attention lowering (tars_mini/llm.py:736-746), runs as one launch of
// the fused attention kernel, all heads at once. Each triple must read its softmax input from the
// NT output and its NN input from the softmax output, every head the same shapes and the same
// score / probability buffers; no head may read (q, K, V) what any head writes, and the heads'
// outputs must not overlap each other or the rest of the queue. The heads then do not interact, so
// running them concurrently (the last head writing the shared buffers) leaves the image exactly as
// the triples run one after another.
struct AttnHead {
  Desc nt, sm, nn;
};

bool pairwise_disjoint(const Segs& v) {
  for (size_t i = 0; i < v.size(); ++i)
    for (size_t j = i + 1; j < v.size(); ++j)
      if (meets(v[i], v[j])) return false;
  return true;
}

tars::AttnArgs attention_args(uint8_t* image, const std::vector<AttnHead>& heads) {
  tars::AttnArgs a{};
  const Desc& nt0 = heads[0].nt;
  const Desc& sm0 = heads[0].sm;
  const Desc& nn0 = heads[0].nn;
  for (size_t h = 0; h < heads.size(); ++h) {
    const Desc& nt = heads[h].nt;
    const Desc& nn = heads[h].nn;
    a.q[h] = reinterpret_cast<const float*>(image + nt[F_BASE_ADDR] + nt[F_A_OFF]);
    a.k[h] = reinterpret_cast<const float*>(image + nt[F_BASE_ADDR] + nt[F_W_OFF]);
    a.v[h] = image + nn[F_BASE_ADDR] + nn[F_W_OFF];
    a.att[h] = image + nn[F_BASE_ADDR] + nn[F_Y_OFF];
  }
  a.ldq = static_cast<int64_t>(strides(nt0).lda);
  a.ldk = static_cast<int64_t>(b_stride(nt0).first);
  a.ldv = static_cast<int64_t>(b_stride(nn0).first);
  a.ldatt = static_cast<int64_t>(strides(nn0).ldy);
  a.sc = reinterpret_cast<float*>(image + nt0[F_BASE_ADDR] + nt0[F_Y_OFF]);
  a.ldsc = static_cast<int64_t>(strides(nt0).ldy);
  a.pr = reinterpret_cast<float*>(image + sm0[F_BASE_ADDR] + sm0[F_Y_OFF]);
  a.ldpr = static_cast<int64_t>(strides(sm0).ldy);
  a.heads = static_cast<int>(heads.size());
  a.M = static_cast<int>(nt0[F_M]);
  a.nk = static_cast<int>(nt0[F_N]);
  a.hd = static_cast<int>(nt0[F_K]);
  a.causal_k = static_cast<int>(sm0[F_K]);
  a.v_fp16 = (nn0[F_HDR_RSV] & kStateFp16) ? 1 : 0;
  a.out = static_cast<int>(out_code(nn0[F_EPI]));
  const uint32_t osc = static_cast<uint32_t>(nn0[F_OUT_SCALE]);
  std::memcpy(&a.out_scale, &osc, 4);
  return a;
}

// The q / k norm + RoPE prologue of an attention launch: the q norm, q RoPE, k norm and k RoPE
// descriptors, and the query heads per K / V head.
struct RopePrologue {
  Desc qn, qr, kn, kr;
  int qpk = 0, key = 0;  // query heads per K / V head; the key row the k RoPE writes
};

tars::AttnNormRope norm_rope_args(uint8_t* image, const Desc& rd, const Desc& pd) {
  uint8_t* RB = image + rd[F_BASE_ADDR];
  tars::AttnNormRope p{};
  p.x = reinterpret_cast<const float*>(RB + rd[F_A_OFF]);
  p.ldx = static_cast<int64_t>(strides(rd).lda);
  p.gamma = reinterpret_cast<const float*>(RB + rd[F_SCALE_OFF]);
  p.beta = has_bias(rd[F_EPI]) ? reinterpret_cast<const float*>(RB + rd[F_BIAS_OFF]) : nullptr;
  p.eps = f32_bits(rd[F_W_OFF]);
  p.fn = static_cast<int>(rd[F_CTRL] & 7);
  p.n = reinterpret_cast<float*>(RB + rd[F_Y_OFF]);
  p.ldn = static_cast<int64_t>(strides(rd).ldy);
  p.tab = reinterpret_cast<const float*>(image + pd[F_BASE_ADDR] + pd[F_W_OFF]);
  p.rows_per_pos = static_cast<int>(pd[F_GROUP_SIZE]);
  return p;
}

// scratch: the split form's scores between its two launches (null: one workgroup per head). An
// eager dispatch passes its stream's workspace, a launch plan the scratch it owns.
int launch_attention_group(uint8_t* image, const std::vector<AttnHead>& heads, hipStream_t s, float* scratch,
                           const RopePrologue* pro = nullptr) {
  tars::AttnArgs a = attention_args(image, heads);
  if (pro) {
    a.rope = pro->qpk;
    a.rope_key = pro->key;
    a.rq = norm_rope_args(image, pro->qn, pro->qr);
    a.rk = norm_rope_args(image, pro->kn, pro->kr);
  }
  a.scratch = scratch;
  a.scratch_floats = a.scratch ? tars::kAttnScratchFloats : 0;
  const hipError_t e = tars::launch_attention(a, s);
  if (e != hipSuccess) {
    tars::set_last_error(std::string("HIP launch failed: ") + hipGetErrorString(e));
    return TARS_E_DEVICE;
  }
  return TARS_OK;
}

// Whether descriptors (nt, sm, nn) form one head's triple the fused kernel runs.
bool attention_triple(const Checked& nt, const Checked& sm, const Checked& nn, uintptr_t image) {
  const Desc& a = nt.d;
  const Desc& b = sm.d;
  const Desc& c = nn.d;
  for (const Checked* x : {&nt, &sm, &nn})
    if (x->err != E_OK || x->overlap || (image + x->d[F_BASE_ADDR]) % 16) return false;
  if (a[F_OPCODE] != OP_FDOT || (a[F_CTRL] & 1) || out_code(a[F_EPI]) != OUT_FP32) return false;
  if (b[F_OPCODE] != OP_ROW || (b[F_CTRL] & 7) != ROW_SOFTMAX || out_code(b[F_EPI]) != OUT_FP32) return false;
  if (c[F_OPCODE] != OP_FDOT || !(c[F_CTRL] & 1)) return false;
  if (!tars::attention_supported(static_cast<int>(a[F_K]), static_cast<int>(a[F_N]))) return false;
  const uint64_t M = a[F_M], nk = a[F_N], hd = a[F_K];
  if (b[F_M] != M || b[F_N] != nk || c[F_M] != M || c[F_K] != nk || c[F_N] != hd) return false;
  if (addr(b, F_A_OFF) != addr(a, F_Y_OFF) || strides(b).lda != strides(a).ldy) return false;
  if (addr(c, F_A_OFF) != addr(b, F_Y_OFF) || strides(c).lda != strides(b).ldy) return false;
  return true;
}

// The heads of an attention group starting at descriptor i (each a triple the fused kernel runs,
// all of one shape and sharing the score / probability buffers), with the group's inputs (q, K, V)
// and outputs (scores, probabilities, attention rows). False when there is no such group or its
// outputs meet each other or its inputs.
bool collect_attention(const Checked& first, const std::vector<uint8_t>& q, int32_t i, uint64_t in_image, int32_t n,
                       uint64_t image_len, int core_id, bool gemv_only, uintptr_t img, std::vector<AttnHead>& group,
                       Segs& ins, Segs& outs) {
  group.clear();
  ins.clear();
  if (!g_fusion || first.d[F_OPCODE] != OP_FDOT || (first.d[F_CTRL] & 1)) return false;
  Segs atts, sc_y, pr_y;
  for (int32_t j = i; j + 2 < n && static_cast<uint64_t>(j + 2) < in_image &&
                      group.size() < static_cast<size_t>(tars::kAttnMaxHeads);
       j += 3) {
    const Checked nt = j == i ? first : check(q.data() + static_cast<size_t>(j) * kDescBytes, image_len, core_id, gemv_only);
    const Checked sm = check(q.data() + static_cast<size_t>(j + 1) * kDescBytes, image_len, core_id, gemv_only);
    const Checked nn = check(q.data() + static_cast<size_t>(j + 2) * kDescBytes, image_len, core_id, gemv_only);
    if (!attention_triple(nt, sm, nn, img)) break;
    if (!group.empty()) {  // the same shapes, formats and shared buffers as the first head
      const AttnHead& h0 = group[0];
      if (nt.d[F_M] != h0.nt[F_M] || nt.d[F_N] != h0.nt[F_N] || nt.d[F_K] != h0.nt[F_K] ||
          sm.d[F_K] != h0.sm[F_K] || addr(nt.d, F_Y_OFF) != addr(h0.nt, F_Y_OFF) ||
          strides(nt.d).ldy != strides(h0.nt).ldy || addr(sm.d, F_Y_OFF) != addr(h0.sm, F_Y_OFF) ||
          strides(sm.d).ldy != strides(h0.sm).ldy || strides(nt.d).lda != strides(h0.nt).lda ||
          b_stride(nt.d).first != b_stride(h0.nt).first || b_stride(nn.d).first != b_stride(h0.nn).first ||
          strides(nn.d).ldy != strides(h0.nn).ldy || nn.d[F_HDR_RSV] != h0.nn[F_HDR_RSV] ||
          nn.d[F_EPI] != h0.nn[F_EPI] || nn.d[F_OUT_SCALE] != h0.nn[F_OUT_SCALE])
        break;
    } else {
      sc_y = nt.y;
      pr_y = sm.y;
    }
    for (const Segs& r : nt.reads) ins.insert(ins.end(), r.begin(), r.end());  // q and K
    const Desc& c = nn.d;
    ins.push_back(strided_span(addr(c, F_W_OFF), b_stride(c).first, c[F_K], b_stride(c).second));
    atts.insert(atts.end(), nn.y.begin(), nn.y.end());
    group.push_back(AttnHead{nt.d, sm.d, nn.d});
  }
  if (group.empty()) return false;
  outs = sc_y;
  outs.insert(outs.end(), pr_y.begin(), pr_y.end());
  outs.insert(outs.end(), atts.begin(), atts.end());
  if (!pairwise_disjoint(outs) || overlaps(ins, outs)) {
    group.clear();
    return false;
  }
  return true;
}

int fuse_attention(uint8_t* image, const Checked& first, const std::vector<uint8_t>& q, int32_t i, uint64_t in_image,
                   int32_t n, u128 rest_lo, u128 rest_hi, uint64_t image_len, int core_id, bool gemv_only, hipStream_t s,
                   int& fused, std::vector<AttnHead>& group) {
  fused = 0;
  Segs ins, outs;
  if (!collect_attention(first, q, i, in_image, n, image_len, core_id, gemv_only, reinterpret_cast<uintptr_t>(image),
                         group, ins, outs))
    return TARS_OK;
  if (rest_lo < rest_hi && overlaps(Segs{interval(rest_lo, rest_hi)}, outs)) {
    group.clear();
    return TARS_OK;
  }
  const int rc = launch_attention_group(image, group, s, tars::attention_workspace(s));
  if (rc == TARS_OK) fused = static_cast<int>(group.size());
  return rc;
}

// A residual ELT ADD followed by the norm of its output (a decoder's add -> RMSNorm pairs) runs as
// one launch (tars::launch_add_norm), bit-identical to the two in order. Taken when the ELT is dense
// fp32 with an fp32 output, no activation and no fp16 state, the next descriptor is a LayerNorm /
// RMSNorm / L2Norm whose input rows are exactly the ELT's output rows, the rows fit the kernel, the
// ELT runs in place or apart from its A rows, and no output of the pair lands on the ELT's B rows,
// gamma, beta, the other output, the norm's input, or a later descriptor.
// The kernel arguments of a LayerNorm / RMSNorm / L2Norm descriptor (as tars_row_op builds them).
tars::RowArgs norm_args(uint8_t* image, const Desc& rd) {
  uint8_t* RB = image + rd[F_BASE_ADDR];
  tars::RowArgs r{};
  r.x = RB + rd[F_A_OFF];
  r.lda = static_cast<int64_t>(strides(rd).lda);
  r.fn = static_cast<int>(rd[F_CTRL] & 7);
  r.gamma = reinterpret_cast<const float*>(RB + rd[F_SCALE_OFF]);
  r.beta = has_bias(rd[F_EPI]) ? reinterpret_cast<const float*>(RB + rd[F_BIAS_OFF]) : nullptr;
  r.eps = f32_bits(rd[F_W_OFF]);
  r.y = RB + rd[F_Y_OFF];
  r.ldy = static_cast<int64_t>(strides(rd).ldy);
  r.out = static_cast<int>(out_code(rd[F_EPI]));
  r.out_scale = f32_bits(rd[F_OUT_SCALE]);
  r.M = static_cast<int>(rd[F_M]);
  r.N = static_cast<int>(rd[F_N]);
  return r;
}

int launch_add_norm_pair(uint8_t* image, const Desc& d, const Desc& rd, hipStream_t s) {
  uint8_t* B = image + d[F_BASE_ADDR];
  const int M = static_cast<int>(d[F_M]), N = static_cast<int>(d[F_N]);
  tars::EltArgs e{};
  e.A = B + d[F_A_OFF];
  e.lda = static_cast<int64_t>(strides(d).lda);
  e.B = reinterpret_cast<const float*>(B + d[F_W_OFF]);
  e.ldb = static_cast<int64_t>(b_stride(d).first);
  e.bmode = BM_DENSE;
  e.op = tars::ELTOP_ADD;
  e.Y = B + d[F_Y_OFF];
  e.ldy = static_cast<int64_t>(strides(d).ldy);
  e.M = M;
  e.N = N;
  const hipError_t err = tars::launch_add_norm(e, norm_args(image, rd), s);
  if (err != hipSuccess) {
    tars::set_last_error(std::string("HIP launch failed: ") + hipGetErrorString(err));
    return TARS_E_DEVICE;
  }
  return TARS_OK;
}

int fuse_add_norm(uint8_t* image, const Checked& e, const std::vector<uint8_t>& q, int32_t i, uint64_t in_image,
                  int32_t n, u128 rest_lo, u128 rest_hi, uint64_t image_len, int core_id, bool gemv_only, hipStream_t s,
                  int& fused, Desc& norm) {
  fused = 0;
  const Desc& d = e.d;
  if (!g_fusion || d[F_OPCODE] != OP_ELT || (d[F_CTRL] & 3) != ELT_ADD || d[F_HDR_RSV] != 0 ||
      act_code(d[F_EPI]) != 0 || out_code(d[F_EPI]) != OUT_FP32 || i + 1 >= n || static_cast<uint64_t>(i) + 1 >= in_image)
    return TARS_OK;
  const Checked r = check(q.data() + static_cast<size_t>(i + 1) * kDescBytes, image_len, core_id, gemv_only);
  const Desc& rd = r.d;
  const uint64_t fn = rd[F_CTRL] & 7;
  const uintptr_t img = reinterpret_cast<uintptr_t>(image);
  if (e.err != E_OK || e.overlap || r.err != E_OK || r.overlap || rd[F_OPCODE] != OP_ROW ||
      (fn != ROW_LAYERNORM && fn != ROW_RMSNORM && fn != ROW_L2NORM) || (img + d[F_BASE_ADDR]) % 16 ||
      (img + rd[F_BASE_ADDR]) % 16 || rd[F_M] != d[F_M] || rd[F_N] != d[F_N] ||
      !tars::add_norm_supported(static_cast<int>(d[F_M]), static_cast<int>(d[F_N])) ||
      addr(rd, F_A_OFF) != addr(d, F_Y_OFF) || strides(rd).lda != strides(d).ldy)
    return TARS_OK;
  const uint64_t M = d[F_M], N = d[F_N];
  const Segs a_rows = strided(addr(d, F_A_OFF), strides(d).lda, M, 4 * N);
  Segs ins = strided(addr(d, F_W_OFF), b_stride(d).first, M, 4 * N);
  ins.push_back(interval(addr(rd, F_SCALE_OFF), addr(rd, F_SCALE_OFF) + 4 * N));
  if (has_bias(rd[F_EPI])) ins.push_back(interval(addr(rd, F_BIAS_OFF), addr(rd, F_BIAS_OFF) + 4 * N));
  const bool in_place = addr(d, F_Y_OFF) == addr(d, F_A_OFF) && strides(d).ldy == strides(d).lda;
  Segs outs = e.y;
  outs.insert(outs.end(), r.y.begin(), r.y.end());
  if (!pairwise_disjoint(outs) || overlaps(ins, outs) || overlaps(a_rows, r.y) || (!in_place && overlaps(a_rows, e.y)) ||
      (rest_lo < rest_hi && overlaps(Segs{interval(rest_lo, rest_hi)}, outs)))
    return TARS_OK;
  const int rc = launch_add_norm_pair(image, d, rd, s);
  if (rc == TARS_OK) {
    fused = 1;
    norm = rd;
  }
  return rc;
}

// A residual ELT ADD and its norm (or a norm alone) in front of a decode-row quantizer group: the
// ELT (dense fp32, no activation, fp32 output), the LayerNorm / RMSNorm / L2Norm of exactly its
// output (fp32 output), then a ROW_QUANT of exactly the norm's output with the GEMMs fuse_group
// takes, all on one row (tars_mini/llm.py:640, 699, 767: a residual add, then the next norm and
// projections). They run as one launch whose every workgroup forms the sum and the norm in
// registers (the first workgroup stores both), bit-identical to the descriptors in order. Refused
// when the prologue's outputs land on a later descriptor, or (the fused call's checks) on an input
// or another output of the launch, which excludes an ELT in place; and when K is outside the
// kernel's prologue instances. `fused` = descriptors after i folded into i's launch.
int fuse_norm_group(uint8_t* image, const Checked& c, const std::vector<uint8_t>& q, int32_t i, uint64_t in_image,
                    int32_t n, u128 queue_addr, u128 q_end, uint64_t image_len, int core_id, bool gemv_only, hipStream_t s,
                    int& fused, bool& has_add, Desc& add, Desc& norm, Desc& quant, std::vector<Desc>& group, Desc& elt,
                    bool& gated) {
  fused = 0;
  has_add = false;
  if (!g_fusion) return TARS_OK;
  const Desc& d = c.d;
  auto is_norm = [](const Desc& r) {
    const uint64_t fn = r[F_CTRL] & 7;
    return r[F_OPCODE] == OP_ROW && (fn == ROW_LAYERNORM || fn == ROW_RMSNORM || fn == ROW_L2NORM) &&
           out_code(r[F_EPI]) == OUT_FP32 && r[F_M] == 1;
  };
  if (d[F_OPCODE] == OP_ELT) {
    if ((d[F_CTRL] & 3) != ELT_ADD || d[F_HDR_RSV] != 0 || act_code(d[F_EPI]) != 0 || out_code(d[F_EPI]) != OUT_FP32 ||
        d[F_M] != 1)
      return TARS_OK;
    has_add = true;
  } else if (!is_norm(d)) {
    return TARS_OK;
  }
  const int32_t ir = has_add ? i + 1 : i, iq = ir + 1;
  if (iq + 1 >= n || static_cast<uint64_t>(iq) + 1 >= in_image) return TARS_OK;
  const Checked r = has_add ? check(q.data() + static_cast<size_t>(ir) * kDescBytes, image_len, core_id, gemv_only) : c;
  const Desc& rd = r.d;
  if (r.err != E_OK || r.overlap || !is_norm(rd) || !tars::quant_gemv_norm_supported(static_cast<int>(rd[F_N])) ||
      (has_add && (d[F_N] != rd[F_N] || addr(rd, F_A_OFF) != addr(d, F_Y_OFF))))
    return TARS_OK;
  const Checked qc = check(q.data() + static_cast<size_t>(iq) * kDescBytes, image_len, core_id, gemv_only);
  const Desc& dq = qc.d;
  if (qc.err != E_OK || qc.overlap || dq[F_OPCODE] != OP_ROW || (dq[F_CTRL] & 7) != ROW_QUANT || dq[F_N] != rd[F_N] ||
      addr(dq, F_A_OFF) != addr(rd, F_Y_OFF))
    return TARS_OK;
  const uintptr_t img = reinterpret_cast<uintptr_t>(image);
  auto aligned16 = [&](const Desc& x, Field f) { return (img + x[F_BASE_ADDR] + x[f]) % 16 == 0; };
  if (!aligned16(rd, F_A_OFF) || !aligned16(rd, F_Y_OFF) || !aligned16(rd, F_SCALE_OFF) ||
      (has_bias(rd[F_EPI]) && !aligned16(rd, F_BIAS_OFF)) ||
      (has_add && (!aligned16(d, F_A_OFF) || !aligned16(d, F_W_OFF) || !aligned16(d, F_Y_OFF))))
    return TARS_OK;
  Segs outs = r.y;
  if (has_add) outs.insert(outs.end(), c.y.begin(), c.y.end());
  const u128 later = queue_addr + static_cast<u128>(kDescBytes) * (static_cast<uint64_t>(i) + 1);
  if (later < q_end && overlaps(Segs{interval(later, q_end)}, outs)) return TARS_OK;
  int fq = 0;
  const int rc = fuse_group(image, qc, q, iq, in_image, n,
                            queue_addr + static_cast<u128>(kDescBytes) * (static_cast<uint64_t>(iq) + 1), q_end, image_len,
                            core_id, gemv_only, s, fq, group, elt, gated, has_add ? &d : nullptr, &rd);
  if (rc != TARS_OK || fq == 0) return rc;
  fused = (iq - i) + fq;
  add = d;
  norm = rd;
  quant = dq;
  return TARS_OK;
}

// A norm with an fp32 output followed by the RoPE of its output rows (a decoder's q / k norm and
// rotation) runs as one launch (tars::launch_norm_rope), bit-identical to the two in order. Taken
// when the RoPE's input rows are exactly the norm's output rows, both write fp32, the rows fit the
// kernel, and neither output lands on an input of the pair (the norm's rows, gamma, beta, the
// table), on the other output or on a later descriptor.
tars::RopeArgs rope_args(uint8_t* image, const Desc& pd) {
  uint8_t* PB = image + pd[F_BASE_ADDR];
  tars::RopeArgs p{};
  p.x = PB + pd[F_A_OFF];
  p.lda = static_cast<int64_t>(strides(pd).lda);
  p.tab = reinterpret_cast<const float*>(PB + pd[F_W_OFF]);
  p.rows_per_pos = static_cast<int>(pd[F_GROUP_SIZE]);
  p.rot = static_cast<int>(pd[F_K]);
  p.y = PB + pd[F_Y_OFF];
  p.ldy = static_cast<int64_t>(strides(pd).ldy);
  p.M = static_cast<int>(pd[F_M]);
  p.N = static_cast<int>(pd[F_N]);
  return p;
}

// One fused (norm, RoPE) pair, or two independent ones (r2 / p2 not null) in one launch.
int launch_norm_rope_pair(uint8_t* image, const Desc& rd, const Desc& pd, hipStream_t s, const Desc* r2 = nullptr,
                          const Desc* p2 = nullptr) {
  const hipError_t err = r2 ? tars::launch_norm_rope2(norm_args(image, rd), rope_args(image, pd), norm_args(image, *r2),
                                                      rope_args(image, *p2), s)
                            : tars::launch_norm_rope(norm_args(image, rd), rope_args(image, pd), s);
  if (err != hipSuccess) {
    tars::set_last_error(std::string("HIP launch failed: ") + hipGetErrorString(err));
    return TARS_E_DEVICE;
  }
  return TARS_OK;
}

// Whether descriptors (r, p) form a pair the norm_rope kernel runs (a norm with an fp32 output and
// the RoPE of exactly its output rows, fp32), and the pair's reads and writes.
bool norm_rope_pair(const Checked& r, const Checked& p, uintptr_t img, Segs& ins, Segs& outs) {
  const Desc& rd = r.d;
  const Desc& pd = p.d;
  const uint64_t fn = rd[F_CTRL] & 7;
  if (r.err != E_OK || r.overlap || p.err != E_OK || p.overlap || rd[F_OPCODE] != OP_ROW ||
      (fn != ROW_LAYERNORM && fn != ROW_RMSNORM && fn != ROW_L2NORM) || out_code(rd[F_EPI]) != OUT_FP32 ||
      pd[F_OPCODE] != OP_ROPE || out_code(pd[F_EPI]) != OUT_FP32 || (img + rd[F_BASE_ADDR]) % 16 ||
      (img + pd[F_BASE_ADDR]) % 16 || pd[F_M] != rd[F_M] || pd[F_N] != rd[F_N] ||
      !tars::add_norm_supported(static_cast<int>(rd[F_M]), static_cast<int>(rd[F_N])) ||
      addr(pd, F_A_OFF) != addr(rd, F_Y_OFF) || strides(pd).lda != strides(rd).ldy)
    return false;
  ins.clear();
  for (const Segs& x : r.reads) ins.insert(ins.end(), x.begin(), x.end());
  const uint64_t tab_rows = (pd[F_M] - 1) / pd[F_GROUP_SIZE] + 1;
  ins.push_back(interval(addr(pd, F_W_OFF), addr(pd, F_W_OFF) + static_cast<u128>(4 * pd[F_K]) * tab_rows));
  outs = r.y;
  outs.insert(outs.end(), p.y.begin(), p.y.end());
  return true;
}

// A norm and the RoPE of its output rows as one launch (the pair's outputs disjoint, neither read
// by the pair nor lying on a later descriptor). When the next two descriptors form another such
// pair that neither reads nor writes what the first pair writes, and whose reads the first pair
// does not write (a decoder's q and then k norm and rotation), both pairs run in the same launch.
// `fused` = descriptors folded into descriptor i's launch (1 or 3).
// A decoder's q and k (norm, RoPE) pairs and the attention group right after them, as one attention
// launch whose scores kernel runs the pairs first (AttnArgs::rope). Taken when the attention has one
// query row per head, both norms are of one kind, every RoPE rotates the whole row, the q pair has
// a row per head whose RoPE
// rows are exactly the heads' query rows, the k pair a row per K / V head whose RoPE row g is exactly
// one key row (the same for every head) of that head's keys (the heads of a K / V head
// consecutive), the attention's split form runs, and no write of the launch lands where it could
// change what another part reads: the pairs' outputs apart from the pairs' inputs and from every K
// and V row (the new key row aside), the attention's outputs apart from the pairs' inputs and
// outputs, nothing on a later descriptor.
bool rope_attention(uint8_t* image, const Checked& r, const Checked& p, const Checked& r1, const Checked& p1,
                    const Segs& pins, const Segs& pouts, const std::vector<AttnHead>& heads, const Segs& aouts,
                    const Segs& rest, hipStream_t s, RopePrologue& pro) {
  const size_t H = heads.size();
  const Desc& nt0 = heads[0].nt;
  const uint64_t hd = nt0[F_K], nk = nt0[F_N], ldk = b_stride(nt0).first;
  const uint64_t Hk = r1.d[F_M];
  if (nt0[F_M] != 1 || hd % 32 || r.d[F_N] != hd || r.d[F_M] != H || p.d[F_K] != hd || r1.d[F_N] != hd ||
      p1.d[F_K] != hd || Hk == 0 || H % Hk || ldk < 4 * hd || (r.d[F_CTRL] & 7) != (r1.d[F_CTRL] & 7))
    return false;
  const uint64_t qpk = H / Hk;
  // the key row the k RoPE writes: its row 0 lands on a key row of head 0's keys
  const u128 k0 = addr(nt0, F_W_OFF), r0 = addr(p1.d, F_Y_OFF);
  if (r0 < k0 || (r0 - k0) % ldk || (r0 - k0) / ldk >= nk) return false;
  const uint64_t key = static_cast<uint64_t>((r0 - k0) / ldk);
  Segs kv;  // every K row but the new ones, and every V row
  for (size_t h = 0; h < H; ++h) {
    const Desc& nt = heads[h].nt;
    const Desc& nn = heads[h].nn;
    if (addr(nt, F_A_OFF) != addr(p.d, F_Y_OFF) + static_cast<u128>(h) * strides(p.d).ldy ||
        addr(nt, F_W_OFF) + static_cast<u128>(key) * ldk != addr(p1.d, F_Y_OFF) + static_cast<u128>(h / qpk) * strides(p1.d).ldy ||
        (h % qpk && addr(nt, F_W_OFF) != addr(heads[h - 1].nt, F_W_OFF)))
      return false;
    if (key > 0) kv.push_back(strided_span(addr(nt, F_W_OFF), ldk, key, 4 * hd));
    if (key + 1 < nk) kv.push_back(strided_span(addr(nt, F_W_OFF) + static_cast<u128>(key + 1) * ldk, ldk, nk - 1 - key, 4 * hd));
    kv.push_back(strided_span(addr(nn, F_W_OFF), b_stride(nn).first, nk, b_stride(nn).second));
  }
  const float* ws = tars::attention_workspace(s);
  if (!ws || !tars::attention_split_fits(static_cast<int>(H), 1, static_cast<int>(nk), tars::kAttnScratchFloats))
    return false;
  Segs pall = pins;  // the pairs' inputs and outputs
  pall.insert(pall.end(), pouts.begin(), pouts.end());
  Segs new_keys = p1.y;
  Segs others;  // the pairs' outputs but the new key rows
  for (const Checked* c : {&r, &p, &r1}) others.insert(others.end(), c->y.begin(), c->y.end());
  if (overlaps(others, kv) || overlaps(new_keys, kv) || overlaps(aouts, pall) ||
      (!rest.empty() && (overlaps(rest, pouts) || overlaps(rest, aouts))))
    return false;
  pro = RopePrologue{r.d, p.d, r1.d, p1.d, static_cast<int>(qpk), static_cast<int>(key)};
  return true;
}

int fuse_norm_rope(uint8_t* image, const Checked& r, const std::vector<uint8_t>& q, int32_t i, uint64_t in_image,
                   int32_t n, u128 rest_lo, u128 rest_hi, uint64_t image_len, int core_id, bool gemv_only, hipStream_t s,
                   int& fused, Desc& rope, Desc& r2, Desc& rope2, std::vector<AttnHead>& heads, RopePrologue& pro) {
  fused = 0;
  heads.clear();
  const Desc& rd = r.d;
  const uint64_t fn = rd[F_CTRL] & 7;
  if (!g_fusion || rd[F_OPCODE] != OP_ROW || (fn != ROW_LAYERNORM && fn != ROW_RMSNORM && fn != ROW_L2NORM) ||
      out_code(rd[F_EPI]) != OUT_FP32 || i + 1 >= n || static_cast<uint64_t>(i) + 1 >= in_image)
    return TARS_OK;
  const Checked p = check(q.data() + static_cast<size_t>(i + 1) * kDescBytes, image_len, core_id, gemv_only);
  const uintptr_t img = reinterpret_cast<uintptr_t>(image);
  Segs ins, outs;
  if (!norm_rope_pair(r, p, img, ins, outs)) return TARS_OK;
  const Segs rest = {interval(rest_lo, rest_hi)};
  if (!pairwise_disjoint(outs) || overlaps(ins, outs) || (rest_lo < rest_hi && overlaps(rest, outs))) return TARS_OK;
  bool two = false;
  Checked r1, p1;
  Segs ins1, outs1;
  if (i + 3 < n && static_cast<uint64_t>(i) + 3 < in_image) {
    r1 = check(q.data() + static_cast<size_t>(i + 2) * kDescBytes, image_len, core_id, gemv_only);
    p1 = check(q.data() + static_cast<size_t>(i + 3) * kDescBytes, image_len, core_id, gemv_only);
    if (norm_rope_pair(r1, p1, img, ins1, outs1)) {
      Segs all = outs;
      all.insert(all.end(), outs1.begin(), outs1.end());
      two = pairwise_disjoint(all) && !overlaps(ins1, all) && !overlaps(ins, outs1) &&
            !(rest_lo < rest_hi && overlaps(rest, outs1));
    }
  }
  if (two && i + 4 < n && static_cast<uint64_t>(i) + 4 < in_image) {  // and the attention after them
    const Checked first = check(q.data() + static_cast<size_t>(i + 4) * kDescBytes, image_len, core_id, gemv_only);
    Segs ains, aouts;
    if (first.err == E_OK && !first.overlap &&
        collect_attention(first, q, i + 4, in_image, n, image_len, core_id, gemv_only, img, heads, ains, aouts)) {
      Segs pins = ins, pouts = outs;
      pins.insert(pins.end(), ins1.begin(), ins1.end());
      pouts.insert(pouts.end(), outs1.begin(), outs1.end());
      if (rope_attention(image, r, p, r1, p1, pins, pouts, heads, aouts, rest_lo < rest_hi ? rest : Segs{}, s, pro)) {
        const int rc = launch_attention_group(image, heads, s, tars::attention_workspace(s), &pro);
        if (rc == TARS_OK) fused = 3 + 3 * static_cast<int>(heads.size());
        return rc;
      }
    }
    heads.clear();
  }
  const int rc = two ? launch_norm_rope_pair(image, rd, p.d, s, &r1.d, &p1.d) : launch_norm_rope_pair(image, rd, p.d, s);
  if (rc == TARS_OK) {
    fused = two ? 3 : 1;
    rope = p.d;
    if (two) {
      r2 = r1.d;
      rope2 = p1.d;
    }
  }
  return rc;
}

// ---------------------------------------------------------------------------- launch plans
// A decode loop runs the same descriptor bytes every token. A queue that ran to the end with no
// hand-off and no output over its own descriptors leaves a plan (its launches in order, with the
// decisions the checks made); when the same bytes run again on the same image with the same
// settings, the plan is captured once into a HIP graph (on a private stream; the plan records no
// memset) and every later run is one graph launch. The checks that produced the plan depend only
// on the descriptor bytes, the image address and length, core_id, the profile and the library's
// switches, which are the cache key.
struct Step {
  Desc d;                   // the descriptor (the quantizer of a fused group)
  std::vector<Desc> group;  // the GEMMs fused with it (empty: a single launch)
  std::vector<AttnHead> attn;  // or: the heads of a fused attention launch
  Desc second{};               // or: the second descriptor of a fused pair with d
  bool add_norm = false;       // d an ELT ADD, second its norm
  bool norm_rope = false;      // d a norm, second its RoPE
  Desc third{}, fourth{};      // with norm_rope2: a second (norm, RoPE) pair in the same launch
  bool norm_rope2 = false;
  Desc elt{};                  // a gated group's ELT MUL (gated: group is gate and up)
  bool gated = false;
  Desc pro_add{}, pro_norm{};  // with pro: the group's prologue (pro_has_add: the ELT ADD, then the norm)
  bool pro = false, pro_has_add = false;
  bool rope = false;           // attn: the q and k (norm, RoPE) pairs run in the attention launch
  RopePrologue rope_pro;
};

struct Plan {
  uint8_t* image;
  uint64_t image_len, queue_addr;
  int32_t n;
  int core_id, gemv_only, w8a8_path;
  bool fusion;
  std::vector<uint8_t> bytes;
  std::vector<Step> steps;
  hipGraphExec_t exec = nullptr;
  // The split attention's scores scratch of the plan's graph (allocated with the graph when a step
  // runs attention): the plan's own, so replays on any stream never share it with eager work or with
  // another plan. Freed with the graph (hipFree waits for the device first).
  float* scratch = nullptr;
  uint64_t last_use = 0;
};

void drop_graph(Plan& p) {
  if (p.exec) (void)hipGraphExecDestroy(p.exec);
  if (p.scratch) (void)hipFree(p.scratch);
  p.exec = nullptr;
  p.scratch = nullptr;
}

// Fused launches run (diagnostics for tests and benchmarks): quantizer + GEMMs, attention,
// residual ADD + norm, norm + RoPE pairs (two when two pairs share a launch), launches that ran two
// such pairs, and (also counted as quantizer + GEMMs) the gated product's ELT MUL folded into its
// GEMMs and a norm (with its residual ADD) in front of the quantizer, and (also counted as
// attention and as two norm + RoPE pairs) attention launches that ran a layer's q and k norm + RoPE
// pairs; counted when a queue is dispatched and when a plan replays.
constexpr int kFusionKinds = 8;
std::atomic<int64_t> g_fused_launches[kFusionKinds];

void count_fused(const std::vector<Step>& steps) {
  for (const Step& st : steps) {
    const int k = !st.group.empty() ? 0 : !st.attn.empty() ? 1 : st.add_norm ? 2 : st.norm_rope ? 3 : -1;
    if (k >= 0) g_fused_launches[k].fetch_add(st.norm_rope2 ? 2 : 1, std::memory_order_relaxed);
    if (st.gated) g_fused_launches[4].fetch_add(1, std::memory_order_relaxed);
    if (st.norm_rope2) g_fused_launches[5].fetch_add(1, std::memory_order_relaxed);
    if (st.pro) g_fused_launches[6].fetch_add(1, std::memory_order_relaxed);
    if (st.rope) {
      g_fused_launches[3].fetch_add(2, std::memory_order_relaxed);
      g_fused_launches[7].fetch_add(1, std::memory_order_relaxed);
    }
  }
}

constexpr size_t kMaxPlans = 8;
std::mutex g_plans_mu;
std::vector<Plan> g_plans;
uint64_t g_plan_clock = 0;
bool g_graphs = true;

int replay_steps(uint8_t* image, const std::vector<Step>& steps, hipStream_t s, float* scratch) {
  for (const Step& st : steps) {
    bool needs_host = false;
    const int rc = st.add_norm        ? launch_add_norm_pair(image, st.d, st.second, s)
                   : st.norm_rope     ? launch_norm_rope_pair(image, st.d, st.second, s, st.norm_rope2 ? &st.third : nullptr,
                                                          st.norm_rope2 ? &st.fourth : nullptr)
                   : !st.attn.empty() ? launch_attention_group(image, st.attn, s, scratch, st.rope ? &st.rope_pro : nullptr)
                   : st.group.empty() ? launch(image, st.d, s, needs_host)
                                      : launch_fused(image, st.d, st.group, s, st.gated ? &st.elt : nullptr,
                                                     st.pro_has_add ? &st.pro_add : nullptr, st.pro ? &st.pro_norm : nullptr);
    if (rc != TARS_OK) return rc;
  }
  return TARS_OK;
}

// The graph of a plan's launches (captured on a private default-priority stream).
int capture(Plan& p) {
  const bool attn = std::any_of(p.steps.begin(), p.steps.end(), [](const Step& st) { return !st.attn.empty(); });
  if (attn && !p.scratch) {
    void* m = nullptr;
    if (hipMalloc(&m, static_cast<size_t>(tars::kAttnScratchFloats) * sizeof(float)) != hipSuccess) {
      (void)hipGetLastError();
      return TARS_E_DEVICE;
    }
    p.scratch = static_cast<float*>(m);
  }
  hipStream_t cs = nullptr;
  if (hipStreamCreateWithFlags(&cs, hipStreamNonBlocking) != hipSuccess) return TARS_E_DEVICE;
  hipGraph_t g = nullptr;
  int rc = TARS_OK;
  if (hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal) != hipSuccess) {
    rc = TARS_E_DEVICE;
  } else {
    rc = replay_steps(p.image, p.steps, cs, p.scratch);
    if (hipStreamEndCapture(cs, &g) != hipSuccess && rc == TARS_OK) rc = TARS_E_DEVICE;
  }
  if (rc == TARS_OK && hipGraphInstantiate(&p.exec, g, nullptr, nullptr, 0) != hipSuccess) {
    p.exec = nullptr;
    rc = TARS_E_DEVICE;
  }
  if (g) (void)hipGraphDestroy(g);
  (void)hipStreamDestroy(cs);
  return rc;
}


}  // namespace

namespace {

int queue_fail(int code, const std::string& what) {
  tars::set_last_error(what);
  return code;
}

}  // namespace

extern "C" {

int tars_check_descriptor(const uint8_t* desc, uint64_t image_len, int32_t core_id, int32_t gemv_only,
                          int32_t* err_code, int32_t* gpu) {
  tars::set_last_error("");
  if (!desc || !err_code) return queue_fail(TARS_E_ARG, "NULL descriptor or err_code");
  const Checked c = check(desc, image_len, core_id, gemv_only != 0);
  *err_code = c.err;
  if (gpu) *gpu = (c.err == E_OK && !c.overlap && gpu_kind(c.d)) ? 1 : 0;
  if (c.err == E_OK && c.overlap) return queue_fail(TARS_E_OVERLAP, "an output overlaps an input");
  return TARS_OK;
}

int tars_decode_descriptor(const uint8_t* desc, uint64_t* fields) {
  if (!desc || !fields) return TARS_E_ARG;
  const Desc d = decode(desc);
  for (int i = 0; i < kFields; ++i) fields[i] = d.f[i];
  return TARS_OK;
}

uint32_t tars_descriptor_crc(const uint8_t* desc) { return desc ? crc32_desc(desc) : 0u; }

int tars_encode_descriptor(const uint64_t* fields, int32_t fix_crc, uint8_t* desc) {
  tars::set_last_error("");
  if (!fields || !desc) return queue_fail(TARS_E_ARG, "NULL fields or descriptor");
  uint8_t raw[kDescBytes] = {};
  for (int i = 0; i < kFields; ++i) {
    const BitRange r = kBits[i];
    if (r.width < 64 && (fields[i] >> r.width) != 0)
      return queue_fail(TARS_E_ARG, "a field value does not fit its width");
    for (int b = 0; b < r.width; ++b)
      if ((fields[i] >> b) & 1) raw[(r.lo + b) / 8] |= static_cast<uint8_t>(1u << ((r.lo + b) % 8));
  }
  if (fix_crc) {
    const uint32_t c = crc32_desc(raw);
    for (int b = 0; b < 4; ++b) raw[4 + b] = static_cast<uint8_t>(c >> (8 * b));
  }
  std::memcpy(desc, raw, kDescBytes);
  return TARS_OK;
}

int tars_set_queue_fusion(int on) {
  const int prev = g_fusion ? 1 : 0;
  g_fusion = on != 0;
  return prev;
}

int tars_run_queue(uint8_t* image, uint64_t image_len, uint64_t queue_addr, int32_t n, const uint8_t* host_queue,
                   int32_t core_id, int32_t gemv_only, tars_queue_status* st, void* stream) {
  tars::set_last_error("");
  if (!image || !st || n < 0) return queue_fail(TARS_E_ARG, "NULL image or status, or n < 0");
  hipStream_t s = static_cast<hipStream_t>(stream);
  *st = tars_queue_status{0, E_OK, 0, 0};
  // the descriptors that lie inside the image, read after the stream's earlier work
  const u128 q_end = static_cast<u128>(queue_addr) + static_cast<u128>(kDescBytes) * static_cast<uint64_t>(n);
  const uint64_t in_image = queue_addr >= image_len ? 0
                            : static_cast<uint64_t>(std::min<u128>(q_end, image_len) - queue_addr) / kDescBytes;
  std::vector<uint8_t> q(static_cast<size_t>(in_image) * kDescBytes);
  auto reread = [&](uint64_t from) -> int {
    if (from >= in_image) return TARS_OK;
    const size_t off = static_cast<size_t>(from * kDescBytes);
    if (hipMemcpyAsync(q.data() + off, image + queue_addr + off, q.size() - off, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
      return queue_fail(TARS_E_DEVICE, "reading the queue from the image failed");
    return TARS_OK;
  };
  if (host_queue) {
    if (!q.empty()) std::memcpy(q.data(), host_queue, q.size());
  } else if (int rc = reread(0)) {
    return rc;
  }
  const int path = tars::w8a8_path();
  auto same_key = [&](const Plan& p) {
    return p.image == image && p.image_len == image_len && p.queue_addr == queue_addr && p.n == n &&
           p.core_id == core_id && p.gemv_only == gemv_only && p.w8a8_path == path && p.fusion == g_fusion &&
           p.bytes.size() == q.size() && std::memcmp(p.bytes.data(), q.data(), q.size()) == 0;
  };
  if (g_graphs) {
    std::lock_guard<std::mutex> lock(g_plans_mu);
    for (size_t k = 0; k < g_plans.size(); ++k) {
      Plan& p = g_plans[k];
      if (!same_key(p)) continue;
      if (!p.exec && capture(p) != TARS_OK) {  // no graph for this plan: forget it, run the queue as usual
        drop_graph(p);
        g_plans.erase(g_plans.begin() + static_cast<std::ptrdiff_t>(k));
        break;
      }
      if (hipGraphLaunch(p.exec, s) != hipSuccess) return queue_fail(TARS_E_DEVICE, "graph launch failed");
      count_fused(p.steps);
      p.last_use = ++g_plan_clock;
      st->done = 1;
      st->op_idx = n;
      return TARS_OK;
    }
  }
  std::vector<Step> steps;
  bool cacheable = g_graphs && in_image == static_cast<uint64_t>(n);
  for (int32_t i = 0; i < n; ++i) {
    st->op_idx = i;
    if (static_cast<uint64_t>(i) >= in_image) {  // the descriptor itself lies past the image
      st->err_code = E_RANGE;
      return TARS_OK;
    }
    const uint8_t* raw = q.data() + static_cast<size_t>(i) * kDescBytes;
    const Checked c = check(raw, image_len, core_id, gemv_only != 0);
    if (c.err != E_OK) {
      st->err_code = c.err;
      return TARS_OK;
    }
    if (c.overlap) return queue_fail(TARS_E_OVERLAP, "descriptor " + std::to_string(i) + ": an output overlaps an input");
    if (!gpu_kind(c.d)) {
      st->host_op = 1;
      return TARS_OK;
    }
    const u128 later = static_cast<u128>(queue_addr) + static_cast<u128>(kDescBytes) * (static_cast<uint64_t>(i) + 1);
    int fused = 0;
    std::vector<Desc> group;
    Desc elt{};
    bool gated = false;
    if (int rc = fuse_group(image, c, q, i, in_image, n, later, q_end, image_len, core_id, gemv_only != 0, s, fused,
                            group, elt, gated))
      return queue_fail(rc, "descriptor " + std::to_string(i) + ": " + tars_last_error());
    if (fused) {
      g_fused_launches[0].fetch_add(1, std::memory_order_relaxed);
      if (gated) g_fused_launches[4].fetch_add(1, std::memory_order_relaxed);
      if (cacheable) {
        Step st{c.d, std::move(group), {}};
        st.elt = elt;
        st.gated = gated;
        steps.push_back(std::move(st));
      }
      i += fused;  // the quantizer and `fused` GEMMs (and a gated product's ELT) ran as one launch
      continue;
    }
    std::vector<AttnHead> heads;
    if (int rc = fuse_attention(image, c, q, i, in_image, n, static_cast<u128>(queue_addr) + static_cast<u128>(kDescBytes) *
                                (static_cast<uint64_t>(i) + 3), q_end, image_len, core_id, gemv_only != 0, s, fused, heads))
      return queue_fail(rc, "descriptor " + std::to_string(i) + ": " + tars_last_error());
    if (fused) {
      g_fused_launches[1].fetch_add(1, std::memory_order_relaxed);
      if (cacheable) steps.push_back(Step{c.d, {}, std::move(heads)});
      i += 3 * fused - 1;  // `fused` heads of three descriptors ran as one launch
      continue;
    }
    {
      bool has_add = false;
      Desc add{}, nrm{}, quant{};
      if (int rc = fuse_norm_group(image, c, q, i, in_image, n, static_cast<u128>(queue_addr), q_end, image_len, core_id,
                                   gemv_only != 0, s, fused, has_add, add, nrm, quant, group, elt, gated))
        return queue_fail(rc, "descriptor " + std::to_string(i) + ": " + tars_last_error());
      if (fused) {
        g_fused_launches[0].fetch_add(1, std::memory_order_relaxed);
        g_fused_launches[6].fetch_add(1, std::memory_order_relaxed);
        if (gated) g_fused_launches[4].fetch_add(1, std::memory_order_relaxed);
        if (cacheable) {
          Step st{quant, std::move(group), {}};
          st.elt = elt;
          st.gated = gated;
          st.pro = true;
          st.pro_has_add = has_add;
          st.pro_add = add;
          st.pro_norm = nrm;
          steps.push_back(std::move(st));
        }
        i += fused;  // the (ELT and) norm, the quantizer and its GEMMs (and a gated ELT) ran as one launch
        continue;
      }
    }
    Desc norm{};
    if (int rc = fuse_add_norm(image, c, q, i, in_image, n, static_cast<u128>(queue_addr) + static_cast<u128>(kDescBytes) *
                               (static_cast<uint64_t>(i) + 2), q_end, image_len, core_id, gemv_only != 0, s, fused, norm))
      return queue_fail(rc, "descriptor " + std::to_string(i) + ": " + tars_last_error());
    if (fused) {
      g_fused_launches[2].fetch_add(1, std::memory_order_relaxed);
      if (cacheable) {
        Step st2{c.d, {}, {}};
        st2.second = norm;
        st2.add_norm = true;
        steps.push_back(std::move(st2));
      }
      ++i;  // the ELT and its norm ran as one launch
      continue;
    }
    Desc rope{}, norm2{}, rope2{};
    std::vector<AttnHead> rheads;
    RopePrologue rpro;
    if (int rc = fuse_norm_rope(image, c, q, i, in_image, n, static_cast<u128>(queue_addr) + static_cast<u128>(kDescBytes) *
                                (static_cast<uint64_t>(i) + 2), q_end, image_len, core_id, gemv_only != 0, s, fused, rope,
                                norm2, rope2, rheads, rpro))
      return queue_fail(rc, "descriptor " + std::to_string(i) + ": " + tars_last_error());
    if (fused && !rheads.empty()) {
      g_fused_launches[1].fetch_add(1, std::memory_order_relaxed);
      g_fused_launches[3].fetch_add(2, std::memory_order_relaxed);
      g_fused_launches[7].fetch_add(1, std::memory_order_relaxed);
      if (cacheable) {
        Step st2{c.d, {}, std::move(rheads)};
        st2.rope = true;
        st2.rope_pro = rpro;
        steps.push_back(std::move(st2));
      }
      i += fused;  // the q and k (norm, RoPE) pairs and the attention ran as one attention launch
      continue;
    }
    if (fused) {
      g_fused_launches[3].fetch_add(fused == 3 ? 2 : 1, std::memory_order_relaxed);
      if (fused == 3) g_fused_launches[5].fetch_add(1, std::memory_order_relaxed);
      if (cacheable) {
        Step st2{c.d, {}, {}};
        st2.second = rope;
        st2.norm_rope = true;
        if (fused == 3) {
          st2.third = norm2;
          st2.fourth = rope2;
          st2.norm_rope2 = true;
        }
        steps.push_back(std::move(st2));
      }
      i += fused;  // one or two (norm, RoPE) pairs ran as one launch
      continue;
    }
    bool needs_host = false;
    if (int rc = launch(image, c.d, s, needs_host)) {
      return queue_fail(rc, "descriptor " + std::to_string(i) + ": " + tars_last_error());
    }
    if (needs_host) {
      st->host_op = 1;
      return TARS_OK;
    }
    if (cacheable) steps.push_back(Step{c.d, {}, {}});
    // an output written over a later descriptor of this queue: wait for it and read them again
    const Segs rest = {interval(later, q_end)};
    if (later < q_end && (overlaps(rest, c.y) || (!c.extra.empty() && overlaps(rest, c.extra)))) {
      cacheable = false;
      if (int rc = reread(static_cast<uint64_t>(i) + 1)) return rc;
    }
  }
  st->done = 1;
  st->op_idx = n;
  if (cacheable) {
    std::lock_guard<std::mutex> lock(g_plans_mu);
    if (g_plans.size() >= kMaxPlans) {
      auto lru = std::min_element(g_plans.begin(), g_plans.end(),
                                  [](const Plan& a, const Plan& b) { return a.last_use < b.last_use; });
      drop_graph(*lru);
      g_plans.erase(lru);
    }
    Plan p;
    p.image = image;
    p.image_len = image_len;
    p.queue_addr = queue_addr;
    p.n = n;
    p.core_id = core_id;
    p.gemv_only = gemv_only;
    p.w8a8_path = path;
    p.fusion = g_fusion;
    p.bytes = std::move(q);
    p.steps = std::move(steps);
    p.last_use = ++g_plan_clock;
    g_plans.push_back(std::move(p));
  }
  return TARS_OK;
}

int tars_queue_fusion_counts(int64_t* counts, int32_t ncounts, int32_t reset) {
  if (ncounts < 0) return TARS_E_ARG;
  for (int k = 0; k < kFusionKinds; ++k) {
    const int64_t v = reset ? g_fused_launches[k].exchange(0) : g_fused_launches[k].load();
    if (counts && k < ncounts) counts[k] = v;
  }
  return TARS_OK;
}

int tars_set_queue_graphs(int on) {
  std::lock_guard<std::mutex> lock(g_plans_mu);
  const int prev = g_graphs ? 1 : 0;
  g_graphs = on != 0;
  if (!g_graphs) {
    for (Plan& p : g_plans) drop_graph(p);
    g_plans.clear();
  }
  return prev;
}

}  // extern "C"
