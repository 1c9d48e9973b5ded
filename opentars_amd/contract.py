"""Codes of the openTARS descriptor contract used by the matrix path and the queue executor
(tars_mini/contract.py:39-133).

The values are the contract's own (they are what a descriptor carries), so they must be equal.
"""
from __future__ import annotations

# quantization modes (CTRL[2:0])
QM_NONE, QM_TENSOR, QM_CHANNEL, QM_ROWCOL = 0, 1, 2, 3
QM_GROUP = QM_ROWCOL
# element types (CTRL a_dtype / w_dtype)
DT_BF16, DT_INT8, DT_INT4, DT_FP8, DT_FP32 = 0, 1, 2, 3, 4
W4_GROUP = 128
# epilogue activation (EPI[1:0] | EPI[5] << 2) and output format (EPI[3:2])
ACT_NONE, ACT_RELU, ACT_RELU6, ACT_GELU, ACT_SILU, ACT_SIGMOID, ACT_SOFTPLUS, ACT_EXP = range(8)
OUT_FP32, OUT_BF16, OUT_INT8, OUT_FP16 = 0, 1, 2, 3
ESIZE = {OUT_FP32: 4, OUT_BF16: 2, OUT_INT8: 1, OUT_FP16: 2}
# queue error codes (CSR 0x803), lowest failing check wins
E_OK, E_MAGIC, E_VERSION, E_CRC, E_VALID, E_OPCODE, E_FIELD, E_ALIGN, E_RANGE = range(9)
ERR_NAMES = {E_OK: "OK", E_MAGIC: "E_MAGIC", E_VERSION: "E_VERSION", E_CRC: "E_CRC", E_VALID: "E_VALID",
             E_OPCODE: "E_OPCODE", E_FIELD: "E_FIELD", E_ALIGN: "E_ALIGN", E_RANGE: "E_RANGE"}
K_MAX = 65535
GEMV_K = 4096        # the KV260 GEMV unit's longest x: the reference splits longer K (llm.py:195)

# descriptor header and opcodes (contract.py:39-57, 74-86)
MAGIC, VERSION = 0xAA55, 0x0002
DESC_BYTES = 64
OP_CONV, OP_GEMM, OP_RELU, OP_ROW, OP_CONV_ACT, OP_ELT, OP_ROPE, OP_FDOT = 1, 2, 3, 4, 5, 6, 7, 8
ROW_SOFTMAX, ROW_LAYERNORM, ROW_RMSNORM, ROW_L2NORM, ROW_QUANT = 0, 1, 2, 3, 4
# ELT op (CTRL[1:0]), B / A broadcast (HDR_RSV[1:0] / HDR_RSV[2]), fp16 state (HDR_RSV[3]) and FDOT
# layout (CTRL[0]) of the row-engine opcodes (contract.py:63-72, 102-104)
ELT_MUL, ELT_ADD, ELT_MULADD, ELT_SUB = 0, 1, 2, 3
BM_DENSE, BM_ROW, BM_COL, BM_SCALAR = 0, 1, 2, 3
FDOT_NT, FDOT_NN = 0, 1
STATE_FP16 = 1 << 3


def ctrl(qmode: int = QM_TENSOR, symmetric: int = 1, a_dtype: int = DT_INT8, w_dtype: int = DT_INT8,
         fusion: int = 0) -> int:
    """The CTRL field: qmode[2:0], symmetric[3], a_dtype[7:4], w_dtype[11:8], fusion[12]."""
    return (qmode & 7) | (symmetric & 1) << 3 | (a_dtype & 15) << 4 | (w_dtype & 15) << 8 | (fusion & 1) << 12


def epi(act: int = ACT_NONE, out: int = OUT_FP32, bias: int = 0) -> int:
    """The EPI field: act[1:0], out[3:2], bias[4], act[2] at bit 5."""
    return (act & 3) | (out & 3) << 2 | (bias & 1) << 4 | (act >> 2 & 1) << 5
