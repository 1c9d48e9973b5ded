"""Codes of the openTARS descriptor contract used by the matrix path (tars_mini/contract.py:88-111).

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
