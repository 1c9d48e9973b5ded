"""Writes tests/golden/descriptor_cases.json: the reference's descriptor test tables as data.

Each case is a descriptor (its field values; CTRL / EPI spelled with the contract's bit packing,
contract.py:121-133), the image size and profile it is checked with, and the ERR_CODE the
reference's tests expect. Sources (reference repository):
  tests/test_golden.py:73-82 (_base), :93-113 (test_error_codes), :122-125 (test_crc_error),
      :128-131 (test_field_error_has_priority_over_align)
  tests/test_v04.py:14, :170-172 (_desc), :175-205 (test_v04_rules)
  tests/test_w4a16.py:14-26 (_desc, _w4), :182-196 (test_w4_rules, gemv_only profile),
      :219-238 (test_w4_ranges_and_segments)
  tests/test_contract.py:12-14, :47-84 (the contract document's worked example)
The expected codes are the reference's; nothing here runs reference code.

    python tests/golden/make_descriptor_cases.py
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

E_OK, E_MAGIC, E_VERSION, E_CRC, E_VALID, E_OPCODE, E_FIELD, E_ALIGN, E_RANGE = range(9)
MAGIC, VERSION = 0xAA55, 0x0002
OP_CONV, OP_GEMM, OP_RELU, OP_ROW, OP_ELT, OP_ROPE, OP_FDOT = 1, 2, 3, 4, 6, 7, 8
QM_NONE, QM_TENSOR, QM_CHANNEL, QM_ROWCOL = 0, 1, 2, 3
DT_BF16, DT_INT8, DT_INT4, DT_FP32 = 0, 1, 2, 4
OUT_FP32, OUT_BF16, OUT_INT8 = 0, 1, 2
ACT_RELU, ACT_SOFTPLUS, ACT_EXP = 1, 6, 7
ROW_SOFTMAX, ROW_RMSNORM, ROW_L2NORM, ROW_QUANT = 0, 2, 3, 4
ELT_MULADD = 2
BM_COL, BM_SCALAR = 2, 3


def ctrl(qmode=QM_TENSOR, symmetric=1, a_dtype=DT_INT8, w_dtype=DT_INT8, fusion=0):
    return (qmode & 7) | (symmetric & 1) << 3 | (a_dtype & 15) << 4 | (w_dtype & 15) << 8 | (fusion & 1) << 12


def epi(act=0, out=OUT_FP32, bias=0):
    return (act & 3) | (out & 3) << 2 | (bias & 1) << 4 | (act >> 2 & 1) << 5


def f32_bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


cases = []

# ---- test_golden.py: one GEMM at 0x2000 in a 16 KiB image
good = dict(MAGIC=MAGIC, VERSION=VERSION, OPCODE=OP_GEMM, CTRL=ctrl(QM_TENSOR), EPI=epi(), BASE_ADDR=0,
            A_OFF=0x100, W_OFF=0x200, Y_OFF=0x800, SCALE_OFF=0x400, M=1, N=16, K=16, VALID=1)
golden_table = [
    (E_MAGIC, {"MAGIC": 0x55AA}), (E_VERSION, {"VERSION": 1}), (E_VALID, {"VALID": 0}),
    (E_OPCODE, {"OPCODE": 0x0F}), (E_FIELD, {"CORE_ID": 1}), (E_FIELD, {"HDR_RSV": 1}),
    (E_FIELD, {"DEP_SIG": 1}), (E_FIELD, {"GROUP_SIZE": 128}), (E_FIELD, {"CTRL": ctrl(QM_NONE)}),
    (E_FIELD, {"CTRL": ctrl(QM_TENSOR, a_dtype=DT_BF16)}), (E_FIELD, {"CTRL": ctrl(QM_TENSOR, fusion=1)}),
    (E_FIELD, {"EPI": epi(ACT_RELU)}), (E_FIELD, {"OUT_SCALE": 1}), (E_ALIGN, {"N": 8}), (E_ALIGN, {"K": 24}),
    (E_ALIGN, {"M": 0}), (E_ALIGN, {"A_OFF": 0x108}), (E_RANGE, {"Y_OFF": 0x3FF0}),
    (E_RANGE, {"BASE_ADDR": 1 << 40}),
]
for code, change in golden_table:
    cases.append(dict(src="test_golden.py:93-119", image=1 << 14, gemv_only=False, fields={**good, **change},
                      fix_crc=True, expect=code))
cases.append(dict(src="test_golden.py:122-125", image=1 << 14, gemv_only=False, fields=good, fix_crc=False,
                  expect=E_CRC))
cases.append(dict(src="test_golden.py:128-131", image=1 << 14, gemv_only=False,
                  fields={**good, "CORE_ID": 1, "N": 8}, fix_crc=True, expect=E_FIELD))
cases.append(dict(src="test_golden.py:73-82 (the base GEMM)", image=1 << 14, gemv_only=False, fields=good,
                  fix_crc=True, expect=E_OK))

# ---- test_v04.py: single descriptors in a 64 KiB image
v04 = dict(MAGIC=MAGIC, VERSION=VERSION, VALID=1, A_OFF=0x100, Y_OFF=0x800, W_OFF=0x1000, M=2, N=16)
v04_table = [
    (dict(OPCODE=OP_ELT, CTRL=4), E_FIELD),
    (dict(OPCODE=OP_ELT, HDR_RSV=16), E_FIELD),
    (dict(OPCODE=OP_ELT, CTRL=ELT_MULADD), E_FIELD),
    (dict(OPCODE=OP_ELT, EPI=epi(bias=1), BIAS_OFF=0x400), E_FIELD),
    (dict(OPCODE=OP_ELT, CTRL=ELT_MULADD, EPI=epi(out=OUT_BF16, bias=1), BIAS_OFF=0x400), E_FIELD),
    (dict(OPCODE=OP_ELT, K=16), E_FIELD),
    (dict(OPCODE=OP_ELT, W_OFF=0x1004), E_ALIGN),
    (dict(OPCODE=OP_ELT, W_OFF=0x1004, HDR_RSV=BM_SCALAR), E_OK),
    (dict(OPCODE=OP_ELT, W_OFF=0x1002, HDR_RSV=BM_COL), E_ALIGN),
    (dict(OPCODE=OP_ELT, GROUP_SIZE=1), E_ALIGN),
    (dict(OPCODE=OP_ROPE, K=16, GROUP_SIZE=1), E_ALIGN),
    (dict(OPCODE=OP_ROPE, K=32, N=16, GROUP_SIZE=1), E_ALIGN),
    (dict(OPCODE=OP_ROPE, K=16), E_FIELD),
    (dict(OPCODE=OP_ROPE, K=16, GROUP_SIZE=1, EPI=epi(ACT_EXP)), E_FIELD),
    (dict(OPCODE=OP_FDOT, K=16, CTRL=2), E_FIELD),
    (dict(OPCODE=OP_FDOT, K=8), E_ALIGN),
    (dict(OPCODE=OP_FDOT, K=16, EPI=epi(bias=1), BIAS_OFF=0x400), E_FIELD),
    (dict(OPCODE=OP_FDOT, K=16), E_OK),
    (dict(OPCODE=OP_ROW, CTRL=5, SCALE_OFF=0x400), E_FIELD),
    (dict(OPCODE=OP_ROW, CTRL=ROW_QUANT, SCALE_OFF=0x400, W_OFF=0), E_FIELD),
    (dict(OPCODE=OP_ROW, CTRL=ROW_QUANT, SCALE_OFF=0x400, W_OFF=0, EPI=epi(out=OUT_INT8)), E_OK),
    (dict(OPCODE=OP_ROW, CTRL=ROW_QUANT, SCALE_OFF=0x400, EPI=epi(out=OUT_INT8)), E_FIELD),
    (dict(OPCODE=OP_ROW, CTRL=ROW_RMSNORM, SCALE_OFF=0x400, K=1), E_FIELD),
    (dict(OPCODE=OP_ROW, CTRL=ROW_SOFTMAX, W_OFF=0, K=3), E_OK),
    (dict(OPCODE=OP_ROW, CTRL=ROW_L2NORM, SCALE_OFF=0x400, W_OFF=f32_bits(1e-6)), E_OK),
    (dict(OPCODE=OP_GEMM, CTRL=ctrl(QM_ROWCOL), K=16, SCALE_OFF=0x400, HDR_RSV=0x50), E_OK),
    (dict(OPCODE=OP_CONV, CTRL=ctrl(QM_ROWCOL), K=16), E_FIELD),
    (dict(OPCODE=OP_GEMM, CTRL=ctrl(QM_CHANNEL), K=16, HDR_RSV=1), E_FIELD),
    (dict(OPCODE=OP_RELU, EPI=epi(ACT_SOFTPLUS), W_OFF=0), E_OK),
    (dict(OPCODE=0x09), E_OPCODE),
]
for change, code in v04_table:
    cases.append(dict(src="test_v04.py:175-205", image=1 << 16, gemv_only=False, fields={**v04, **change},
                      fix_crc=True, expect=code))

# ---- test_w4a16.py: W4A16 descriptors, gemv_only profile
w4desc = dict(MAGIC=MAGIC, VERSION=VERSION, VALID=1, A_OFF=0x100, Y_OFF=0x4000, W_OFF=0x1000, M=2, N=16)


def w4(**f):
    base = dict(OPCODE=OP_GEMM, CTRL=ctrl(QM_ROWCOL, a_dtype=DT_FP32, w_dtype=DT_INT4), K=256, GROUP_SIZE=128,
                SCALE_OFF=0x400)
    base.update(f)
    return base


w4_table = [
    (w4(), E_OK),
    (w4(CTRL=ctrl(QM_ROWCOL, a_dtype=DT_BF16, w_dtype=DT_INT4)), E_OK),
    (w4(CTRL=ctrl(QM_ROWCOL, a_dtype=DT_INT8, w_dtype=DT_INT4)), E_FIELD),
    (w4(CTRL=ctrl(QM_CHANNEL, a_dtype=DT_FP32, w_dtype=DT_INT4)), E_FIELD),
    (w4(CTRL=ctrl(QM_ROWCOL, a_dtype=DT_FP32, w_dtype=DT_INT4, symmetric=0)), E_FIELD),
    (w4(HDR_RSV=1), E_FIELD),
    (w4(GROUP_SIZE=0), E_FIELD),
    (w4(GROUP_SIZE=64), E_FIELD),
    (w4(K=64), E_ALIGN),
    (w4(K=384 - 128 + 64), E_ALIGN),
    (w4(LDA16=16), E_ALIGN),
    (w4(A_OFF=0x104), E_ALIGN),
    (w4(CTRL=ctrl(QM_ROWCOL), GROUP_SIZE=128), E_FIELD),
]
for change, code in w4_table:
    cases.append(dict(src="test_w4a16.py:182-196", image=1 << 16, gemv_only=True, fields={**w4desc, **change},
                      fix_crc=True, expect=code))
for field, size in (("W_OFF", 32 * 128), ("SCALE_OFF", 32 * 2 * 2)):
    for over in (False, True):
        ff = w4(M=3, N=32, K=256)
        ff[field] = (1 << 16) - size + ((128 if field == "W_OFF" else 16) if over else 0)
        cases.append(dict(src="test_w4a16.py:219-238", image=1 << 16, gemv_only=False, fields={**w4desc, **ff},
                          fix_crc=True, expect=E_RANGE if over else E_OK))

worked = dict(
    src="test_contract.py:12-14,47-84",
    desc_hex=("000000807FC4843700000000000020001000020000070000000600000010000000020000000100"
              "000000000000000000150000001A11020000000000020055AA"),
    fields=dict(MAGIC=MAGIC, VERSION=VERSION, OPCODE=OP_GEMM, BASE_ADDR=0, A_OFF=0x100, W_OFF=0x200,
                SCALE_OFF=0x600, BIAS_OFF=0x700, Y_OFF=0x1000, M=2, N=16, K=32, VALID=1,
                CTRL=ctrl(QM_CHANNEL, fusion=1), EPI=epi(ACT_RELU, OUT_BF16, bias=1)),
    crc=0x3784C47F, ctrl=0x111A, epi=0x0015,
    # inputs: numpy default_rng(2026): A int8 (2, 32), W int8 (16, 32), S = uniform(0.5, 2, 16) / 4096
    # as fp32, B = uniform(-8, 8, 16) as fp32; queue at 0x8000 in a 64 KiB image
    queue_addr=0x8000, image=1 << 16, y_elem01_bf16=0x3F16, acc01=-11968,
    scale1_bits=0x39F80671, bias1_bits=0x40C7EA42, pre_act01_bits=0x3F15EC68,
)

out = Path(__file__).resolve().parent / "descriptor_cases.json"
out.write_text(json.dumps({"cases": cases, "worked_example": worked}, indent=1))
print(f"{len(cases)} cases -> {out}")
