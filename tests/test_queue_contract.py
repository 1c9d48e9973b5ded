"""The descriptor contract on the CPU: the oracle's codec, validator, segments and queue walk pinned
against the reference's own tables and worked example (tests/golden/descriptor_cases.json), and
the library's native decoder, CRC and validator (tars_check_descriptor, host only) compared with
the oracle on those cases and on a large fuzz of mutated descriptors of every opcode."""
from __future__ import annotations

import json
import struct
import zlib
from pathlib import Path

import numpy as np
import pytest

from oracle import golden as G
from oracle import numerics as F
from oracle import queue as Q

CASES = json.loads((Path(__file__).resolve().parent / "golden" / "descriptor_cases.json").read_text())
WORKED = CASES["worked_example"]


def encode_case(c) -> bytes:
    return Q.encode(c["fields"], fix_crc=c["fix_crc"])


# ------------------------------------------------------------------------------ oracle pinning
def test_layout_covers_512_bits_once():
    used = np.zeros(512, int)
    for hi, lo in Q.LAYOUT.values():
        used[lo:hi + 1] += 1
    assert (used == 1).all() and len(Q.LAYOUT) == 23


def test_worked_example_bytes_crc_and_codes():
    raw = Q.encode(WORKED["fields"])
    assert raw == bytes.fromhex(WORKED["desc_hex"])
    d = Q.decode(raw)
    assert (d["CRC32"], d["CTRL"], d["EPI"]) == (WORKED["crc"], WORKED["ctrl"], WORKED["epi"])
    assert raw[62:64] == b"\x55\xAA"


def worked_image() -> bytearray:
    rng = np.random.default_rng(2026)
    M, N, K = 2, 16, 32
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    W = rng.integers(-128, 128, (N, K), dtype=np.int8)
    S = (rng.uniform(0.5, 2.0, N) / 4096).astype(np.float32)
    B = rng.uniform(-8, 8, N).astype(np.float32)
    ddr = bytearray(WORKED["image"])
    ddr[0x100:0x100 + M * K] = A.tobytes()
    ddr[0x200:0x200 + N * K] = W.tobytes()
    ddr[0x600:0x600 + 4 * N] = S.astype("<f4").tobytes()
    ddr[0x700:0x700 + 4 * N] = B.astype("<f4").tobytes()
    q = WORKED["queue_addr"]
    ddr[q:q + 64] = bytes.fromhex(WORKED["desc_hex"])
    return ddr


def test_worked_example_runs_to_the_documented_bf16():
    m = Q.Machine(worked_image())
    st = m.run_queue(WORKED["queue_addr"], 1)
    assert st.done and st.op_idx == 1
    assert struct.unpack("<H", m.read(0x1002, 2))[0] == WORKED["y_elem01_bf16"]
    A = np.frombuffer(m.read(0x100, 64), np.int8).reshape(2, 32).astype(np.int64)
    W = np.frombuffer(m.read(0x200, 512), np.int8).reshape(16, 32).astype(np.int64)
    assert int(A[0] @ W[1]) == WORKED["acc01"]
    assert struct.unpack("<I", m.read(0x604, 4))[0] == WORKED["scale1_bits"]
    assert struct.unpack("<I", m.read(0x704, 4))[0] == WORKED["bias1_bits"]
    pre = F.fadd(F.fmul(F.i2f(np.int64(WORKED["acc01"])), np.frombuffer(m.read(0x604, 4), "<f4")),
                 np.frombuffer(m.read(0x704, 4), "<f4"))
    assert F.bits(pre)[0] == WORKED["pre_act01_bits"]


@pytest.mark.parametrize("i", range(len(CASES["cases"])))
def test_oracle_validation_matches_the_reference_tables(i):
    c = CASES["cases"][i]
    err = Q.validate(encode_case(c), 0, c["gemv_only"])[0]
    if err == Q.E_OK:
        err = Q.check(encode_case(c), c["image"], 0, c["gemv_only"])[0]
    assert err == c["expect"], (c["src"], c["fields"])


@pytest.mark.parametrize("seed", range(10))
def test_encode_decode_roundtrip_and_crc(seed):
    rng = np.random.default_rng(seed)
    f = {n: int(rng.integers(0, 1 << min(hi - lo + 1, 62))) for n, (hi, lo) in Q.LAYOUT.items() if n != "CRC32"}
    raw = Q.encode(f)
    d = Q.decode(raw)
    assert all(d[n] == v for n, v in f.items()) and Q.crc_ok(raw)


def test_crc_detects_every_single_bit_flip():
    raw = Q.encode({"MAGIC": Q.MAGIC, "VERSION": Q.VERSION, "OPCODE": Q.OP_GEMM, "VALID": 1})
    for byte in range(64):
        for bit in range(8):
            b = bytearray(raw)
            b[byte] ^= 1 << bit
            assert not Q.crc_ok(bytes(b))


def test_w4_segments_match_the_reference():
    """test_w4a16.py:219-226: the W and scale segments, no row-scale read, the fp32 row bytes."""
    f = dict(MAGIC=Q.MAGIC, VERSION=Q.VERSION, VALID=1, A_OFF=0x100, Y_OFF=0x4000, W_OFF=0x1000, M=3, N=32,
             OPCODE=Q.OP_GEMM, CTRL=Q.ctrl(Q.QM_GROUP, a_dtype=Q.DT_FP32, w_dtype=Q.DT_INT4), K=256,
             GROUP_SIZE=128, SCALE_OFF=0x400)
    d = Q.decode(Q.encode(f))
    reads, y = Q.segments(d)
    assert reads[1] == [(0x1000, 0x1000 + 32 * 128)]
    assert reads[2] == [(0x400, 0x400 + 32 * 2 * 2)]
    assert len(reads) == 3 and Q.strides(d)[2] == 4 * 256


# ------------------------------------------------------------------------------ the queue walk
GEMM = dict(MAGIC=Q.MAGIC, VERSION=Q.VERSION, OPCODE=Q.OP_GEMM, CTRL=Q.ctrl(Q.QM_TENSOR), EPI=Q.epi(),
            A_OFF=0x100, W_OFF=0x200, Y_OFF=0x800, SCALE_OFF=0x400, M=1, N=16, K=16, VALID=1)


def base_image() -> bytearray:
    ddr = bytearray(1 << 14)                                       # test_golden.py:73-82
    ddr[0x100:0x110] = bytes(range(16))
    ddr[0x200:0x300] = bytes([1]) * 256
    ddr[0x400:0x404] = struct.pack("<f", 1.0)
    return ddr


def run(ddr, *descs):
    mem = bytearray(ddr)
    for i, r in enumerate(descs):
        mem[0x2000 + 64 * i:0x2000 + 64 * (i + 1)] = r
    m = Q.Machine(mem)
    return m.run_queue(0x2000, len(descs)), m


def test_queue_stops_and_keeps_earlier_writes():
    """test_golden.py:134-138."""
    st, m = run(base_image(), Q.encode(GEMM), Q.encode({**GEMM, "MAGIC": 0}), Q.encode({**GEMM, "Y_OFF": 0xC00}))
    assert (st.err_code, st.op_idx) == (Q.E_MAGIC, 1)
    assert m.read(0x800, 64) != bytes(64) and m.read(0xC00, 64) == bytes(64)


def test_output_overlapping_input_is_refused():
    with pytest.raises(Q.ContractError):
        run(base_image(), Q.encode({**GEMM, "Y_OFF": 0x200}))


def test_gemm_result_is_the_hand_computed_sum():
    """W all ones, scale 1.0: y = sum(a) in every column (test_golden.py:160-162)."""
    st, m = run(base_image(), Q.encode(GEMM))
    assert st.done
    assert np.array_equal(np.frombuffer(m.read(0x800, 64), "<f4"), np.full(16, sum(range(16)), np.float32))


def test_row_quant_then_rowcol_gemm_chain():
    """ROW_QUANT writes int8 rows and scales that a QM_ROWCOL GEMM then reads (RAW), equal to the
    op-level oracle on the same inputs."""
    rng = np.random.default_rng(5)
    M, K, N = 3, 64, 32
    ddr = bytearray(1 << 15)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    W = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sc = rng.uniform(1e-3, 1e-2, N).astype(np.float32)
    ddr[0x1000:0x1000 + x.nbytes] = x.tobytes()
    ddr[0x2000:0x2000 + W.nbytes] = W.tobytes()
    ddr[0x3000:0x3000 + sc.nbytes] = sc.tobytes()
    quant = dict(MAGIC=Q.MAGIC, VERSION=Q.VERSION, VALID=1, OPCODE=Q.OP_ROW, CTRL=Q.ROW_QUANT,
                 EPI=Q.epi(out=Q.OUT_INT8), A_OFF=0x1000, Y_OFF=0x4000, SCALE_OFF=0x4800, M=M, N=K)
    gemm = dict(MAGIC=Q.MAGIC, VERSION=Q.VERSION, VALID=1, OPCODE=Q.OP_GEMM, CTRL=Q.ctrl(Q.QM_ROWCOL),
                EPI=Q.epi(), A_OFF=0x4000, W_OFF=0x2000, SCALE_OFF=0x3000, HDR_RSV=0x4800 // 16, Y_OFF=0x5000,
                M=M, N=N, K=K)
    for i, f in enumerate((quant, gemm)):
        ddr[0x6000 + 64 * i:0x6040 + 64 * i] = Q.encode(f)
    m = Q.Machine(ddr)
    assert m.run_queue(0x6000, 2).done
    q, s = F.quant_rows(x)
    assert m.read(0x4000, M * K) == q.tobytes() and m.read(0x4800, 4 * M) == s.tobytes()
    assert m.read(0x5000, 4 * M * N) == G.gemm_rowcol(q, s, W, sc).astype("<f4").tobytes()


def test_convolutions_stop_with_host_op():
    """A valid convolution is the one descriptor kind the executor leaves to the host: the queue
    stops there with host_op, keeping the earlier writes."""
    conv = dict(MAGIC=Q.MAGIC, VERSION=Q.VERSION, VALID=1, OPCODE=Q.OP_CONV, CTRL=Q.ctrl(Q.QM_CHANNEL),
                EPI=Q.epi(), A_OFF=0x100, W_OFF=0x200, SCALE_OFF=0x400, Y_OFF=0x3000, M=16, N=16, K=9 * 16,
                HDR_RSV=(4 << 12) | (3 << 8) | (3 << 4) | 1, GROUP_SIZE=4)
    assert Q.check(Q.encode(conv), 1 << 14)[0] == Q.E_OK
    st, m = run(base_image(), Q.encode(GEMM), Q.encode(conv), Q.encode(GEMM))
    assert (st.done, st.err_code, st.op_idx, st.host_op) == (False, Q.E_OK, 1, True)
    assert m.read(0x800, 64) != bytes(64)


def test_relu_descriptor_runs():
    """OP_RELU (golden.py:351-356): act on fp32 rows, converted to the output format."""
    ddr = base_image()
    x = np.linspace(-3, 3, 32, dtype=np.float32)
    ddr[0x1000:0x1080] = x.tobytes()
    relu = dict(MAGIC=Q.MAGIC, VERSION=Q.VERSION, OPCODE=Q.OP_RELU, M=2, N=16, VALID=1, EPI=Q.epi(1, out=Q.OUT_BF16),
                A_OFF=0x1000, Y_OFF=0x1200)
    st, m = run(ddr, Q.encode(relu))
    assert st.done
    assert m.read(0x1200, 64) == F.to_bf16_bits(F.relu_plain(x)).astype("<u2").tobytes()


# ------------------------------------------------------------------------------ the native checker
lib_needed = pytest.importorskip  # noqa: E305  (the library loads on a CPU host; no device call)


def native():
    from opentars_amd import queue as NQ
    return NQ


@pytest.mark.parametrize("i", range(len(CASES["cases"])))
def test_native_validation_matches_the_reference_tables(i):
    NQ = native()
    c = CASES["cases"][i]
    err, _ = NQ.check_descriptor(encode_case(c), c["image"], 0, c["gemv_only"])
    assert err == c["expect"], (c["src"], c["fields"])


def test_native_decode_and_crc_match_on_random_bytes():
    NQ = native()
    rng = np.random.default_rng(11)
    for _ in range(2000):
        raw = rng.integers(0, 256, 64, dtype=np.uint8).tobytes()
        d = Q.decode(raw)
        assert NQ.decode_descriptor(raw) == [d[n] for n in Q.FIELDS]
        z = bytearray(raw)
        z[4:8] = b"\0\0\0\0"
        assert NQ.descriptor_crc(raw) == zlib.crc32(bytes(z)) & 0xFFFFFFFF


def test_native_encode_matches_the_oracle():
    NQ = native()
    rng = np.random.default_rng(12)
    for _ in range(500):
        f = {n: int(rng.integers(0, 1 << min(hi - lo + 1, 63))) for n, (hi, lo) in Q.LAYOUT.items()}
        fix = bool(rng.integers(0, 2))
        assert NQ.encode_descriptor(f, fix) == Q.encode(f if not fix else {k: v for k, v in f.items() if k != "CRC32"},
                                                        fix_crc=fix)
    with pytest.raises(Exception):
        NQ.encode_descriptor({"M": 1 << 16})


def valid_templates() -> list[dict]:
    """One valid descriptor of each kind the contract knows."""
    b = dict(MAGIC=Q.MAGIC, VERSION=Q.VERSION, VALID=1, A_OFF=0x100, Y_OFF=0x800, W_OFF=0x1000, M=2, N=16)
    return [
        {**b, "OPCODE": Q.OP_GEMM, "CTRL": Q.ctrl(Q.QM_TENSOR), "K": 32, "SCALE_OFF": 0x400},
        {**b, "OPCODE": Q.OP_GEMM, "CTRL": Q.ctrl(Q.QM_CHANNEL, fusion=1), "EPI": Q.epi(4, Q.OUT_BF16, 1), "K": 48,
         "SCALE_OFF": 0x400, "BIAS_OFF": 0x500},
        {**b, "OPCODE": Q.OP_GEMM, "CTRL": Q.ctrl(Q.QM_ROWCOL), "K": 16, "SCALE_OFF": 0x400, "HDR_RSV": 0x50},
        {**b, "OPCODE": Q.OP_GEMM, "CTRL": Q.ctrl(Q.QM_GROUP, a_dtype=Q.DT_FP32, w_dtype=Q.DT_INT4), "K": 256,
         "GROUP_SIZE": 128, "SCALE_OFF": 0x400, "Y_OFF": 0x4000},
        {**b, "OPCODE": Q.OP_ROW, "CTRL": Q.ROW_QUANT, "EPI": Q.epi(out=Q.OUT_INT8), "SCALE_OFF": 0x400, "W_OFF": 0},
        {**b, "OPCODE": Q.OP_ROW, "CTRL": Q.ROW_RMSNORM, "SCALE_OFF": 0x400, "W_OFF": 0x3A83126F},
        {**b, "OPCODE": Q.OP_ROW, "CTRL": Q.ROW_SOFTMAX, "W_OFF": 0, "K": 3},
        {**b, "OPCODE": Q.OP_RELU, "EPI": Q.epi(1), "W_OFF": 0},
        {**b, "OPCODE": Q.OP_ELT, "CTRL": Q.ELT_MULADD, "EPI": Q.epi(bias=1), "BIAS_OFF": 0x800},
        {**b, "OPCODE": Q.OP_ELT, "HDR_RSV": Q.BM_COL, "W_OFF": 0x1004},
        {**b, "OPCODE": Q.OP_ROPE, "K": 32, "N": 32, "GROUP_SIZE": 2},
        {**b, "OPCODE": Q.OP_FDOT, "K": 16, "CTRL": 1, "HDR_RSV": Q.STATE_FP16},
        {**b, "OPCODE": Q.OP_CONV, "CTRL": Q.ctrl(Q.QM_CHANNEL), "K": 9 * 16, "M": 16,
         "HDR_RSV": (4 << 12) | (3 << 8) | (3 << 4) | 1, "GROUP_SIZE": 4, "SCALE_OFF": 0x400, "Y_OFF": 0x6000},
    ]


def mutate(f: dict, rng) -> dict:
    g = dict(f)
    for _ in range(int(rng.integers(1, 4))):
        name = Q.FIELDS[int(rng.integers(0, len(Q.FIELDS)))]
        if name == "CRC32":
            continue
        hi, lo = Q.LAYOUT[name]
        w = hi - lo + 1
        pick = int(rng.integers(0, 6))
        if pick == 0:
            g[name] = int(rng.integers(0, 1 << min(w, 62)))
        elif pick == 1:
            g[name] = g.get(name, 0) ^ (1 << int(rng.integers(0, min(w, 62))))
        elif pick == 2:
            g[name] = int(rng.choice([0, 1, 2, 3, 4, 8, 16, 24, 64, 128, 256, 4096, 4112])) & ((1 << w) - 1)
        elif pick == 3:
            g[name] = int(rng.integers(0, 0x8000)) & ~0xF & ((1 << w) - 1)
        elif pick == 4 and name in ("CTRL", "EPI", "HDR_RSV"):
            g[name] = int(rng.integers(0, 1 << min(w, 14)))
        else:
            g[name] = int(rng.integers(0, 1 << min(w, 8)))
    return g


@pytest.mark.parametrize("seed", range(4))
def test_native_validation_matches_the_oracle_on_mutations(seed):
    """Thousands of single- to triple-field mutations of valid descriptors of every kind: the same
    ERR_CODE (E_RANGE against a 64 KiB image included), the same overlap refusals, and the GPU
    flag exactly for the valid GEMM / ROW_QUANT descriptors."""
    NQ = native()
    rng = np.random.default_rng(100 + seed)
    temps = valid_templates()
    counts = np.zeros(9, int)
    for t in temps:
        err = Q.check(Q.encode(t), 1 << 16)[0]
        assert err == Q.E_OK, t
    for _ in range(4000):
        f = mutate(temps[int(rng.integers(0, len(temps)))], rng)
        raw = Q.encode(f, fix_crc=bool(rng.integers(0, 20)))
        try:
            want = Q.check(raw, 1 << 16, 0, seed == 3)
            want_err, want_gpu = want[0], want[0] == Q.E_OK and Q.gpu_kind(want[1])
        except Q.ContractError:
            with pytest.raises(Exception) as ei:
                NQ.check_descriptor(raw, 1 << 16, 0, seed == 3)
            assert "overlap" in str(ei.value), f
            continue
        got = NQ.check_descriptor(raw, 1 << 16, 0, seed == 3)
        assert got == (want_err, want_gpu), (f, got, want_err)
        counts[want_err] += 1
    assert (counts > 0).sum() >= 6, counts           # the fuzz reaches most error classes


@pytest.mark.parametrize("seed", range(3))
def test_overlap_of_strided_rows_matches_the_oracle(seed):
    """Outputs and inputs with row strides, packed into a few KiB so that their rows interleave,
    touch and partly overlap: the executor's closed-form row test refuses exactly the descriptors
    whose rows the oracle finds sharing a byte (golden.py:195-256, 440-448)."""
    NQ = native()
    rng = np.random.default_rng(700 + seed)
    refused = accepted = 0
    for _ in range(3000):
        kind = int(rng.integers(0, 4))
        M, N, K = int(rng.integers(1, 9)), 16 * int(rng.integers(1, 5)), 16 * int(rng.integers(1, 5))
        f = dict(MAGIC=Q.MAGIC, VERSION=Q.VERSION, VALID=1, M=M, N=N,
                 A_OFF=16 * int(rng.integers(0, 256)), W_OFF=16 * int(rng.integers(0, 256)),
                 Y_OFF=16 * int(rng.integers(0, 256)))
        if kind == 0:    # FDOT NT / NN with strided A, B and Y
            nn = int(rng.integers(0, 2))
            f.update(OPCODE=Q.OP_FDOT, CTRL=nn, K=K, LDA16=(4 * K) // 16 + int(rng.integers(0, 9)),
                     GROUP_SIZE=(4 * (N if nn else K)) // 16 + int(rng.integers(0, 9)),
                     LDY16=(4 * N) // 16 + int(rng.integers(0, 9)))
        elif kind == 1:  # ELT with a dense strided B, sometimes in place
            f.update(OPCODE=Q.OP_ELT, CTRL=int(rng.choice([Q.ELT_MUL, Q.ELT_ADD, Q.ELT_SUB])), LDA16=(4 * N) // 16 + int(rng.integers(0, 5)),
                     GROUP_SIZE=(4 * N) // 16 + int(rng.integers(0, 5)), LDY16=(4 * N) // 16 + int(rng.integers(0, 5)))
            if rng.integers(0, 4) == 0:
                f.update(Y_OFF=f["A_OFF"], LDY16=f["LDA16"])
        elif kind == 2:  # row function with strided rows and its gamma
            f.update(OPCODE=Q.OP_ROW, CTRL=Q.ROW_RMSNORM, SCALE_OFF=16 * int(rng.integers(0, 256)), W_OFF=0x3A83126F,
                     LDA16=(4 * N) // 16 + int(rng.integers(0, 9)), LDY16=(4 * N) // 16 + int(rng.integers(0, 9)))
        else:            # ROPE reading a table, strided rows
            f.update(OPCODE=Q.OP_ROPE, K=32, GROUP_SIZE=int(rng.integers(1, 4)), N=max(N, 32),
                     LDA16=(4 * max(N, 32)) // 16 + int(rng.integers(0, 9)),
                     LDY16=(4 * max(N, 32)) // 16 + int(rng.integers(0, 9)))
        raw = Q.encode(f)
        try:
            want = Q.check(raw, 1 << 16)
        except Q.ContractError:
            with pytest.raises(Exception) as ei:
                NQ.check_descriptor(raw, 1 << 16)
            assert "overlap" in str(ei.value), f
            refused += 1
            continue
        assert want[0] == Q.E_OK, f
        assert NQ.check_descriptor(raw, 1 << 16)[0] == Q.E_OK, f
        accepted += 1
    assert refused > 300 and accepted > 300, (refused, accepted)
