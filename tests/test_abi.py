"""The C ABI boundary on a CPU-only host: the library loads, exports what the header declares, and
rejects bad arguments with the contract's codes before it touches a device.

Every call below fails validation by construction; the placeholder addresses are never
dereferenced and no kernel is launched (a call that would pass validation is never made here)."""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

from opentars_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "opentars_amd.h"

P = 0x7F0000000000          # a 16-byte (and 128-byte) aligned placeholder address, never dereferenced
MB = 1 << 20


def declared() -> list[str]:
    return re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(tars_\w+)\s*\(", HEADER.read_text(), re.M)


def test_header_declares_the_entry_points():
    names = declared()
    assert set(names) == set(_lib.SIGNATURES), names


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in declared():
        assert hasattr(lib, name), name
    assert _lib.version().startswith("opentars_amd")


def status_codes_match_header():
    text = HEADER.read_text()
    return {m.group(1): int(m.group(2)) for m in re.finditer(r"#define TARS_(E_\w+|OK)\s+\(?(-?\d+)\)?", text)}


def test_status_codes_match_header():
    codes = status_codes_match_header()
    assert codes["OK"] == _lib.OK and codes["E_FIELD"] == _lib.E_FIELD and codes["E_ALIGN"] == _lib.E_ALIGN
    assert codes["E_RANGE"] == _lib.E_RANGE and codes["E_OVERLAP"] == _lib.E_OVERLAP
    assert codes["E_ARG"] == _lib.E_ARG and codes["E_DEVICE"] == _lib.E_DEVICE
    # the contract's own numbering (tars_mini/contract.py:108): E_FIELD 6, E_ALIGN 7, E_RANGE 8
    assert (_lib.E_FIELD, _lib.E_ALIGN, _lib.E_RANGE) == (-6, -7, -8)


def w8(**kw):
    """A tars_gemm_w8a8 call with a valid-looking layout overridden by kw (must fail validation)."""
    a = dict(A=P, lda=0, srow=P + 1 * MB, W=P + 2 * MB, scol=P + 3 * MB, bias=None,
             Y=P + 4 * MB, ldy=0, M=1, N=64, K=1024, act=0, out=0, osb=0)
    a.update(kw)
    a.setdefault("scol_count", a["N"])
    rc = _lib.lib().tars_gemm_w8a8(a["A"], a["lda"], a["srow"], a["W"], a["scol"], a["scol_count"], a["bias"],
                                   a["Y"], a["ldy"], a["M"], a["N"], a["K"], a["act"], a["out"], a["osb"], None)
    assert rc != _lib.OK, "test bug: this call would have launched"
    return rc


@pytest.mark.parametrize("kw,code", [
    (dict(act=8), _lib.E_FIELD),
    (dict(out=3), _lib.E_FIELD),                         # FP16 is not a GEMM output (golden.py:90)
    (dict(osb=0x40A00000), _lib.E_FIELD),                # OUT_SCALE without INT8 (golden.py:92)
    (dict(K=65536 + 16), _lib.E_FIELD),
    (dict(scol_count=1), _lib.E_FIELD),                  # a row scale needs per-channel scales
    (dict(N=40), _lib.E_ALIGN),
    (dict(K=1000), _lib.E_ALIGN),
    (dict(M=0), _lib.E_ALIGN),
    (dict(lda=1008), _lib.E_ALIGN),                      # stride must hold a row
    (dict(lda=1032), _lib.E_ALIGN),                      # and be a multiple of 16
    (dict(ldy=128), _lib.E_ALIGN),
    (dict(A=P + 4), _lib.E_ALIGN),
    (dict(srow=P + 1 * MB + 8), _lib.E_ALIGN),
    (dict(Y=P + 2 * MB), _lib.E_OVERLAP),                # output on the weights
    (dict(Y=P + 2 * MB + 64 * 1024 - 16), _lib.E_OVERLAP),
    (dict(Y=P - 128), _lib.E_OVERLAP),                   # output running into A
    (dict(W=None), _lib.E_ARG),
    (dict(act=9, N=40), _lib.E_FIELD),                   # E_FIELD is checked before E_ALIGN
])
def test_w8a8_validation(kw, code):
    assert w8(**kw) == code
    assert _lib.last_error()


def test_ksplit_validation():
    lib = _lib.lib()
    import ctypes
    ptrs = (ctypes.c_void_p * 2)(P + 2 * MB, P + 3 * MB)

    def call(ks, n=64, y=P + 6 * MB, nb=2):
        karr = (ctypes.c_int32 * 2)(*ks)
        rc = lib.tars_gemm_w8a8_ksplit(P, 0, P + MB, ptrs, karr, nb, P + 5 * MB, y, 0, 1, n, None)
        assert rc != _lib.OK
        return rc
    assert call([4096, 2810]) == _lib.E_ALIGN
    assert call([4096, 70000]) == _lib.E_FIELD
    assert call([4096, 2816], n=40) == _lib.E_ALIGN
    assert call([4096, 2816], nb=9) == _lib.E_ARG
    assert call([4096, 2816], y=P + 3 * MB) == _lib.E_OVERLAP


def test_w4_validation():
    lib = _lib.lib()

    def call(K=1536, N=64, W=P + 2 * MB, dt=4, act=0, out=0, osb=0, Y=P + 4 * MB, lda=0):
        rc = lib.tars_gemm_w4a16(P, lda, dt, W, P + 3 * MB, None, Y, 0, 1, N, K, act, out, osb, None)
        assert rc != _lib.OK
        return rc
    assert call(K=384) == _lib.E_ALIGN            # K % 256 (golden.py:145-147)
    assert call(K=128) == _lib.E_ALIGN
    assert call(K=8448) == _lib.E_ALIGN           # K <= 8192
    assert call(W=P + 2 * MB + 64) == _lib.E_ALIGN  # weights on a 128-byte boundary
    assert call(dt=1) == _lib.E_FIELD             # activations fp32 or bf16 only
    assert call(out=3) == _lib.E_FIELD
    assert call(lda=1024) == _lib.E_ALIGN         # 1024 bytes < one fp32 K=1536 row
    assert call(Y=P + 2 * MB + 512) == _lib.E_OVERLAP


def test_quant_and_align_validation():
    lib = _lib.lib()
    assert lib.tars_quant_rows(P, 0, P + MB, 0, P + 2 * MB, 1, 1000, None) == _lib.E_ALIGN
    assert lib.tars_quant_rows(P, 0, P + 16, 0, P + 2 * MB, 1, 1024, None) == _lib.E_OVERLAP
    assert lib.tars_quant_rows(P, 0, P + MB, 0, P + 2, 1, 1024, None) == _lib.E_ALIGN
    assert lib.tars_quant_rows(None, 0, P + MB, 0, P + 2 * MB, 1, 1024, None) == _lib.E_ARG
    assert lib.tars_align_w4(P, 0, 4, P + MB, 0, P + 2 * MB, 0, 1, 200, None) == _lib.E_ALIGN
    assert lib.tars_align_w4(P, 0, 2, P + MB, 0, P + 2 * MB, 0, 1, 256, None) == _lib.E_FIELD
    assert lib.tars_align_w4(P, 0, 4, P + 64, 0, P + 2 * MB, 0, 1, 256, None) == _lib.E_OVERLAP


def _gfx950_disassembly(tmp_path: Path) -> str:
    objdump = shutil.which("llvm-objdump") or "/opt/rocm/llvm/bin/llvm-objdump"
    if not Path(objdump).exists():
        pytest.skip("llvm-objdump not available")
    lib = tmp_path / "lib.so"
    shutil.copy(_lib.LIB_PATH, lib)
    subprocess.run([objdump, "--offloading", str(lib)], cwd=tmp_path, capture_output=True, check=True)
    objs = sorted(tmp_path.glob("lib.so.*gfx950"))
    assert objs, "no gfx950 code object in the library"
    return "\n".join(subprocess.run([objdump, "-d", "--mcpu=gfx950", str(o)], capture_output=True, text=True,
                                    check=True).stdout for o in objs)


_MAGIC_ADDEND = "0x4b400000"  # 1.5 * 2^23


def _fp32_fmas_other_than_rounding(dis: str) -> list:
    """Every fused fp32 multiply-add in `dis` except the W4A16 aligner's mantissa rounding, which is
    RN(x * p + 1.5 * 2^23) in `align_w4_kernel` and the W4A16 GEMM kernels (`gemv_w4a16_kernel`,
    `gemv_w4a16_kslice_kernel`, `gemm_w4a16_mfma_kernel`): `v_fmaak_f32` with that literal addend,
    or `v_fmac_f32` whose accumulator's last write is a move of that literal."""
    bad, fn, body = [], "", []

    def check(fn, body):
        rounding_ok = "align_w4" in fn or "w4a16" in fn
        for i, ins in enumerate(body):
            m = re.match(r"(v_(?:fma|fmac|mad|fmaak|fmamk|mac)_f32\w*)\s+(.*)", ins)
            if not m:
                continue
            ops = [o.strip() for o in m.group(2).split(",")]
            good = False
            if m.group(1) == "v_fmaak_f32":
                good = ops[-1] == _MAGIC_ADDEND
            elif m.group(1).startswith("v_fmac_f32"):
                for prev in reversed(body[:i]):
                    words = prev.split()
                    if len(words) > 1 and words[1].rstrip(",") == ops[0]:
                        good = prev.startswith("v_mov_b32") and prev.endswith(_MAGIC_ADDEND)
                        break
            if not (good and rounding_ok):
                bad.append((fn[:80], ins))

    for line in dis.splitlines():
        m = re.match(r"^[0-9a-f]+ <(.*)>:", line)
        if m:
            check(fn, body)
            fn, body = m.group(1), []
        elif line.startswith("\t"):
            body.append(line.split("//")[0].strip())
    check(fn, body)
    return bad


def test_fma_rule_accepts_only_the_rounding_form():
    head = "0000000000001000 <_ZN4tars12_GLOBAL__N_117gemv_w4a16_kernelILi8EE>:\n"
    other = "0000000000002000 <_ZN4tars12_GLOBAL__N_120quant_gemv_w8a8_kernelILi64EE>:\n"
    assert not _fp32_fmas_other_than_rounding(head + "\tv_fmaak_f32 v1, v2, v3, 0x4b400000\n")
    assert not _fp32_fmas_other_than_rounding(
        head + "\tv_mov_b32_e32 v5, 0x4b400000\n\tv_fmac_f32_e32 v5, v2, v3\n")
    assert _fp32_fmas_other_than_rounding(head + "\tv_fmaak_f32 v1, v2, v3, 0x3f800000\n")
    assert _fp32_fmas_other_than_rounding(
        head + "\tv_mov_b32_e32 v5, 0x4b400000\n\tv_add_f32_e32 v5, v5, v6\n\tv_fmac_f32_e32 v5, v2, v3\n")
    assert _fp32_fmas_other_than_rounding(head + "\tv_fma_f32 v1, v2, v3, v4\n")
    assert _fp32_fmas_other_than_rounding(other + "\tv_fmaak_f32 v1, v2, v3, 0x4b400000\n")


def test_codegen_has_no_fused_or_packed_fp32(tmp_path):
    """The epilogues must round every multiply and add on its own: the built gfx950 code holds no
    fused multiply-add (but the W4A16 aligner's mantissa rounding, whose exactness the device
    numerics tests prove) and no packed fp32 instruction, and no kernel spills to scratch."""
    dis = _gfx950_disassembly(tmp_path)
    bad = _fp32_fmas_other_than_rounding(dis)
    assert not bad, bad[:8]
    packed = re.findall(r"\bv_pk_(?:fma|mul|add)_f32\w*", dis)
    assert not packed, sorted(set(packed))
    assert "scratch_" not in dis
    assert "v_mfma_i32_16x16x64_i8" in dis and "v_dot4" in dis


def test_fused_validation():
    lib = _lib.lib()
    W8 = _lib.W8A8Out

    def call(outs, K=1024, q=None, s=None, x=P, lda=0):
        arr = (W8 * len(outs))(*outs)
        rc = lib.tars_quant_gemm_w8a8(x, lda, q, 0, s, 1, K, arr, len(outs), None)
        assert rc != _lib.OK
        return rc

    good = W8(P + 2 * MB, P + 3 * MB, None, P + 4 * MB, 0, 64, 0, 0, 0)
    assert call([good], K=1000) == _lib.E_ALIGN
    assert call([W8(P + 2 * MB, P + 3 * MB, None, P + 4 * MB, 0, 40, 0, 0, 0)]) == _lib.E_ALIGN
    assert call([W8(P + 2 * MB, P + 3 * MB, None, P + 4 * MB, 0, 64, 9, 0, 0)]) == _lib.E_FIELD
    assert call([good], q=P + 8 * MB) == _lib.E_ARG                      # q without s
    assert call([good, good]) == _lib.E_OVERLAP                           # two outputs on one buffer
    assert call([W8(P + 2 * MB, P + 3 * MB, None, P + 2 * MB + 64, 0, 64, 0, 0, 0)]) == _lib.E_OVERLAP
    assert call([good], q=P + 16, s=P + 8 * MB) == _lib.E_OVERLAP       # q over x
    assert call([good] * 5) == _lib.E_ARG
    assert ctypes_sizeof_desc() == 56


def ctypes_sizeof_desc() -> int:
    import ctypes
    return ctypes.sizeof(_lib.W8A8Out)


def test_rowop_validation():
    """tars_row_op / tars_elt / tars_rope / tars_relu / tars_fdot refuse bad arguments with the
    contract's codes before any launch (every call below is invalid)."""
    lib = _lib.lib()
    E = _lib
    X, Y, G = P, P + 8 * MB, P + 16 * MB
    row = lambda **k: lib.tars_row_op(*[k.get(n, d) for n, d in (
        ("x", X), ("lda", 0), ("fn", 0), ("gamma", None), ("beta", None), ("eps", 0), ("ck", 0), ("valid", None),
        ("y", Y), ("ldy", 0), ("out", 0), ("osc", 0), ("M", 2), ("N", 16))], None)
    assert row(fn=4) == E.E_FIELD                                   # ROW_QUANT has its own entry point
    assert row(fn=2) == E.E_ARG                                     # a norm needs gamma
    assert row(gamma=G) == E.E_FIELD                                # softmax takes no gamma
    assert row(fn=2, gamma=G, ck=3) == E.E_FIELD                    # only softmax is causal
    assert row(out=3) == E.E_FIELD                                  # FP16 is an ELT output only
    assert row(osc=0x40000000) == E.E_FIELD                         # out_scale without INT8
    assert row(ldy=60) == E.E_ALIGN                                 # a stride shorter than a row
    assert row(x=X + 2) == E.E_ALIGN                                # fp32 data 4-byte aligned
    assert row(y=X + 32) == E.E_OVERLAP                             # y over x
    assert row(x=None) == E.E_ARG
    elt = lambda **k: lib.tars_elt(*[k.get(n, d) for n, d in (
        ("A", X), ("lda", 0), ("a16", 0), ("arow", 0), ("B", G), ("ldb", 0), ("bm", 0), ("C", None), ("ldc", 0),
        ("op", 0), ("act", 0), ("Y", Y), ("ldy", 0), ("out", 0), ("osc", 0), ("M", 4), ("N", 16))], None)
    assert elt(op=4) == E.E_FIELD
    assert elt(bm=4) == E.E_FIELD
    assert elt(op=2) == E.E_ARG                                     # MULADD needs C
    assert elt(op=2, C=P + 24 * MB, out=1) == E.E_FIELD             # MULADD adds in fp32 / fp16 only
    assert elt(C=P + 24 * MB) == E.E_FIELD                          # C only for MULADD
    assert elt(Y=X, a16=1, out=0) == E.E_OVERLAP                    # in place needs the same format
    assert elt(Y=X + 16) == E.E_OVERLAP                             # a partial overlap
    assert elt(Y=G) == E.E_OVERLAP                                  # over B
    rope = lambda **k: lib.tars_rope(*[k.get(n, d) for n, d in (
        ("x", X), ("lda", 0), ("tab", G), ("G", 2), ("rot", 16), ("y", Y), ("ldy", 0), ("out", 0), ("osc", 0),
        ("M", 4), ("N", 16))], None)
    assert rope(rot=15) == E.E_ALIGN
    assert rope(rot=32) == E.E_ALIGN                                # rot past the row
    assert rope(G=0) == E.E_ALIGN
    assert rope(y=G + 8) == E.E_OVERLAP                             # over the table
    assert lib.tars_relu(X, 0, 9, Y, 0, 0, 0, 2, 16, None) == E.E_FIELD          # act code 9
    fdot = lambda **k: lib.tars_fdot(*[k.get(n, d) for n, d in (
        ("A", X), ("lda", 0), ("B", G), ("ldb", 0), ("nn", 0), ("b16", 0), ("Y", Y), ("ldy", 0), ("out", 0),
        ("osc", 0), ("M", 2), ("N", 16), ("K", 64))], None)
    assert fdot(b16=1) == E.E_FIELD                                 # fp16 B only in the NN form
    assert fdot(nn=2) == E.E_FIELD
    assert fdot(K=0) == E.E_ALIGN
    assert fdot(ldb=128) == E.E_ALIGN                               # NT rows of 64 fp32 are 256 bytes
    assert fdot(Y=G + 64) == E.E_OVERLAP


def test_embed_rows_validation():
    """tars_embed_rows refuses bad arguments before any launch (every call below is invalid)."""
    import ctypes
    lib = _lib.lib()
    T, D = P, P + 64 * MB

    def call(ids=(1, 2), **k):
        arr = (ctypes.c_int32 * max(len(ids), 1))(*ids)
        a = dict(table=T, ldt=0, rows=512, cols=256, n=len(ids), scaled=0, sb=0, dst=D, ldd=0)
        a.update(k)
        return lib.tars_embed_rows(a["table"], a["ldt"], a["rows"], a["cols"], arr, a["n"], a["scaled"], a["sb"],
                                   a["dst"], a["ldd"], None)
    assert call(table=None) == _lib.E_ARG
    assert call(scaled=2) == _lib.E_FIELD
    assert call(n=0) == _lib.E_ALIGN
    assert call(cols=0) == _lib.E_ALIGN
    assert call(ldt=256) == _lib.E_ALIGN                            # 256 bf16 are 512 bytes
    assert call(ldd=1000) == _lib.E_ALIGN                           # 256 fp32 are 1024 bytes
    assert call(ldd=1030) == _lib.E_ALIGN                           # not a multiple of 4
    assert call(dst=D + 2) == _lib.E_ALIGN
    assert call(ids=(1, 512)) == _lib.E_RANGE                       # past the table
    assert call(ids=(-1,)) == _lib.E_RANGE
    assert call(dst=T + 100 * 512) == _lib.E_OVERLAP                # rows into the table


def test_attention_validation():
    """tars_attention refuses bad arguments before any launch (every call below is invalid)."""
    import ctypes
    lib = _lib.lib()
    Qb, K, V, A, S = P, P + 64 * MB, P + 128 * MB, P + 192 * MB, P + 256 * MB

    def call(heads=4, kv=2, hd=128, nk=256, M=1, q=None, att=None, **k):
        grp = heads // kv
        arr = lambda vals: (ctypes.c_void_p * max(heads, 1))(*vals)
        qp = arr(q if q is not None else [Qb + 4 * h * hd for h in range(heads)])
        kp = arr([K + 4 * (h // grp) * hd for h in range(heads)])
        vp = arr([V + 4 * (h // grp) * hd for h in range(heads)])
        ap = arr(att if att is not None else [A + 4 * h * hd for h in range(heads)])
        a = dict(ldq=4 * heads * hd, ldk=4 * kv * hd, ldv=4 * kv * hd, v16=0, ldatt=4 * heads * hd, out=0, osc=0,
                 sc=S, ldsc=0, pr=S + MB, ldpr=0, causal=nk)
        a.update(k)
        return lib.tars_attention(qp, a["ldq"], kp, a["ldk"], vp, a["ldv"], a["v16"], ap, a["ldatt"], a["out"],
                                  a["osc"], a["sc"], a["ldsc"], a["pr"], a["ldpr"], heads, M, nk, hd, a["causal"], None)
    assert call(q=[None, Qb, Qb, Qb]) == _lib.E_ARG
    assert call(heads=0, kv=1) == _lib.E_ARG
    assert call(heads=33, kv=1) == _lib.E_ARG
    assert call(v16=2) == _lib.E_FIELD
    assert call(out=3) == _lib.E_FIELD                              # fp16 is no attention output
    assert call(osc=0x3F800000) == _lib.E_FIELD                     # a scale without INT8 output
    assert call(causal=-1) == _lib.E_FIELD
    assert call(M=0) == _lib.E_ALIGN
    assert call(hd=48) == _lib.E_ARG                                # head sizes 64, 128, 256
    assert call(nk=4096) == _lib.E_ARG                              # past 4080 keys
    assert call(ldk=4 * 128 + 4) == _lib.E_ALIGN                    # not a multiple of 16
    assert call(ldq=256) == _lib.E_ALIGN                            # shorter than a row
    assert call(sc=S + 8) == _lib.E_ALIGN
    assert call(att=[A + 4, A + 516, A + 1028, A + 1540]) == _lib.E_ALIGN
    assert call(att=[A, A, A + 1024, A + 1536]) == _lib.E_OVERLAP   # two heads' outputs
    assert call(att=[Qb + 4 * 128 * h for h in range(4)]) == _lib.E_OVERLAP   # over the q rows
    assert call(pr=V) == _lib.E_OVERLAP                             # over the V rows
    assert call(pr=S) == _lib.E_OVERLAP                             # the score and probability rows
