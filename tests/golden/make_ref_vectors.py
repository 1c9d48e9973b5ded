"""Write tests/golden/ref_vectors.npz: input/output vectors of the reference golden model's
functions whose exact bits no known-answer test or closed form pins.

Those are the fixed-sequence primitives (recip_f, exp_f and the activations built from them),
quant_rows, whose 127 * recip(amax) decides every q8 rounding, and the W4A16 GEMM, whose four
fp32 banks fix the order of the group sums. The reference's own tests bound the primitives only in
ulps (tests/test_golden.py:308-359, tests/test_v04.py:34-54) and check the W4 bank order only with
a restatement of it (tests/test_w4a16.py:149-162), so their bits come from the reference itself:
this script imports tars_mini from the reference checkout (read-only, in the build container only)
and records what it returns. Nothing else is taken from it. The .npz holds data only and is what the tests read; the GPU box never runs this.

    python tests/golden/make_ref_vectors.py [/path/to/reference]
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

REF = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
OUT = Path(__file__).resolve().parent / "ref_vectors.npz"

F32 = np.float32


def special_f32() -> np.ndarray:
    b = [0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00000, 0x7F800001,
         0x00000001, 0x807FFFFF, 0x00800000, 0x80800000, 0x7F7FFFFF, 0xFF7FFFFF, 0x3F800000,
         0xBF800000, 0x3F7FFFFF, 0x3FFFFFFF, 0x7E800000, 0x7F000000, 0x7EFFFFFF, 0x01000000,
         0x00FFFFFF, 0x42FE0000, 0x3C010204]
    return np.array(b, np.uint32).view(F32)


def main() -> None:
    sys.path.insert(0, str(REF))
    from tars_mini import numerics as N      # the reference's numeric contract (read-only)

    rng = np.random.default_rng(20261201)
    out: dict[str, np.ndarray] = {}

    # recip_f: every exponent, both signs, random mantissas, powers of two, specials
    rb = (rng.integers(0, 256, 3000, dtype=np.uint32) << 23) | rng.integers(0, 1 << 23, 3000, dtype=np.uint32)
    rb |= rng.integers(0, 2, 3000, dtype=np.uint32) << 31
    p2 = np.ldexp(1.0, np.arange(-126, 128)).astype(F32)
    xr = np.concatenate([rb.view(F32), p2, -p2, special_f32(),
                         rng.uniform(0.5, 200.0, 1000).astype(F32)])
    out["recip_x"], out["recip_y"] = xr, N.recip_f(xr)

    # exp_f: the working range, the clamp edges, rint ties of x*log2e, specials
    xe = np.concatenate([rng.uniform(-110, 95, 3000), rng.uniform(-2, 2, 1000),
                         np.arange(-210, 210) * 0.5 / 1.4426950408889634,
                         [88.99, 89.0, 89.01, -103.99, -104.0, -104.01]]).astype(F32)
    xe = np.concatenate([xe, special_f32()])
    out["exp_x"], out["exp_y"] = xe, N.exp_f(xe)

    # activations: silu, gelu, sigmoid, softplus over their interesting ranges
    xa = np.concatenate([rng.uniform(-30, 30, 3000), rng.uniform(-3, 3, 1500),
                         [19.99, 20.0, 20.01, 1e20, -1e20, 1e5, -1e5, 1e-30, -1e-30]]).astype(F32)
    xa = np.concatenate([xa, special_f32()])
    out["act_x"] = xa
    for code in range(8):
        out[f"act{code}_y"] = N.act_fn(xa, code)

    # quant_rows: seeded N(0,1) rows at the path's widths, plus edge rows
    for name, (m, k) in {"qr_1x1024": (1, 1024), "qr_4x1024": (4, 1024), "qr_4x3072": (4, 3072),
                         "qr_1x6912": (1, 6912), "qr_3x2048": (3, 2048)}.items():
        x = rng.normal(0, 1, (m, k)).astype(F32)
        q, s = N.quant_rows(x)
        out[name + "_x"], out[name + "_q"], out[name + "_s"] = x, q, s
    edge = np.zeros((12, 64), F32)
    edge[1, 3] = np.inf                                   # inf row: inv = 0
    edge[2, 5] = np.nan                                   # NaN row: q = 0, s = NaN
    edge[3, :] = np.array([0x00000001], np.uint32).view(F32)[0]   # all subnormal -> zero row
    edge[4, :] = rng.normal(0, 1, 64)
    edge[4, 7] = -np.inf
    edge[5, :] = np.arange(64) - 31.5                     # amax 32.5 over a ramp
    edge[6, :] = (np.arange(64) % 2 * 2 - 1) * 127.0      # +-127: inv close to 1
    edge[7, :] = rng.normal(0, 1e-30, 64)                 # tiny values, some subnormal
    edge[8, :] = np.clip(rng.normal(0, 1e38, 64), -3.4e38, 3.4e38)   # near overflow
    edge[9, :] = np.linspace(-1, 1, 64)
    edge[10, :] = (np.arange(64) - 32) * 0.5 * 127.0 / 32.0   # halves at amax 127 -> ties
    edge[11, :] = -0.0
    q, s = N.quant_rows(edge)
    out["qr_edge_x"], out["qr_edge_q"], out["qr_edge_s"] = edge, q, s

    # W4A16 GEMMs run through the reference's golden Machine on descriptor images
    from tars_mini import contract as C
    from tars_mini.golden import Machine
    w4_cases = [  # (M, N, K, bf16 activations, bias, act, out)
        (1, 32, 256, False, False, 0, C.OUT_FP32),
        (2, 48, 1024, False, True, C.ACT_SILU, C.OUT_FP32),
        (3, 16, 768, True, True, C.ACT_GELU, C.OUT_BF16),
        (1, 16, 6144, False, False, 0, C.OUT_FP32),
        (1, 16, 512, False, False, 0, C.OUT_FP32),          # inf / huge / subnormal planted below
        (1, 16, 8192, False, True, C.ACT_RELU, C.OUT_INT8),
        (1, 64, 1536, False, False, 0, C.OUT_FP32),
        (2, 16, 512, True, False, 0, C.OUT_FP32),           # a NaN group in row 0 only
    ]
    for i, (m, n, k, half, bias, act, fmt) in enumerate(w4_cases):
        x = (rng.normal(0, 1, (m, k // 128, 128)) * np.exp2(rng.integers(-20, 20, (m, k // 128, 1)))).reshape(m, k)
        x = x.astype(F32)
        if i == 4:
            x[0, 3] = np.inf                                  # group 0: +inf with finite values
            x[0, 260:262] = [np.inf, -np.inf]                  # group 2: both infinities
            x[0, 130] = 3e38                                   # group 1: near the top exponent
            x[0, 400:404] = np.array([1, 0x00400000, 0x80000001, 0x00800000], np.uint32).view(F32)
            x[0, 384:400] = 0.0                                # group 3: zeros, subnormals, one normal
            x[0, 404:512] = 0.0
        if i == 7:
            x[0, 140] = np.nan
        nib = rng.integers(-8, 8, (n, k))
        wp = ((nib[:, 0::2] & 15) | ((nib[:, 1::2] & 15) << 4)).astype(np.uint8)
        ws = rng.uniform(1e-3, 1e-2, (n, k // 128)).astype(np.float16).view(np.uint16)
        if i == 4:
            ws[0, 0], ws[1, 1], ws[2, 2], ws[3, 3] = 0x0001, 0x7C00, 0x7E01, 0x8000
        b = rng.normal(0, 2, n).astype(F32)
        if half:
            xin = N.to_bf16_bits(x)
            abytes = xin.astype("<u2").tobytes()
        else:
            xin = x
            abytes = x.astype("<f4").tobytes()
        a_off, w_off = 0x1000, 0x1000 + ((len(abytes) + 127) // 128) * 128
        s_off = w_off + wp.size
        b_off = s_off + ((ws.size * 2 + 15) // 16) * 16
        y_off = b_off + 4 * n
        y_bytes = m * n * {C.OUT_FP32: 4, C.OUT_BF16: 2, C.OUT_INT8: 1}[fmt]
        qa = ((y_off + y_bytes + 63) // 64) * 64
        ddr = bytearray(qa + 64)
        ddr[a_off:a_off + len(abytes)] = abytes
        ddr[w_off:w_off + wp.size] = wp.tobytes()
        ddr[s_off:s_off + 2 * ws.size] = ws.astype("<u2").tobytes()
        ddr[b_off:b_off + 4 * n] = b.astype("<f4").tobytes()
        f = dict(MAGIC=C.MAGIC, VERSION=C.VERSION, VALID=1, OPCODE=C.OP_GEMM, M=m, N=n, K=k,
                 CTRL=C.ctrl(C.QM_GROUP, a_dtype=C.DT_BF16 if half else C.DT_FP32, w_dtype=C.DT_INT4,
                             fusion=int(act != 0)),
                 EPI=C.epi(act, fmt, int(bias)), GROUP_SIZE=C.W4_GROUP, A_OFF=a_off, W_OFF=w_off,
                 SCALE_OFF=s_off, BIAS_OFF=b_off if bias else 0, Y_OFF=y_off)
        if fmt == C.OUT_INT8:
            f["OUT_SCALE"] = C.f32_bits(40.0)
        ddr[qa:qa + 64] = C.encode(f)
        mach = Machine(ddr)
        st = mach.run_queue(qa, 1)
        assert st.done, st
        y = np.frombuffer(mach.read(y_off, y_bytes), np.uint8).copy()
        key = f"w4_{i}"
        out[key + "_x"], out[key + "_wp"], out[key + "_ws"] = xin, wp, ws
        out[key + "_bias"] = b if bias else np.zeros(0, F32)
        out[key + "_meta"] = np.array([m, n, k, int(half), int(bias), act, fmt, C.f32_bits(40.0)], np.int64)
        out[key + "_y"] = y

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
