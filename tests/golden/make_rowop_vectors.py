"""Write tests/golden/rowop_vectors.npz: input/output vectors of the reference golden model's row,
rotary and fp32 dot-product functions whose exact bits no known-answer test or closed form pins.

rsqrt_f is a fixed seed-and-Newton sequence that the reference's tests bound only in ulps
(tests/test_golden.py:308-333); softmax (plain and causal) and the three norms compose exp_f,
recip_f, rsqrt_f, the 16-lane sum and 1/N in an order the reference's tests check only to a
tolerance (tests/test_v04.py:87-97) or through the model-level transformer comparisons. Their bits
therefore come from the reference itself: this script imports tars_mini from the reference
checkout (read-only, in the build container only) and records what it returns. fdot_nt/fdot_nn
and rope_rows are recorded too, as a second pin beside the reference tests' own restatements
(tests/test_v04.py:57-84). Nothing else is taken from it; the .npz holds data only and the GPU box
never runs this.

    python tests/golden/make_rowop_vectors.py [/path/to/reference]
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

REF = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
OUT = Path(__file__).resolve().parent / "rowop_vectors.npz"

F32 = np.float32


def special_f32() -> np.ndarray:
    b = [0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00000, 0x7F800001,
         0x00000001, 0x807FFFFF, 0x00800000, 0x80800000, 0x7F7FFFFF, 0xFF7FFFFF, 0x3F800000,
         0xBF800000, 0x3F7FFFFF, 0x3FFFFFFF, 0x40000000, 0x40800000, 0x3E800000, 0x7E800000,
         0x01000000, 0x00FFFFFF, 0x01800000]
    return np.array(b, np.uint32).view(F32)


def edge_rows(rng, n: int) -> np.ndarray:
    """Rows that exercise the specials: equal values, an infinity, a NaN, huge and tiny values,
    zeros, subnormals, one dominant element."""
    r = np.zeros((10, n), F32)
    r[0] = 3.0
    r[1] = rng.normal(0, 1, n)
    r[1, n // 3] = np.inf
    r[2] = rng.normal(0, 1, n)
    r[2, n // 2] = np.nan
    r[3] = rng.normal(0, 60, n)
    r[4] = np.array([0x00000001], np.uint32).view(F32)[0]
    r[5] = rng.normal(0, 1e-19, n)
    r[6] = rng.normal(0, 1, n)
    r[6, 1] = -np.inf
    r[7] = np.clip(rng.normal(0, 1e37, n), -3e38, 3e38)
    r[8] = rng.normal(0, 1, n)
    r[8, 0] = 95.0
    # r[9] stays all +0
    return r


def main() -> None:
    sys.path.insert(0, str(REF))
    from tars_mini import numerics as N      # the reference's numeric contract (read-only)

    rng = np.random.default_rng(20261202)
    out: dict[str, np.ndarray] = {}

    # rsqrt_f: every exponent (odd and even), both signs, random mantissas, powers of two, specials
    rb = (rng.integers(0, 256, 4000, dtype=np.uint32) << 23) | rng.integers(0, 1 << 23, 4000, dtype=np.uint32)
    rb[:1000] |= np.uint32(0x80000000)
    p2 = np.ldexp(1.0, np.arange(-126, 128)).astype(F32)
    xr = np.concatenate([rb.view(F32), p2, special_f32(), rng.uniform(0.25, 4.0, 1000).astype(F32),
                         rng.uniform(1e-6, 1e3, 1000).astype(F32)])
    out["rsqrt_x"], out["rsqrt_y"] = xr, N.rsqrt_f(xr)

    # softmax rows: random widths and scales, plus the edge rows
    for name, (m, n, sd) in {"sm_4x64": (4, 64, 1.0), "sm_3x256": (3, 256, 4.0), "sm_2x1024": (2, 1024, 10.0),
                             "sm_5x16": (5, 16, 0.1)}.items():
        x = rng.normal(0, sd, (m, n)).astype(F32)
        out[name + "_x"], out[name + "_y"] = x, N.softmax_rows(x)
    x = edge_rows(rng, 48)
    out["sm_edge_x"], out["sm_edge_y"] = x, N.softmax_rows(x)

    # causal softmax: valid lengths from 1 to N, one row per length class
    x = rng.normal(0, 2, (8, 80)).astype(F32)
    valid = np.array([1, 2, 15, 16, 17, 33, 79, 80])
    out["smc_x"], out["smc_valid"], out["smc_y"] = x, valid, N.softmax_rows_causal(x, valid)
    x = edge_rows(rng, 32)
    valid = np.array([1, 32, 20, 5, 32, 7, 2, 32, 16, 9])
    out["smc_edge_x"], out["smc_edge_valid"], out["smc_edge_y"] = x, valid, N.softmax_rows_causal(x, valid)

    # the norms: hidden widths, with and without beta, several eps, plus edge rows
    for name, (m, n) in {"n_3x1024": (3, 1024), "n_2x2048": (2, 2048), "n_4x128": (4, 128), "n_2x16": (2, 16)}.items():
        x = rng.normal(0, 1.5, (m, n)).astype(F32)
        g = rng.normal(1, 0.2, n).astype(F32)
        b = rng.normal(0, 0.1, n).astype(F32)
        out[name + "_x"], out[name + "_g"], out[name + "_b"] = x, g, b
        for fn, f in (("ln", N.layernorm_rows), ("rms", N.rmsnorm_rows), ("l2", N.l2norm_rows)):
            out[f"{name}_{fn}_eps6_y"] = f(x, g, b, F32(1e-6))
            out[f"{name}_{fn}_eps5_nob_y"] = f(x, g, None, F32(1e-5))
    x = edge_rows(rng, 64)
    g = rng.normal(1, 0.2, 64).astype(F32)
    b = rng.normal(0, 0.1, 64).astype(F32)
    out["n_edge_x"], out["n_edge_g"], out["n_edge_b"] = x, g, b
    for fn, f in (("ln", N.layernorm_rows), ("rms", N.rmsnorm_rows), ("l2", N.l2norm_rows)):
        out[f"n_edge_{fn}_eps6_y"] = f(x, g, b, F32(1e-6))
        out[f"n_edge_{fn}_eps0_y"] = f(x, g, None, F32(0.0))

    # fp32 dot products at attention shapes
    a = rng.normal(0, 1, (3, 128)).astype(F32)
    bt = rng.normal(0, 1, (40, 128)).astype(F32)
    out["fnt_a"], out["fnt_b"], out["fnt_y"] = a, bt, N.fdot_nt(a, bt)
    p = rng.uniform(0, 0.1, (2, 40)).astype(F32)
    v = rng.normal(0, 1, (40, 128)).astype(F32)
    out["fnn_a"], out["fnn_b"], out["fnn_y"] = p, v, N.fdot_nn(p, v)

    # rotary embedding: 2 rows per position, 64 of 128 elements rotated
    x = rng.normal(0, 1, (6, 128)).astype(F32)
    pos = np.arange(3, dtype=F32)
    inv = (1.0 / (1e6 ** (np.arange(0, 64, 2, dtype=F32) / F32(64)))).astype(F32)
    fr = (pos[:, None] * inv[None, :]).astype(F32)
    tab = np.concatenate([np.cos(fr), np.sin(fr)], 1).astype(F32)
    out["rope_x"], out["rope_tab"], out["rope_y"] = x, tab, N.rope_rows(x, tab, 2, 64)

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({len(out)} arrays)")


if __name__ == "__main__":
    main()
