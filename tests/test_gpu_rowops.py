"""The row functions, RELU, ELT, RoPE and FDOT kernels against the oracle, bit for bit, through the
C ABI (opentars_amd.ops): the reference's own vectors, seeded rows with specials, every output
format, broadcast and in-place forms. Needs a gfx950 GPU."""
from __future__ import annotations

import zlib
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import golden as G
from oracle import numerics as F
from oracle import rowops as R
from opentars_amd import ops
from opentars_amd.contract import OUT_BF16, OUT_FP16, OUT_FP32, OUT_INT8
from opentars_amd.ops import ContractError, TarsError

pytestmark = pytest.mark.gpu

VEC = np.load(Path(__file__).resolve().parent / "golden" / "rowop_vectors.npz")
f32, u32 = np.float32, np.uint32
OUTS = [OUT_FP32, OUT_BF16, OUT_INT8]


def bits(a) -> np.ndarray:
    a = np.asarray(a)
    return a.view(u32) if a.dtype == f32 else a.view(np.uint16) if a.itemsize == 2 else a.view(np.uint8)


def same(got, want) -> bool:
    return np.array_equal(bits(got), bits(want))


def mismatch(got, want) -> str:
    g, w = bits(got), bits(want)
    bad = np.argwhere(g != w)
    return f"{len(bad)} differ; first at {tuple(bad[0])}: {g[tuple(bad[0])]:#x} vs {w[tuple(bad[0])]:#x}" if len(bad) else ""


def conv(y, out, osc=None):
    return G.convert(y, out, osc)


def rows_with_specials(seed, M, N, scale=1.0):
    rng = np.random.default_rng(seed)
    x = (rng.normal(0, 1, (M, N)) * scale * np.exp2(rng.integers(-6, 7, (M, 1)))).astype(f32)
    if M >= 6:
        x[1, N // 2] = np.inf
        x[2, N // 3] = np.nan
        x[3, :] = 0.0
        x[4, 1] = -np.inf
        x[5, :] = np.array([0x00000003], u32).view(f32)[0]
    return x


# ------------------------------------------------------------------------------ softmax
@pytest.mark.parametrize("name", ["sm_4x64", "sm_3x256", "sm_2x1024", "sm_5x16", "sm_edge"])
def test_softmax_reference_vectors(name):
    got = ops.softmax_rows(VEC[name + "_x"])
    assert same(got, VEC[name + "_y"]), mismatch(got, VEC[name + "_y"])


@pytest.mark.parametrize("name", ["smc", "smc_edge"])
def test_softmax_causal_reference_vectors(name):
    got = ops.softmax_rows_causal(VEC[name + "_x"], VEC[name + "_valid"])
    assert same(got, VEC[name + "_y"]), mismatch(got, VEC[name + "_y"])


@pytest.mark.parametrize("out", OUTS)
@pytest.mark.parametrize("M,N,k", [(1, 16, 0), (7, 80, 0), (16, 250, 0), (33, 512, 0), (16, 256, 5), (9, 96, 90),
                                   (3, 4096, 0), (2, 12288, 0), (2, 13000, 7000)])
def test_softmax_seeded(M, N, k, out):
    x = rows_with_specials(M * 7 + N, M, N, scale=4.0)
    osc = f32(3.0) if out == OUT_INT8 else None
    got = ops.softmax_rows(x, out=out, out_scale=osc, causal_k=k)
    want = R.softmax_rows_causal(x, np.minimum(N, k + np.arange(M))) if k else R.softmax_rows(x)
    want = conv(want, out, osc)
    assert same(got, want), mismatch(got, want)


# ------------------------------------------------------------------------------ norms
@pytest.mark.parametrize("name", ["n_3x1024", "n_2x2048", "n_4x128", "n_2x16", "n_edge"])
@pytest.mark.parametrize("fn", ["ln", "rms", "l2"])
def test_norm_reference_vectors(name, fn):
    f = {"ln": ops.layernorm_rows, "rms": ops.rmsnorm_rows, "l2": ops.l2norm_rows}[fn]
    x, g, b = VEC[name + "_x"], VEC[name + "_g"], VEC[name + "_b"]
    got = f(x, g, b, f32(1e-6))
    assert same(got, VEC[f"{name}_{fn}_eps6_y"]), mismatch(got, VEC[f"{name}_{fn}_eps6_y"])
    key, eps = (f"{name}_{fn}_eps0_y", f32(0.0)) if name == "n_edge" else (f"{name}_{fn}_eps5_nob_y", f32(1e-5))
    got = f(x, g, None, eps)
    assert same(got, VEC[key]), mismatch(got, VEC[key])


@pytest.mark.parametrize("fn", ["ln", "rms", "l2"])
@pytest.mark.parametrize("out", OUTS)
@pytest.mark.parametrize("M,N", [(1, 1024), (6, 48), (40, 2560), (2, 10), (2, 16400)])
def test_norms_seeded(fn, out, M, N):
    rng = np.random.default_rng(zlib.crc32(repr((fn, out, M, N)).encode()))
    x = rows_with_specials(M + N, M, N)
    g = rng.normal(1, 0.3, N).astype(f32)
    b = rng.normal(0, 0.1, N).astype(f32) if rng.integers(0, 2) else None
    eps = f32(rng.choice([1e-6, 1e-5, 0.0]))
    osc = f32(2.0) if out == OUT_INT8 else None
    op = {"ln": ops.layernorm_rows, "rms": ops.rmsnorm_rows, "l2": ops.l2norm_rows}[fn]
    ref = {"ln": R.layernorm_rows, "rms": R.rmsnorm_rows, "l2": R.l2norm_rows}[fn]
    got = op(x, g, b, eps, out=out, out_scale=osc)
    want = conv(ref(x, g, b, eps), out, osc)
    assert same(got, want), mismatch(got, want)


def test_rsqrt_through_l2norm_rows():
    """The device rsqrt on 4096 inputs spread over every exponent: L2Norm of [v, 0, ..., 0] rows
    with gamma = 1 and eps = t gives v * rsqrt(v*v + t); compared with the oracle."""
    rng = np.random.default_rng(5)
    M = 4096
    x = np.zeros((M, 16), f32)
    x[:, 0] = (np.exp2(rng.uniform(-60, 60, M)) * rng.choice([-1, 1], M)).astype(f32)
    for eps in (f32(0.0), f32(1e-30), f32(3.0)):
        got = ops.l2norm_rows(x, np.ones(16, f32), None, eps)
        want = R.l2norm_rows(x, np.ones(16, f32), None, eps)
        assert same(got, want), mismatch(got, want)


# ------------------------------------------------------------------------------ RELU / act
@pytest.mark.parametrize("act", range(1, 8))
@pytest.mark.parametrize("out", OUTS)
def test_relu_op(act, out):
    x = rows_with_specials(act * 3 + out, 7, 96, scale=8.0)
    osc = f32(5.0) if out == OUT_INT8 else None
    got = ops.relu(x, act, out=out, out_scale=osc)
    want = conv(F.act_fn(x, act), out, osc)
    assert same(got, want), mismatch(got, want)


@pytest.mark.parametrize("act", [3, 4, 5, 6, 7])
def test_exp_based_activations_over_a_bit_pattern_sweep(act):
    """GELU, SiLU, sigmoid, softplus and exp (every one built on exp_f) on every 1024th fp32 bit
    pattern (both signs, every exponent: zeros, subnormals, normals, infinities, NaNs), bit for bit
    against the oracle."""
    x = (np.arange(1 << 22, dtype=np.uint64) << np.uint64(10)).astype(np.uint32).view(f32).reshape(4096, 1024)
    got = ops.relu(x, act)
    want = F.act_fn(x, act)
    assert same(got, want), mismatch(got, want)


# ------------------------------------------------------------------------------ ELT
@pytest.mark.parametrize("op", [R.ELT_MUL, R.ELT_ADD, R.ELT_SUB, R.ELT_MULADD])
@pytest.mark.parametrize("bm", [R.BM_DENSE, R.BM_ROW, R.BM_COL, R.BM_SCALAR])
@pytest.mark.parametrize("a_fp16,a_row", [(False, False), (True, False), (False, True)])
def test_elt_modes(op, bm, a_fp16, a_row):
    rng = np.random.default_rng(zlib.crc32(repr((op, bm, a_fp16, a_row)).encode()))
    M, N = 9, 48
    a = rows_with_specials(op * 16 + bm, 1 if a_row else M, N)
    a_dev = a.astype(np.float16).view(np.uint16) if a_fp16 else a
    a_val = F.from_fp16_bits(a_dev) if a_fp16 else a
    bv = rng.normal(0, 2, {R.BM_DENSE: (M, N), R.BM_ROW: N, R.BM_COL: M, R.BM_SCALAR: 1}[bm]).astype(f32)
    act = int(rng.integers(0, 8))
    out = OUT_FP16 if op == R.ELT_MULADD and rng.integers(0, 2) else (OUT_FP32 if op == R.ELT_MULADD else
                                                                       int(rng.choice([0, 1, 2, 3])))
    c = rng.normal(0, 1, (M, N)).astype(f32) if op == R.ELT_MULADD else None
    c_dev = None if c is None else (c.astype(np.float16).view(np.uint16) if out == OUT_FP16 else c)
    c_val = None if c is None else (F.from_fp16_bits(c_dev) if out == OUT_FP16 else c)
    osc = f32(4.0) if out == OUT_INT8 else None
    got = ops.elt(op, a_dev, bv, bm, c_dev, act=act, out=out, out_scale=osc, a_fp16=a_fp16, a_row=a_row,
                  shape=(M, N))
    A = np.broadcast_to(a_val, (M, N))
    want = conv(R.elt(op, A, R.broadcast_b(bv, bm, M, N), c_val, act), out, osc)
    assert same(got, want), mismatch(got, want)


@pytest.mark.parametrize("fp16", [False, True])
def test_elt_in_place(fp16):
    """y = A (same buffer, golden.py:440-448) and y = C: the delta-rule update of tests/test_v04.py:124-137."""
    rng = np.random.default_rng(11)
    M, N = 16, 32
    S0 = rng.normal(0, 1, (M, N)).astype(f32)
    d = rng.normal(0, 1, (1, N)).astype(f32)
    k = rng.normal(0, 1, M).astype(f32)
    out = OUT_FP16 if fp16 else OUT_FP32
    S = torch.from_numpy(S0.astype(np.float16).view(np.int16) if fp16 else S0).cuda()
    Sval = F.from_fp16_bits(S0.astype(np.float16).view(np.uint16)) if fp16 else S0
    # S = S + d (x) k: A = d broadcast as a row, B = k per row (COL), C = Y = S
    ops.elt(R.ELT_MULADD, d, k, R.BM_COL, S, out=out, y=S, a_row=True, shape=(M, N))
    want = conv(R.elt(R.ELT_MULADD, np.broadcast_to(d, (M, N)), R.broadcast_b(k, R.BM_COL, M, N), Sval), out)
    # then S = S * k[0] in place through A
    ops.elt(R.ELT_MUL, S, k[:1], R.BM_SCALAR, out=out, y=S, a_fp16=fp16)
    wval = F.from_fp16_bits(want) if fp16 else want
    want2 = conv(R.elt(R.ELT_MUL, wval, R.broadcast_b(k[:1], R.BM_SCALAR, M, N)), out)
    got = S.cpu().numpy().view(np.uint16) if fp16 else S.cpu().numpy()
    assert same(got, want2), mismatch(got, want2)


def test_elt_partial_overlap_is_refused():
    a = torch.zeros((4, 16), dtype=torch.float32, device="cuda")
    with pytest.raises(ContractError):
        ops.elt(R.ELT_ADD, a, a, R.BM_DENSE, y=a[1:])


def test_fp16_output_rounding_and_specials():
    """OUT_FP16 (numerics.py:14-18) over the whole binary16 range: normal, subnormal, overflow to inf,
    ties, NaN -> 0x7E00, through an identity ELT (x * 1)."""
    rng = np.random.default_rng(3)
    x = np.concatenate([[65504, 65519.99, 65520, 65536, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -25,
                         2.0 ** -14, 2.0 ** -14 * (1 - 2.0 ** -11), 0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40,
                         1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11],
                        rng.normal(0, 1, 2000) * np.exp2(rng.integers(-30, 17, 2000))]).astype(f32)
    x = x[: len(x) // 16 * 16].reshape(-1, 16)
    got = ops.elt(R.ELT_MUL, x, np.ones(1, f32), R.BM_SCALAR, out=OUT_FP16)
    want = F.to_fp16_bits(R.elt(R.ELT_MUL, x, np.ones(x.shape, f32)))
    assert same(got, want), mismatch(got, want)


# ------------------------------------------------------------------------------ RoPE
def test_rope_reference_vectors():
    got = ops.rope_rows(VEC["rope_x"], VEC["rope_tab"], 2, 64)
    assert same(got, VEC["rope_y"]), mismatch(got, VEC["rope_y"])


@pytest.mark.parametrize("M,N,G,rot", [(1, 128, 1, 128), (16, 128, 2, 64), (40, 256, 8, 256), (7, 96, 3, 32)])
@pytest.mark.parametrize("out", OUTS)
def test_rope_seeded(M, N, G, rot, out):
    rng = np.random.default_rng(M * N + G)
    x = rows_with_specials(M + rot, M, N)
    rows = (M - 1) // G + 1
    fr = np.arange(rows, dtype=f32)[:, None] * rng.uniform(0.001, 1, rot // 2).astype(f32)[None, :]
    tab = np.concatenate([np.cos(fr), np.sin(fr)], 1).astype(f32)
    osc = f32(3.0) if out == OUT_INT8 else None
    got = ops.rope_rows(x, tab, G, rot, out=out, out_scale=osc)
    want = conv(R.rope_rows(x, tab, G, rot), out, osc)
    assert same(got, want), mismatch(got, want)


# ------------------------------------------------------------------------------ FDOT
def test_fdot_reference_vectors():
    got = ops.fdot_nt(VEC["fnt_a"], VEC["fnt_b"])
    assert same(got, VEC["fnt_y"]), mismatch(got, VEC["fnt_y"])
    got = ops.fdot_nn(VEC["fnn_a"], VEC["fnn_b"])
    assert same(got, VEC["fnn_y"]), mismatch(got, VEC["fnn_y"])


@pytest.mark.parametrize("M,N,K", [(1, 250, 128), (16, 40, 128), (3, 5, 64), (8, 300, 80), (2, 17, 16)])
@pytest.mark.parametrize("out", OUTS)
def test_fdot_nt_seeded(M, N, K, out):
    a = rows_with_specials(M * K, M, K)
    b = rows_with_specials(N * K + 1, N, K)
    osc = f32(2.0) if out == OUT_INT8 else None
    got = ops.fdot_nt(a, b, out=out, out_scale=osc)
    want = conv(R.fdot_nt(a, b), out, osc)
    assert same(got, want), mismatch(got, want)


@pytest.mark.parametrize("M,N,K", [(16, 128, 250), (1, 128, 1000), (4, 64, 13), (9, 300, 40)])
@pytest.mark.parametrize("b_fp16", [False, True])
def test_fdot_nn_seeded(M, N, K, b_fp16):
    rng = np.random.default_rng(M * N * K)
    a = rng.uniform(0, 0.1, (M, K)).astype(f32)
    b = rows_with_specials(K + N, K, N)
    bdev = b.astype(np.float16).view(np.uint16) if b_fp16 else b
    bval = F.from_fp16_bits(bdev) if b_fp16 else b
    got = ops.fdot_nn(a, bdev, b_fp16=b_fp16)
    want = R.fdot_nn(a, bval)
    assert same(got, want), mismatch(got, want)


def test_rowop_validation_errors():
    x = np.zeros((2, 16), f32)
    with pytest.raises(TarsError):
        ops.layernorm_rows(x, None, None, 1e-6)                    # a norm needs gamma
    with pytest.raises(TarsError):
        ops.rope_rows(x, np.zeros((2, 15), f32), 1, 15)            # odd rot
    with pytest.raises(TarsError):
        ops.elt(R.ELT_MULADD, x, x, R.BM_DENSE, x, out=OUT_BF16)   # MULADD adds in fp32 / fp16 only
