"""Bit-exact parity of the HIP path (through the C ABI) with the CPU oracle and with the vectors the
reference golden model wrote itself. Needs a gfx950 GPU."""
from __future__ import annotations

import zlib
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import golden as G
from oracle import numerics as F
from opentars_amd import ops
from opentars_amd.contract import (ACT_GELU, ACT_NONE, ACT_RELU, ACT_SILU, ACT_SOFTPLUS, OUT_BF16, OUT_FP32,
                                   OUT_INT8)

pytestmark = pytest.mark.gpu

VEC = np.load(Path(__file__).resolve().parent / "golden" / "ref_vectors.npz")
f32 = np.float32


def cuda(a) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def same(a, b) -> bool:
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and a.tobytes() == b.tobytes()


def mismatch(a, b) -> str:
    a, b = np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8)
    if a.shape != b.shape:
        return f"shape {a.shape} vs {b.shape}"
    idx = np.nonzero(a != b)[0]
    return f"{idx.size} differing bytes, first at {idx[:8].tolist()}"


def w8_inputs(seed: int, M: int, N: int, K: int):
    """Seeded C1-style operands: int8 weights in [-127, 127], per-channel scales in [1e-3, 1e-2],
    N(0,1) activations quantized per token by the oracle."""
    rng = np.random.default_rng(seed)
    W = rng.integers(-127, 128, (N, K), dtype=np.int8)
    scol = rng.uniform(1e-3, 1e-2, N).astype(f32)
    x = rng.normal(0, 1, (M, K)).astype(f32)
    q, s = F.quant_rows(x)
    return x, q, s, W, scol, rng


def oracle_rowcol_blocked(q, s, W, scol, rows: int = 16384, **kw):
    """The oracle on row blocks of W (each output element is independent; bounds host memory)."""
    return np.concatenate([G.gemm_rowcol(q, s, W[i:i + rows], scol[i:i + rows] if scol.size > 1 else scol,
                                         **({**kw, "bias": kw["bias"][i:i + rows]} if kw.get("bias") is not None else kw))
                           for i in range(0, W.shape[0], rows)], axis=1)


# ------------------------------------------------------------------------------ quant_rows
@pytest.mark.parametrize("name", ["qr_1x1024", "qr_4x1024", "qr_4x3072", "qr_1x6912", "qr_3x2048", "qr_edge"])
def test_quant_rows_reference_vectors(name):
    x = VEC[name + "_x"]
    q, s = ops.quant_rows(cuda(x))
    assert same(host(q), VEC[name + "_q"]), mismatch(host(q), VEC[name + "_q"])
    assert same(host(s), VEC[name + "_s"])


@pytest.mark.parametrize("M,K", [(1, 16), (1, 1024), (1, 6912), (4, 3072), (256, 1024), (7, 65520), (3, 4112)])
def test_quant_rows_seeded(M, K):
    rng = np.random.default_rng(M * 100003 + K)
    x = (rng.normal(0, 1, (M, K)) * np.exp2(rng.integers(-60, 60, (M, 1)))).astype(f32)
    x[0, K // 2] = 0.0
    q, s = ops.quant_rows(cuda(x))
    wq, ws = F.quant_rows(x)
    assert same(host(q), wq) and same(host(s), ws)


def test_quant_rows_strided_rows_and_gaps():
    rng = np.random.default_rng(9)
    M, K, pad = 5, 1024, 64
    big = cuda(rng.normal(0, 1, (M, K + pad)).astype(f32))
    x = big[:, :K]
    qbuf = torch.full((M, K + 48), 99, dtype=torch.int8, device="cuda")
    q = qbuf[:, :K]
    s = torch.empty(M, dtype=torch.float32, device="cuda")
    ops.quant_rows(x, q=q, s=s)
    wq, ws = F.quant_rows(host(x).copy())
    assert same(host(q).copy(), wq) and same(host(s), ws)
    assert (host(qbuf)[:, K:] == 99).all()


# ------------------------------------------------------------------------------ W8A8 GEMV (M = 1)
@pytest.mark.parametrize("seed", range(5))
def test_c1_gemv_qwen3_gate_proj(seed):
    """Config 1: M=1, K=1024, N=3072, bit-exact."""
    x, q, s, W, scol, _ = w8_inputs(seed, 1, 3072, 1024)
    qg, sg = ops.quant_rows(cuda(x))
    assert same(host(qg), q) and same(host(sg), s)
    y = ops.gemm_rowcol(qg, sg, cuda(W), cuda(scol))
    want = G.gemm_rowcol(q, s, W, scol)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("K", [16, 32, 48, 112, 496, 784, 1024, 1040, 2048, 2816, 3072, 3456, 4096, 4112, 6912,
                               8192, 9216, 20000])
def test_gemv_every_k_shape(K):
    x, q, s, W, scol, _ = w8_inputs(K, 1, 96, K)
    y = ops.gemm_rowcol(cuda(q), cuda(s), cuda(W), cuda(scol))
    assert same(host(y), G.gemm_rowcol(q, s, W, scol))


@pytest.mark.parametrize("path,M", [("gemv", 1), ("gemv", 3), ("mfma", 3)])
@pytest.mark.parametrize("qm", ["tensor", "channel", "rowcol"])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("act,out", [(ACT_NONE, OUT_FP32), (ACT_RELU, OUT_INT8), (ACT_SILU, OUT_BF16),
                                     (ACT_SOFTPLUS, OUT_INT8), (ACT_GELU, OUT_FP32)])
def test_epilogue_matrix(path, M, qm, bias, act, out):
    """Every scale mode x bias x activation/format (the reference's GEMV test grid), with a huge
    scale (inf products), a zero activation chunk, and random int8 including -128; the GEMV family
    at M = 1 and with several activation rows per block (M = 3), and the MFMA family."""
    rng = np.random.default_rng(zlib.crc32(repr((path, M, qm, bias, act, out)).encode()))
    N, K = 48, 16 * int(rng.integers(1, 40))
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    A[:, 16:32] = 0
    W = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sc = rng.uniform(1e-4, 3e-2, N).astype(f32)
    sc[N // 2] = 3e30
    if qm == "tensor":
        sc = sc[:1]
    srow = rng.uniform(0.1, 2.0, M).astype(f32) if qm == "rowcol" else None
    b = rng.normal(0, 2, N).astype(f32) if bias else None
    osc = f32(5.0) if out == OUT_INT8 else None
    prev = ops.set_w8a8_path(path)
    try:
        y = ops.gemm_rowcol(cuda(A), None if srow is None else cuda(srow), cuda(W), cuda(sc),
                            None if b is None else cuda(b), act=act, out=out, out_scale=osc)
    finally:
        ops.set_w8a8_path(prev)
    want = G.gemm_rowcol(A, srow, W, sc, b, act=act, out=out, out_scale=osc)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("M,K,N", [(3, 512, 48), (11, 2304, 80)])
@pytest.mark.parametrize("qm", ["tensor", "channel", "rowcol"])
@pytest.mark.parametrize("act,out", [(ACT_NONE, OUT_FP32), (ACT_RELU, OUT_INT8), (ACT_SILU, OUT_BF16),
                                     (ACT_SOFTPLUS, OUT_INT8), (ACT_GELU, OUT_FP32)])
def test_epilogue_matrix_chunk_rows(M, K, N, qm, act, out):
    """The LDS-staged chunk-row MFMA kernel (M <= 16, K whole 256-byte blocks; 4 waves at K=512, 8 at
    K=2304) through every scale mode and output format with a bias, a huge scale and int8 -128."""
    rng = np.random.default_rng(zlib.crc32(repr((M, K, N, qm, act, out, "chunk")).encode()))
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    W = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sc = rng.uniform(1e-4, 3e-2, N).astype(f32)
    sc[N // 2] = 3e30
    if qm == "tensor":
        sc = sc[:1]
    srow = rng.uniform(0.1, 2.0, M).astype(f32) if qm == "rowcol" else None
    b = rng.normal(0, 2, N).astype(f32)
    osc = f32(5.0) if out == OUT_INT8 else None
    prev = ops.set_w8a8_path("mfma")
    try:
        y = ops.gemm_rowcol(cuda(A), None if srow is None else cuda(srow), cuda(W), cuda(sc), cuda(b),
                            act=act, out=out, out_scale=osc)
    finally:
        ops.set_w8a8_path(prev)
    want = G.gemm_rowcol(A, srow, W, sc, b, act=act, out=out, out_scale=osc)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("M", [1, 2, 4, 5, 8, 13, 16])
@pytest.mark.parametrize("K,N", [(256, 3072), (1024, 3072), (3072, 1024), (6912, 1152), (2560, 1040)])
def test_mfma_chunk_rows(M, K, N):
    """The chunk-row MFMA kernel at every row count and at K from one 256-byte block to 27 (waves
    with no block, one, two and several batches), the plain epilogue, on strided A and Y rows
    (the gaps left as they were) for odd M."""
    x, q, s, W, scol, rng = w8_inputs(M * 131 + K + N, M, N, K)
    strided = M % 2 == 1
    abig = cuda(np.concatenate([q, np.zeros((M, 256), np.int8)], axis=1)) if strided else cuda(q)
    ybig = torch.full((M, N + 20 if strided else N), -7.0, dtype=torch.float32, device="cuda")
    prev = ops.set_w8a8_path("mfma")
    try:
        ops.gemm_rowcol(abig[:, :K], cuda(s), cuda(W), cuda(scol), y=ybig[:, :N])
    finally:
        ops.set_w8a8_path(prev)
    yb, want = host(ybig), G.gemm_rowcol(q, s, W, scol)
    assert same(yb[:, :N].copy(), want), mismatch(yb[:, :N].copy(), want)
    assert (yb[:, N:] == -7.0).all()


@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("K", [128, 256, 512])
@pytest.mark.parametrize("N", [80, 1040, 4096, 32768])
def test_gemv_short_rows(M, K, N):
    """GEMV rows of at most 32 chunks (8, 16 or 32 lanes per row) at 1, 2, 4 and 8 rows per lane
    group, as the rows-per-wave rule picks them by N, bias and SiLU: bit-exact against the oracle."""
    x, q, s, W, scol, rng = w8_inputs(M * 1009 + K + N, M, N, K)
    b = rng.normal(0, 1, N).astype(f32)
    prev = ops.set_w8a8_path("gemv")
    try:
        y = ops.gemm_rowcol(cuda(q), cuda(s), cuda(W), cuda(scol), cuda(b), act=ACT_SILU)
    finally:
        ops.set_w8a8_path(prev)
    want = G.gemm_rowcol(q, s, W, scol, b, act=ACT_SILU)
    assert same(host(y), want), mismatch(host(y), want)


def test_gemv_nan_from_inf_scale_is_canonical():
    A = np.zeros((1, 16), np.int8)
    W = np.ones((16, 16), np.int8)
    y = host(ops.gemm_rowcol(cuda(A), None, cuda(W), cuda(np.array([np.inf], f32))))
    assert (y.view(np.uint32) == 0x7FC00000).all()


def test_worked_example_on_gpu():
    """The contract document's fused example (tests/test_contract.py:47-84): element (0, 1) is bf16 0x3F16."""
    rng = np.random.default_rng(2026)
    A = rng.integers(-128, 128, (2, 32), dtype=np.int8)
    W = rng.integers(-128, 128, (16, 32), dtype=np.int8)
    S = (rng.uniform(0.5, 2.0, 16) / 4096).astype(f32)
    B = rng.uniform(-8, 8, 16).astype(f32)
    for path in ("gemv", "mfma"):
        prev = ops.set_w8a8_path(path)
        try:
            y = host(ops.gemm_rowcol(cuda(A), None, cuda(W), cuda(S), cuda(B), act=ACT_RELU, out=OUT_BF16))
        finally:
            ops.set_w8a8_path(prev)
        assert y[0, 1] == 0x3F16
        assert same(y, G.gemm_rowcol(A, None, W, S, B, act=ACT_RELU, out=OUT_BF16))


def test_lm_head_full_size():
    """The Qwen3-0.6B lm_head at full size in one launch: K=1024, N=151936, bit-exact with the
    oracle (which the reference computes as 4 blocks of 37984 rows; elements are independent)."""
    x, q, s, W, scol, _ = w8_inputs(77, 1, 151936, 1024)
    y = ops.gemm_rowcol(cuda(q), cuda(s), cuda(W), cuda(scol))
    want = oracle_rowcol_blocked(q, s, W, scol, rows=37984)
    assert same(host(y), want), mismatch(host(y), want)


def test_strided_rows_and_untouched_gaps():
    """Strided A and Y rows give the dense result and leave the gaps untouched (test_golden.py:261-289)."""
    rng = np.random.default_rng(21)
    for path, M in (("gemv", 1), ("gemv", 2), ("gemv", 3), ("gemv", 6), ("mfma", 3), ("mfma", 40)):
        N, K = 64, 272
        A = rng.integers(-128, 128, (M, K), dtype=np.int8)
        W = rng.integers(-128, 128, (N, K), dtype=np.int8)
        sc = rng.uniform(1e-3, 1e-2, N).astype(f32)
        sr = rng.uniform(0.5, 2, M).astype(f32)
        abig = cuda(np.concatenate([A, np.zeros((M, 48), np.int8)], axis=1))
        ybig = torch.full((M, N + 12), -7.0, dtype=torch.float32, device="cuda")
        prev = ops.set_w8a8_path(path)
        try:
            ops.gemm_rowcol(abig[:, :K], cuda(sr), cuda(W), cuda(sc), y=ybig[:, :N])
        finally:
            ops.set_w8a8_path(prev)
        yb = host(ybig)
        assert same(yb[:, :N].copy(), G.gemm_rowcol(A, sr, W, sc)), (path, M)
        assert (yb[:, N:] == -7.0).all()


@pytest.mark.parametrize("M,N,K", [(200, 3072, 1024), (129, 3072, 1024), (300, 3072, 1024), (200, 3088, 256),
                                   (200, 3088, 1536), (100, 1040, 2048), (1040, 2064, 256)])
def test_strided_rows_prompt_tiles(M, N, K):
    """The LDS tile kernels on strided A and Y rows: the whole-K panels (K=1024 at 256, 192 and 320
    tiles, the rule's middle and ends; K=256), 64 x 48 tiles through the ring (K=1536), 32 x 32
    tiles with 512-byte stages (K=2048) and 64 x 64 tiles; the dense result, and the gaps left as
    they were."""
    rng = np.random.default_rng(M * 31 + N + K)
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    W = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sc = rng.uniform(1e-3, 1e-2, N).astype(f32)
    sr = rng.uniform(0.5, 2, M).astype(f32)
    abig = cuda(np.concatenate([A, np.zeros((M, 256), np.int8)], axis=1))
    ybig = torch.full((M, N + 20), -7.0, dtype=torch.float32, device="cuda")
    ops.gemm_rowcol(abig[:, :K], cuda(sr), cuda(W), cuda(sc), y=ybig[:, :N])
    yb = host(ybig)
    assert same(yb[:, :N].copy(), G.gemm_rowcol(A, sr, W, sc))
    assert (yb[:, N:] == -7.0).all()


def test_overlap_is_refused_and_nothing_is_written():
    rng = np.random.default_rng(3)
    buf = torch.zeros(64 * 1024 + 4096, dtype=torch.int8, device="cuda")
    W = buf[:16 * 1024].view(16, 1024)
    W.copy_(cuda(rng.integers(-128, 128, (16, 1024), dtype=np.int8)))
    q = cuda(rng.integers(-128, 128, (1, 1024), dtype=np.int8))
    before = host(buf).copy()
    y = buf[1024:1024 + 64].view(torch.float32).view(1, 16)          # inside W
    with pytest.raises(ops.ContractError):
        ops.gemm_rowcol(q, None, W, cuda(np.ones(16, f32)), y=y)
    assert same(host(buf), before)


# ------------------------------------------------------------------------------ K split (config 2)
@pytest.mark.parametrize("split", [[3456, 3456], [4096, 2816], [2304, 2304, 2304]])
@pytest.mark.parametrize("M", [1, 4])
def test_c2_gemma3_down_ksplit(split, M):
    """Config 2: Gemma-3-1B down_proj, K=6912 N=1152 as K blocks sharing the per-channel scales;
    the per-block partials add in fp32 in block order. Both the reference's 3456+3456 and the
    4096+2816 split, bit-exact, and the two splits differ."""
    x, q, s, W, scol, _ = w8_inputs(sum(split) + M, M, 1152, 6912)
    blocks, c0 = [], 0
    for k in split:
        blocks.append(np.ascontiguousarray(W[:, c0:c0 + k]))
        c0 += k
    qg, sg = ops.quant_rows(cuda(x))
    y = ops.gemm_rowcol_ksplit(qg, sg, [cuda(b) for b in blocks], cuda(scol))
    want = G.gemm_rowcol_ksplit(q, s, blocks, scol)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("M", [2, 3, 7, 16])
@pytest.mark.parametrize("split,N", [([256, 512, 1024], 1040), ([4096, 2816], 1152), ([1024, 256], 80)])
def test_ksplit_chunk_rows(M, split, N):
    """The K split on the chunk-row MFMA kernel (every block whole 256-byte blocks, M <= 16): blocks
    run one after another through the waves' LDS slots, partials added in block order."""
    x, q, s, W, scol, _ = w8_inputs(M * 17 + N + len(split), M, N, sum(split))
    blocks, c0 = [], 0
    for k in split:
        blocks.append(np.ascontiguousarray(W[:, c0:c0 + k]))
        c0 += k
    prev = ops.set_w8a8_path("mfma")
    try:
        y = ops.gemm_rowcol_ksplit(cuda(q), cuda(s), [cuda(b) for b in blocks], cuda(scol))
    finally:
        ops.set_w8a8_path(prev)
    want = G.gemm_rowcol_ksplit(q, s, blocks, scol)
    assert same(host(y), want), mismatch(host(y), want)


def test_ksplit_both_paths_agree():
    x, q, s, W, scol, _ = w8_inputs(5, 2, 256, 6912)
    blocks = [np.ascontiguousarray(W[:, :4096]), np.ascontiguousarray(W[:, 4096:])]
    outs = []
    for path in ("gemv", "mfma"):
        prev = ops.set_w8a8_path(path)
        try:
            outs.append(host(ops.gemm_rowcol_ksplit(cuda(q), cuda(s), [cuda(b) for b in blocks], cuda(scol))))
        finally:
            ops.set_w8a8_path(prev)
    want = G.gemm_rowcol_ksplit(q, s, blocks, scol)
    assert same(outs[0], want) and same(outs[1], want)


@pytest.mark.parametrize("N,split", [(n, sp) for n in (80, 1040, 1152, 1296, 2064)
                                     for sp in ([3456, 3456], [16, 8176], [1040, 2048])] + [(32784, [512, 512])])
def test_ksplit_two_blocks_whole_row_waves(N, split):
    """Two K blocks (the whole-row kernel: one wave per row, 4 to 8 waves per workgroup by N, four
    rows per wave from 32768 rows): block boundaries inside a lane's chunks, a first block of one
    chunk, a total of exactly 8192, ragged last workgroups."""
    K = sum(split)
    x, q, s, W, scol, _ = w8_inputs(N + K, 1, N, K)
    blocks = [np.ascontiguousarray(W[:, :split[0]]), np.ascontiguousarray(W[:, split[0]:])]
    y = ops.gemm_rowcol_ksplit(cuda(q), cuda(s), [cuda(b) for b in blocks], cuda(scol))
    want = G.gemm_rowcol_ksplit(q, s, blocks, scol)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("split", [[16], [16, 32], [48, 1040, 16], [4096, 4096], [4096, 4112], [1024] * 8,
                                   [2816, 3456, 16], [7168, 1024]])
@pytest.mark.parametrize("M", [1, 3])
def test_ksplit_gemv_block_shapes(split, M):
    """The K-split GEMV family: one to eight blocks, widths that are not multiples of 64, a total of
    exactly 8192 (all loads in flight) and just above it (the loop kernel), 1 and 3 rows."""
    K = sum(split)
    x, q, s, W, scol, _ = w8_inputs(K * 3 + M, M, 80, K)
    blocks, c0 = [], 0
    for k in split:
        blocks.append(np.ascontiguousarray(W[:, c0:c0 + k]))
        c0 += k
    prev = ops.set_w8a8_path("gemv")
    try:
        y = ops.gemm_rowcol_ksplit(cuda(q), cuda(s), [cuda(b) for b in blocks], cuda(scol))
    finally:
        ops.set_w8a8_path(prev)
    want = G.gemm_rowcol_ksplit(q, s, blocks, scol)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("M,N,blocks", [(17, 208, [4096, 2816]), (45, 208, [4096, 2816]), (200, 3072, [256, 512]),
                                          (100, 1040, [2048, 1024]), (33, 96, [1040, 256])])
def test_ksplit_staged_prompt_tiles(M, N, blocks):
    """The K split on the LDS tile kernel: 32 x 32 tiles with 256-byte stages (M=17, 45), 64 x 48
    tiles (M=200, N=3072), 32 x 32 tiles with 512-byte stages in 3 slots (M=100, N=1040, blocks
    of whole KiB), and a block that is not a whole number of stages (1040), which takes the direct
    tiles."""
    x, q, s, W, scol, _ = w8_inputs(M * 31 + N, M, N, sum(blocks))
    parts = np.split(W, np.cumsum(blocks)[:-1], axis=1)
    parts = [np.ascontiguousarray(b) for b in parts]
    y = ops.gemm_rowcol_ksplit(cuda(q), cuda(s), [cuda(b) for b in parts], cuda(scol))
    want = G.gemm_rowcol_ksplit(q, s, parts, scol)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("M", [17, 45])
def test_ksplit_prompt_tiles(M):
    """The K split on the prompt-row MFMA tiles (M > 16), with a ragged last row and column tile."""
    x, q, s, W, scol, _ = w8_inputs(M + 77, M, 208, 6912)
    blocks = [np.ascontiguousarray(W[:, :4096]), np.ascontiguousarray(W[:, 4096:])]
    y = ops.gemm_rowcol_ksplit(cuda(q), cuda(s), [cuda(b) for b in blocks], cuda(scol))
    want = G.gemm_rowcol_ksplit(q, s, blocks, scol)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("qm", ["tensor", "channel", "rowcol"])
@pytest.mark.parametrize("act,out", [(ACT_NONE, OUT_FP32), (ACT_RELU, OUT_INT8), (ACT_SILU, OUT_BF16),
                                     (ACT_GELU, OUT_FP32), (ACT_SOFTPLUS, OUT_BF16)])
def test_epilogue_matrix_prompt_tiles(qm, act, out):
    """The prompt-row MFMA tiles (M > 16) through every scale mode and output format with a bias,
    a ragged last row and column tile (M = 45, N = 80), a huge scale and int8 -128."""
    rng = np.random.default_rng(zlib.crc32(repr((qm, act, out, "prompt")).encode()))
    M, N, K = 45, 80, 16 * int(rng.integers(1, 90))
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    W = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sc = rng.uniform(1e-4, 3e-2, N).astype(f32)
    sc[N // 3] = 3e30
    if qm == "tensor":
        sc = sc[:1]
    srow = rng.uniform(0.1, 2.0, M).astype(f32) if qm == "rowcol" else None
    b = rng.normal(0, 2, N).astype(f32)
    osc = f32(5.0) if out == OUT_INT8 else None
    y = ops.gemm_rowcol(cuda(A), None if srow is None else cuda(srow), cuda(W), cuda(sc), cuda(b),
                        act=act, out=out, out_scale=osc)
    want = G.gemm_rowcol(A, srow, W, sc, b, act=act, out=out, out_scale=osc)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("qm", ["tensor", "channel", "rowcol"])
@pytest.mark.parametrize("act,out", [(ACT_NONE, OUT_FP32), (ACT_RELU, OUT_INT8), (ACT_SILU, OUT_BF16),
                                     (ACT_GELU, OUT_FP32), (ACT_SOFTPLUS, OUT_BF16)])
@pytest.mark.parametrize("M,N,K", [(45, 80, 768), (45, 80, 2048), (200, 3072 + 16, 1536), (200, 3072 + 16, 512),
                                   (200, 3072 + 16, 1024), (131, 4608, 1280)])
def test_epilogue_matrix_staged_tiles(qm, act, out, M, N, K):
    """The LDS tile kernels (K a multiple of 256) through every scale mode and output format with a
    bias, ragged last row and column tiles, a huge scale and int8 -128: 32 x 32 tiles with
    256-byte stages (K=768), with 512-byte stages in 3 slots (K=2048), 64 x 48 tiles through the
    ring (M=200, N=3088, K=1536), and the 64 x 48 tiles with the whole K resident (K=512, 1024,
    1280; at M=131 three of the last row tile's four waves have no row to store)."""
    rng = np.random.default_rng(zlib.crc32(repr((qm, act, out, M, N, K, "staged")).encode()))
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    W = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sc = rng.uniform(1e-4, 3e-2, N).astype(f32)
    sc[N // 3] = 3e30
    if qm == "tensor":
        sc = sc[:1]
    srow = rng.uniform(0.1, 2.0, M).astype(f32) if qm == "rowcol" else None
    b = rng.normal(0, 2, N).astype(f32)
    osc = f32(5.0) if out == OUT_INT8 else None
    y = ops.gemm_rowcol(cuda(A), None if srow is None else cuda(srow), cuda(W), cuda(sc), cuda(b),
                        act=act, out=out, out_scale=osc)
    want = G.gemm_rowcol(A, srow, W, sc, b, act=act, out=out, out_scale=osc)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("qm,act,out", [("rowcol", ACT_NONE, OUT_FP32), ("channel", ACT_SILU, OUT_BF16),
                                        ("tensor", ACT_RELU, OUT_INT8)])
def test_large_prompt_tiles(qm, act, out):
    """The 64 x 64 tiles the tile kernel takes when they give 512 or more workgroups (M=1040,
    N=2064: ragged last row and column tiles) through three scale modes and output formats."""
    rng = np.random.default_rng(zlib.crc32(repr((qm, act, out, "large")).encode()))
    M, N, K = 1040, 2064, 256
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    W = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sc = rng.uniform(1e-4, 3e-2, N).astype(f32)
    if qm == "tensor":
        sc = sc[:1]
    srow = rng.uniform(0.1, 2.0, M).astype(f32) if qm == "rowcol" else None
    b = rng.normal(0, 2, N).astype(f32)
    osc = f32(5.0) if out == OUT_INT8 else None
    y = ops.gemm_rowcol(cuda(A), None if srow is None else cuda(srow), cuda(W), cuda(sc), cuda(b),
                        act=act, out=out, out_scale=osc)
    want = G.gemm_rowcol(A, srow, W, sc, b, act=act, out=out, out_scale=osc)
    assert same(host(y), want), mismatch(host(y), want)


# ------------------------------------------------------------------------------ prefill GEMM (config 4)
@pytest.mark.parametrize("path", ["auto", "gemv", "mfma"])
@pytest.mark.parametrize("M", [4, 256])
@pytest.mark.parametrize("K,N", [(1024, 3072), (3072, 1024)])
def test_c4_prefill_gemm(path, M, K, N):
    """Config 4 on both kernel families and the automatic choice."""
    x, q, s, W, scol, _ = w8_inputs(M * 7 + K, M, N, K)
    qg, sg = ops.quant_rows(cuda(x))
    assert same(host(qg), q) and same(host(sg), s)
    prev = ops.set_w8a8_path(path)
    try:
        y = ops.gemm_rowcol(qg, sg, cuda(W), cuda(scol))
    finally:
        ops.set_w8a8_path(prev)
    want = G.gemm_rowcol(q, s, W, scol)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("M", [2, 3, 5, 16, 17, 31, 33, 64, 100, 300])
@pytest.mark.parametrize("K", [64, 256, 1024, 1040, 5000 // 16 * 16])
def test_mfma_ragged_m_and_k(M, K):
    x, q, s, W, scol, rng = w8_inputs(M * 1000 + K, M, 80, K)
    b = rng.normal(0, 1, 80).astype(f32)
    prev = ops.set_w8a8_path("mfma")
    try:
        y = ops.gemm_rowcol(cuda(q), cuda(s), cuda(W), cuda(scol), cuda(b), act=ACT_SILU)
    finally:
        ops.set_w8a8_path(prev)
    want = G.gemm_rowcol(q, s, W, scol, b, act=ACT_SILU)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("M", [2, 3, 4, 5, 7, 9, 16])
@pytest.mark.parametrize("K,N", [(64, 80), (496, 4112), (1040, 80), (4992, 80), (8192, 48), (9216, 32)])
def test_gemv_rows_ragged(M, K, N):
    """The GEMV family with 2 or 4 activation rows per block (and the loop form past K = 8192):
    ragged last row block, every lane-group width, rows per wave 1/2 (N = 4112 has a partial
    block), bias and SiLU."""
    x, q, s, W, scol, rng = w8_inputs(M * 7919 + K + N, M, N, K)
    b = rng.normal(0, 1, N).astype(f32)
    prev = ops.set_w8a8_path("gemv")
    try:
        y = ops.gemm_rowcol(cuda(q), cuda(s), cuda(W), cuda(scol), cuda(b), act=ACT_SILU)
    finally:
        ops.set_w8a8_path(prev)
    want = G.gemm_rowcol(q, s, W, scol, b, act=ACT_SILU)
    assert same(host(y), want), mismatch(host(y), want)


def test_gemv_family_for_prefill_rows_matches():
    x, q, s, W, scol, _ = w8_inputs(11, 4, 3072, 1024)
    prev = ops.set_w8a8_path("gemv")
    try:
        y = host(ops.gemm_rowcol(cuda(q), cuda(s), cuda(W), cuda(scol)))
    finally:
        ops.set_w8a8_path(prev)
    assert same(y, G.gemm_rowcol(q, s, W, scol))


def random_w8_case(rng):
    """A W8A8 GEMM drawn across the launch rules of both families: M from 1 to 300, K and N multiples
    of 16 (K sometimes a whole number of MFMA stages), a scale mode, bias, activation and output
    format, the product bounded so the oracle stays quick."""
    M = int(rng.choice([1, 1, 1, 2, 3, 4, 5, 8, 12, 16, 17, 33, 64, 100, 256, 300]))
    K = 256 * int(rng.integers(1, 25)) if rng.random() < 0.5 else 16 * int(rng.integers(1, 600))
    N = 16 * int(rng.integers(1, max(2, min(2048, 60_000_000 // (M * K * 16)) + 1)))
    qm = str(rng.choice(["tensor", "channel", "rowcol"]))
    act, out = [(ACT_NONE, OUT_FP32), (ACT_RELU, OUT_INT8), (ACT_SILU, OUT_BF16), (ACT_GELU, OUT_FP32),
                (ACT_SOFTPLUS, OUT_INT8)][int(rng.integers(0, 5))]
    return M, K, N, qm, bool(rng.integers(0, 2)), act, out


@pytest.mark.parametrize("seed", range(40))
def test_w8a8_random_shapes(seed):
    """Random GEMMs (random_w8_case) through the automatic path rule and, on every third case, the
    other family forced: bit-exact against the oracle whichever kernel and launch shape run."""
    rng = np.random.default_rng(700 + seed)
    M, K, N, qm, bias, act, out = random_w8_case(rng)
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    W = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sc = rng.uniform(1e-4, 3e-2, N).astype(f32)
    if qm == "tensor":
        sc = sc[:1]
    srow = rng.uniform(0.1, 2.0, M).astype(f32) if qm == "rowcol" else None
    b = rng.normal(0, 2, N).astype(f32) if bias else None
    osc = f32(5.0) if out == OUT_INT8 else None
    path = ["auto", "auto", "gemv" if M > 4 else "mfma"][seed % 3]
    prev = ops.set_w8a8_path(path)
    try:
        y = ops.gemm_rowcol(cuda(A), None if srow is None else cuda(srow), cuda(W), cuda(sc),
                            None if b is None else cuda(b), act=act, out=out, out_scale=osc)
    finally:
        ops.set_w8a8_path(prev)
    want = G.gemm_rowcol(A, srow, W, sc, b, act=act, out=out, out_scale=osc)
    assert same(host(y), want), ((M, K, N, qm, path), mismatch(host(y), want))


@pytest.mark.parametrize("seed", range(12))
def test_w8a8_random_panels(seed):
    """Random GEMMs that the whole-K panel rule takes (K from 256 to 1280, 192 to 320 tiles of
    64 x 48, ragged last row and column tiles), every scale mode, bias, activation and output
    format: bit-exact against the oracle."""
    rng = np.random.default_rng(900 + seed)
    mt = int(rng.integers(3, 6))
    M = 64 * mt - int(rng.integers(0, 63))
    nt = int(rng.integers(-(-192 // mt), 320 // mt + 1))
    N, K = 48 * nt - 16 * int(rng.integers(0, 3)), 256 * int(rng.integers(1, 6))
    qm = str(rng.choice(["tensor", "channel", "rowcol"]))
    act, out = [(ACT_NONE, OUT_FP32), (ACT_RELU, OUT_INT8), (ACT_SILU, OUT_BF16), (ACT_GELU, OUT_FP32),
                (ACT_SOFTPLUS, OUT_INT8)][int(rng.integers(0, 5))]
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    W = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sc = rng.uniform(1e-4, 3e-2, N).astype(f32)
    if qm == "tensor":
        sc = sc[:1]
    srow = rng.uniform(0.1, 2.0, M).astype(f32) if qm == "rowcol" else None
    b = rng.normal(0, 2, N).astype(f32) if rng.random() < 0.5 else None
    osc = f32(5.0) if out == OUT_INT8 else None
    y = ops.gemm_rowcol(cuda(A), None if srow is None else cuda(srow), cuda(W), cuda(sc),
                        None if b is None else cuda(b), act=act, out=out, out_scale=osc)
    want = G.gemm_rowcol(A, srow, W, sc, b, act=act, out=out, out_scale=osc)
    assert same(host(y), want), ((M, N, qm, act, out), mismatch(host(y), want))


@pytest.mark.parametrize("seed", range(24))
def test_ksplit_random_blocks(seed):
    """The K split over random block counts (1 to 5) and block widths (multiples of 16, total K
    up to 9000) at random M and N: bit-exact against the oracle's block-ordered partials."""
    rng = np.random.default_rng(800 + seed)
    M = int(rng.choice([1, 1, 2, 3, 4, 7, 17, 40]))
    nb = int(rng.integers(1, 6))
    ks = [16 * int(rng.integers(1, max(2, 9000 // (16 * nb)))) for _ in range(nb)]
    N = 16 * int(rng.integers(1, max(2, min(256, 30_000_000 // (M * sum(ks) * 16)) + 1)))
    x, q, s, W, scol, _ = w8_inputs(seed * 31 + M, M, N, sum(ks))
    blocks, c0 = [], 0
    for k in ks:
        blocks.append(np.ascontiguousarray(W[:, c0:c0 + k]))
        c0 += k
    qg, sg = ops.quant_rows(cuda(x))
    y = ops.gemm_rowcol_ksplit(qg, sg, [cuda(b) for b in blocks], cuda(scol))
    want = G.gemm_rowcol_ksplit(q, s, blocks, scol)
    assert same(host(y), want), ((M, ks, N), mismatch(host(y), want))


# ------------------------------------------------------------------------------ W4A16 (config 5)
@pytest.mark.parametrize("i", range(8))
def test_w4_reference_vectors(i):
    k = f"w4_{i}"
    m, n, K, half, bias, act, fmt, osb = (int(v) for v in VEC[k + "_meta"])
    x = VEC[k + "_x"]
    y = ops.gemm_w4(cuda(x), cuda(VEC[k + "_wp"]), cuda(VEC[k + "_ws"]),
                    bias=cuda(VEC[k + "_bias"]) if bias else None, act=act, out=fmt,
                    out_scale=np.array([osb], np.uint32).view(f32)[0], x_is_bf16=bool(half))
    got = np.ascontiguousarray(host(y)).view(np.uint8).ravel()
    assert got.tobytes() == VEC[k + "_y"].tobytes(), mismatch(got, VEC[k + "_y"])


def w4_inputs(seed: int, M: int, N: int, K: int):
    rng = np.random.default_rng(seed)
    nib = rng.integers(-8, 8, (N, K))
    Wp = G.pack_int4(nib)
    ws = rng.uniform(1e-3, 1e-2, (N, K // 128)).astype(np.float16).view(np.uint16)
    x = rng.normal(0, 1, (M, K)).astype(f32)
    return x, Wp, ws, rng


def random_w4_shape(rng):
    """A W4A16 launch shape drawn across every form's rule boundaries: M from 1 to 40, K a multiple
    of 256 up to 8192, N a multiple of 16, the product bounded so the oracle stays quick."""
    M = int(rng.choice([1, 1, 1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 16, 17, 24, 33, 40]))
    K = 256 * int(rng.integers(1, 33))
    N = 16 * int(rng.integers(1, max(2, min(1024, 40_000_000 // (M * K * 16)) + 1)))
    return M, K, N


@pytest.mark.parametrize("seed", range(48))
def test_w4a16_random_shapes(seed):
    """Random shapes (random_w4_shape) through the automatic launch rule: whichever form and
    workgroup shape it picks, the result matches the oracle bit for bit, with random bf16 rows, an
    epilogue, and subnormal, zero, infinite and NaN group scales."""
    rng = np.random.default_rng(900 + seed)
    M, K, N = random_w4_shape(rng)
    x, Wp, ws, _ = w4_inputs(seed * 7919 + M + K + N, M, N, K)
    ws = ws.copy()
    for v in (0x0001, 0x0000, 0x7C00, 0xFE01):
        ws[rng.integers(0, N), rng.integers(0, K // 128)] = v
    bf16 = bool(rng.integers(0, 2))
    xin = F.to_bf16_bits(x) if bf16 else x
    epi = int(rng.integers(0, 3))
    kw = {}
    if epi == 1:
        kw = dict(bias=rng.normal(0, 1, N).astype(f32), act=ACT_SILU, out=OUT_BF16)
    elif epi == 2:
        kw = dict(out=OUT_INT8, out_scale=f32(0.125))
    dkw = {k: (cuda(v) if isinstance(v, np.ndarray) else v) for k, v in kw.items()}
    y = ops.gemm_w4(cuda(xin), cuda(Wp), cuda(ws), x_is_bf16=bf16, **dkw)
    want = G.gemm_w4(xin, Wp, ws, x_is_bf16=bf16, **kw)
    assert same(host(y), want), (M, K, N, mismatch(host(y), want))


@pytest.mark.parametrize("K,N", [(1536, 12288), (6144, 1536)])
@pytest.mark.parametrize("seed", range(2))
def test_c5_w4a16_gemma4(K, N, seed):
    """Config 5: Gemma-4-E2B-style W4A16 GEMV, bit-exact (no tolerance needed)."""
    x, Wp, ws, _ = w4_inputs(seed * 31 + K, 1, N, K)
    y = ops.gemm_w4(cuda(x), cuda(Wp), cuda(ws))
    want = G.gemm_w4(x, Wp, ws)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("K,N", [(1536, 12288), (6144, 1536)])
@pytest.mark.parametrize("M", [2, 4, 5, 8])
def test_w4a16_prefill_chunks(K, N, M):
    """W4A16 for prefill chunks (the board's W4 unit serves 1 / 4 / 8 rows): the C5 shapes at
    M = 2, 4, 8 and a ragged M = 5 (two activation rows per block, the last block half empty)."""
    x, Wp, ws, _ = w4_inputs(K + 7 * M, M, N, K)
    y = ops.gemm_w4(cuda(x), cuda(Wp), cuda(ws))
    want = G.gemm_w4(x, Wp, ws)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("K", [256, 512, 768, 1024, 2048, 4096, 8192])
@pytest.mark.parametrize("M", [1, 3])
def test_w4_shapes_bf16_bias_act(K, M):
    x, Wp, ws, rng = w4_inputs(K + M, M, 48, K)
    ws = ws.copy()
    ws[5, 1], ws[6, 0], ws[7, 1] = 0x7E01, 0xFC05, 0x0003          # NaN scales (payloads), a subnormal
    x = (x * np.exp2(rng.integers(-30, 30, (M, K // 128, 1))).repeat(128, axis=2).reshape(M, K)).astype(f32)
    xb = F.to_bf16_bits(x)
    b = rng.normal(0, 1, 48).astype(f32)
    y = ops.gemm_w4(cuda(xb), cuda(Wp), cuda(ws), bias=cuda(b), act=ACT_GELU, out=OUT_BF16, x_is_bf16=True)
    want = G.gemm_w4(xb, Wp, ws, bias=b, act=ACT_GELU, out=OUT_BF16, x_is_bf16=True)
    assert same(host(y), want), mismatch(host(y), want)
    y2 = ops.gemm_w4(cuda(x), cuda(Wp), cuda(ws), out=OUT_INT8, out_scale=f32(0.25))
    assert same(host(y2), G.gemm_w4(x, Wp, ws, out=OUT_INT8, out_scale=f32(0.25)))


@pytest.mark.parametrize("M,K,N", [
    (3, 1536, 8208),                             # 4-row tiles, 4 waves
    (4, 1024, 3072), (9, 2048, 80),              # 4-row tiles, 8 waves
    (7, 768, 4096), (20, 512, 1040),             # 8-row tiles, 8 waves, one weight tile
    (16, 1536, 3088),                            # 8-row tiles, two weight tiles of 16 waves
    (16, 1536, 8208),                            # 8-row tiles, two weight tiles of 8 waves
    (129, 256, 1456),                            # 8-row tiles, four weight tiles
    (12, 6144, 96), (6, 6144, 2048),             # K > 2048: 4-row tiles, 16 waves
    (24, 3072, 1040),                            # K > 2048: 8-row tiles, one weight tile
    (24, 3072, 1424), (3, 4096, 8192),           # K > 2048: 8-row tiles, two weight tiles
    (12, 8192, 32),                              # 64 groups: 4-row tiles, 16 waves
    (2, 256, 16), (8, 1024, 256)])               # the per-lane form
@pytest.mark.parametrize("epi", ["plain", "bias_silu_bf16", "int8"])
@pytest.mark.parametrize("bf16", [False, True])
def test_w4a16_mfma_shapes(M, K, N, epi, bf16):
    """Every launch shape of the W4A16 GEMM at M >= 3 on INT8 MFMA (4- and 8-row activation
    tiles, one, two or four weight tiles per workgroup, groups split over 4 to 16 waves; 8 rows
    past M on the 4-row tiles and rows past M in the last 8-row tile), and the per-lane form
    beside them: K from 256 to 8192, ragged last tiles, fp16 group scales that are subnormal, zero,
    infinite and NaN (payloads of both signs), fp32 and bf16 activation rows, and every output
    format."""
    x, Wp, ws, rng = w4_inputs(M * 1000 + K + N, M, N, K)
    ws = ws.copy()
    ws[0, 0], ws[1 % N, K // 128 - 1], ws[2 % N, 0] = 0x0001, 0x0000, 0x7C00
    ws[3 % N, 1], ws[4 % N, 0] = 0x7E01, 0xFC05                    # NaNs with payloads, both signs
    xin = F.to_bf16_bits(x) if bf16 else x
    kw = {}
    if epi == "bias_silu_bf16":
        kw = dict(bias=rng.normal(0, 1, N).astype(f32), act=ACT_SILU, out=OUT_BF16)
    elif epi == "int8":
        kw = dict(out=OUT_INT8, out_scale=f32(0.125))
    dkw = {k: (cuda(v) if isinstance(v, np.ndarray) else v) for k, v in kw.items()}
    y = ops.gemm_w4(cuda(xin), cuda(Wp), cuda(ws), x_is_bf16=bf16, **dkw)
    want = G.gemm_w4(xin, Wp, ws, x_is_bf16=bf16, **kw)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("M,K,N", [
    (2, 6144, 1536), (4, 8192, 1008), (5, 8192, 48),        # 8-wave workgroups, one row per wave
    (2, 2048, 2048), (4, 1024, 1024),
    (4, 6144, 1536), (3, 3072, 1040), (8, 3072, 1024),      # two rows per wave (ragged N = 1040)
    (4, 2048, 2048), (5, 2048, 1024),
    (8, 6144, 1536), (4, 1536, 3072), (2, 6144, 5120),      # three rows per wave
    (2, 4096, 8192), (8, 2048, 2048), (7, 4096, 2048),      # four rows per wave
    (2, 512, 8192),
    (2, 2304, 8208), (2, 1536, 12304)])                     # wider (M = 2): 4-row waves of 4-wave workgroups
@pytest.mark.parametrize("epi", ["plain", "bias_silu_bf16", "int8"])
def test_w4a16_two_row_blocks(M, K, N, epi):
    """The per-lane W4A16 form with two activation rows per workgroup (M = 2 to 8): every workgroup
    shape its rule picks, one to four chunks per lane, bf16 activations on half the cases, every
    output format, fp16 scales that are subnormal, zero, infinite and NaN."""
    x, Wp, ws, rng = w4_inputs(M * 13 + K + N, M, N, K)
    ws = ws.copy()
    ws[0, 0], ws[1, K // 128 - 1], ws[2, 1], ws[3, 2] = 0x0001, 0x0000, 0x7C00, 0xFC05
    bf16 = (K // 256 + M) % 2 == 0
    xin = F.to_bf16_bits(x) if bf16 else x
    kw = {}
    if epi == "bias_silu_bf16":
        kw = dict(bias=rng.normal(0, 1, N).astype(f32), act=ACT_SILU, out=OUT_BF16)
    elif epi == "int8":
        kw = dict(out=OUT_INT8, out_scale=f32(0.125))
    dkw = {k: (cuda(v) if isinstance(v, np.ndarray) else v) for k, v in kw.items()}
    y = ops.gemm_w4(cuda(xin), cuda(Wp), cuda(ws), x_is_bf16=bf16, **dkw)
    want = G.gemm_w4(xin, Wp, ws, x_is_bf16=bf16, **kw)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("M,K,N", [
    (1, 1536, 256), (1, 6144, 64),               # whole-row waves: one chunk per lane, three
    (1, 2304, 4096),                             # whole-row waves, 16 rows per workgroup
    (1, 8192, 64),                               # K split over the waves
    (2, 1024, 64),                               # the per-lane form with two activation rows
    (3, 1536, 8192), (12, 6144, 96), (20, 512, 1040)])  # the MFMA form: 4- and 8-row tiles
@pytest.mark.parametrize("bf16", [False, True])
def test_w4_strided_rows_and_untouched_gaps(M, K, N, bf16):
    """Every W4A16 kernel form on activation rows and output rows with a gap after each (lda and
    ldy above the row): the dense result, and the output gaps left as they were."""
    x, Wp, ws, _ = w4_inputs(M * 7 + K + N + bf16, M, N, K)
    xin = F.to_bf16_bits(x) if bf16 else x
    xbig = np.concatenate([xin, np.zeros((M, 64), xin.dtype)], axis=1)
    ybig = torch.full((M, N + 12), -7.0, dtype=torch.float32, device="cuda")
    ops.gemm_w4(cuda(xbig)[:, :K], cuda(Wp), cuda(ws), y=ybig[:, :N], x_is_bf16=bf16)
    yb = host(ybig)
    want = G.gemm_w4(xin, Wp, ws, x_is_bf16=bf16)
    assert same(yb[:, :N].copy(), want), mismatch(yb[:, :N].copy(), want)
    assert (yb[:, N:] == -7.0).all()


@pytest.mark.parametrize("K,N", [
    (2304, 1008), (3072, 528),                   # 4 weight rows per workgroup
    (6144, 1536), (8192, 2032), (6144, 1024),    # 8
    (5120, 2560), (2560, 3008),                  # 12
    (4096, 4096), (6144, 3088),                  # 16
    (3072, 6144), (2304, 12288),                 # 24 (also past N = 8192)
    (2304, 8192), (4096, 7008)])                 # 32
@pytest.mark.parametrize("epi", ["plain", "bias_silu_bf16", "int8"])
def test_w4a16_whole_row_shapes(K, N, epi):
    """One activation row past 2048 k on whole-row waves: every workgroup shape of the rule (4 to
    32 weight rows per workgroup, 4 and 8 waves, 1 to 4 rows per wave), ragged N, bf16 activations
    on half the cases, every output format, fp16 scales that are subnormal, zero, infinite and
    NaN."""
    x, Wp, ws, rng = w4_inputs(K * 3 + N, 1, N, K)
    ws = ws.copy()
    ws[0, 0], ws[1, K // 128 - 1], ws[2, 1], ws[3, 2] = 0x0001, 0x0000, 0x7C00, 0xFE01
    bf16 = (K // 256 + N) % 2 == 0
    xin = F.to_bf16_bits(x) if bf16 else x
    kw = {}
    if epi == "bias_silu_bf16":
        kw = dict(bias=rng.normal(0, 1, N).astype(f32), act=ACT_SILU, out=OUT_BF16)
    elif epi == "int8":
        kw = dict(out=OUT_INT8, out_scale=f32(0.125))
    dkw = {k: (cuda(v) if isinstance(v, np.ndarray) else v) for k, v in kw.items()}
    y = ops.gemm_w4(cuda(xin), cuda(Wp), cuda(ws), x_is_bf16=bf16, **dkw)
    want = G.gemm_w4(xin, Wp, ws, x_is_bf16=bf16, **kw)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("K,N", [(8192, 1008), (8192, 64), (6400, 1024), (7424, 528), (6656, 16)])
@pytest.mark.parametrize("epi", ["plain", "bias_silu_bf16", "int8"])
def test_w4a16_ksplit_waves(K, N, epi):
    """One activation row with K split over the waves of a workgroup (past 6144 k at N <= 1024): 4
    weight rows per workgroup, ragged N, a last wave with two groups (G % 4 == 2 at K = 6400,
    7424), bf16 activations on half the cases, every output format."""
    x, Wp, ws, rng = w4_inputs(K + N, 1, N, K)
    ws = ws.copy()
    ws[0, 0], ws[1, K // 128 - 1], ws[2, 1], ws[3, 2] = 0x0001, 0x0000, 0x7C00, 0x7E01
    bf16 = (K // 256) % 2 == 0
    xin = F.to_bf16_bits(x) if bf16 else x
    kw = {}
    if epi == "bias_silu_bf16":
        kw = dict(bias=rng.normal(0, 1, N).astype(f32), act=ACT_SILU, out=OUT_BF16)
    elif epi == "int8":
        kw = dict(out=OUT_INT8, out_scale=f32(0.125))
    dkw = {k: (cuda(v) if isinstance(v, np.ndarray) else v) for k, v in kw.items()}
    y = ops.gemm_w4(cuda(xin), cuda(Wp), cuda(ws), x_is_bf16=bf16, **dkw)
    want = G.gemm_w4(xin, Wp, ws, x_is_bf16=bf16, **kw)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("K,N", [(8192, 64), (6400, 512)])
@pytest.mark.parametrize("kind", ["mixed", "inf", "nan"])
@pytest.mark.parametrize("bf16", [False, True])
def test_w4a16_ksplit_special_groups(K, N, kind, bf16):
    """The K-split form's per-wave aligner on one row's special groups: all-zero, tiny (largest
    exponent below 16), subnormals inside a normal group and the largest finite values beside
    ordinary groups; an infinite group; a NaN group (waves of both kinds in one launch)."""
    rng = np.random.default_rng(K + N + bf16)
    x, Wp, ws, _ = w4_inputs(K * 5 + bf16, 1, N, K)
    g = x.reshape(K // 128, 128)
    if kind == "mixed":
        g[1] = 0.0
        g[2] = rng.normal(0, 1, 128) * np.float32(2.0 ** -115)
        g[5, ::7] = np.array([1, 0x80000003, 0x007FFFFF], np.uint32).view(f32).repeat(7)[:19]
        g[9] = np.float32(3.3e38) * np.sign(rng.normal(0, 1, 128)).astype(f32)
    elif kind == "inf":
        g[7, 5], g[7, 9] = np.inf, -np.inf
        g[8, 3] = np.inf
    else:
        g[K // 128 - 1, 17] = np.nan
    x = g.reshape(1, K).astype(f32)
    xin = F.to_bf16_bits(x) if bf16 else x
    y = ops.gemm_w4(cuda(xin), cuda(Wp), cuda(ws), x_is_bf16=bf16)
    want = G.gemm_w4(xin, Wp, ws, x_is_bf16=bf16)
    assert same(host(y), want), mismatch(host(y), want)


def w4_chains_ending_at_minus_zero(M: int, N: int, K: int):
    """Inputs whose every bank chain ends in a negative subnormal partial sum, which the contract's
    flushed adds turn into -0: in each bank (groups b, b + 4, ...) the last two groups hold the same
    activations (magnitudes 2^-108 to 2^-106 with one sign pattern for every row, element 5 at
    2^-115) and opposite weights (5 with the activation's sign, then -5), except element 5 of the
    last, one lower; with every group scale 2^-20 the first term is normal (about 2^-118), both are
    exact, and they add to -a_5 2^-20 xs (about -2^-134); the bank's other groups are zero (terms
    +0)."""
    G_ = K // 128
    rng = np.random.default_rng(K + M)
    x = np.zeros((M, K), f32)
    w = rng.integers(-6, 7, (N, K)).astype(np.int64)
    for b in range(4):
        g1, g2 = list(range(b, G_, 4))[-2:]
        sgn = rng.choice(np.array([-1, 1]), 128)
        sgn[5] = 1
        blk = ((np.abs(rng.normal(0, 1, (M, 128))) % 2 + 1) * sgn * 2.0 ** -108).astype(f32)
        blk[:, 5] = f32(2.0 ** -115)
        x[:, g1 * 128:(g1 + 1) * 128] = blk
        x[:, g2 * 128:(g2 + 1) * 128] = blk
        w[:, g1 * 128:(g1 + 1) * 128] = 5 * sgn
        w[:, g2 * 128:(g2 + 1) * 128] = -5 * sgn
        w[:, g2 * 128 + 5] -= 1
    nib = (w & 15).astype(np.uint8)
    Wp = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    ws = np.full((N, G_), 0x0010, np.uint16)
    return x, Wp, ws


@pytest.mark.parametrize("M,K", [(1, 1280), (1, 1536), (1, 6144), (1, 8192), (2, 1536), (12, 1536), (12, 6144)])
def test_w4_bank_chains_ending_at_minus_zero(M, K):
    """Every bank's flushed chain ends at -0 (w4_chains_ending_at_minus_zero), so every output is
    -0 only if no +0 is added after a bank's last group: the whole-row waves (their unflushed chains
    run every register step, the steps past the last group adding +0, and are recomputed with the
    flushes when a partial sum is subnormal; 10, 12 and 48 groups), the K split over waves, the
    per-lane form with two activation rows and the MFMA form."""
    N = 64
    x, Wp, ws = w4_chains_ending_at_minus_zero(M, N, K)
    want = G.gemm_w4(x, Wp, ws)
    assert (want.view(np.uint32) == 0x80000000).all()
    y = ops.gemm_w4(cuda(x), cuda(Wp), cuda(ws))
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("K", [1024, 6144])
@pytest.mark.parametrize("M", [6, 12, 16])
@pytest.mark.parametrize("bf16", [False, True])
def test_w4_gemm_special_groups(K, M, bf16):
    """The in-kernel aligners (the per-lane form's at M = 6, the MFMA form's 4-row tiles at M = 12
    and 8-row tiles at M = 16) on groups that leave their fast path: all-zero, tiny (largest
    exponent below 16), subnormal inputs inside normal groups, +-inf, NaN, and the largest finite
    values, in rows whose other groups are ordinary (so waves of both kinds meet in one launch)."""
    rng = np.random.default_rng(K + bf16)
    N = 64 if M < 16 else (2064 if K == 1024 else 1040)
    x, Wp, ws, _ = w4_inputs(K * 3 + bf16 + M, M, N, K)
    g = x.reshape(M, K // 128, 128)
    g[0, 1] = 0.0                                                  # all-zero group
    g[0, 2] = rng.normal(0, 1, 128) * np.float32(2.0 ** -115)      # emax < 16
    g[1, 0, ::7] = np.array([1, 0x80000003, 0x007FFFFF], np.uint32).view(f32).repeat(7)[:19]  # subnormals
    g[2, 3, 5], g[2, 3, 9] = np.inf, -np.inf                       # infinity group
    g[3, K // 128 - 1, 17] = np.nan                                # NaN group
    g[4, 1] = np.float32(3.3e38) * np.sign(rng.normal(0, 1, 128)).astype(f32)
    g[5] = rng.normal(0, 1, (K // 128, 128)) * np.exp2(rng.integers(-126, 100, (K // 128, 1)))
    x = g.reshape(M, K).astype(f32)
    xin = F.to_bf16_bits(x) if bf16 else x
    y = ops.gemm_w4(cuda(xin), cuda(Wp), cuda(ws), x_is_bf16=bf16)
    want = G.gemm_w4(xin, Wp, ws, x_is_bf16=bf16)
    assert same(host(y), want), mismatch(host(y), want)


@pytest.mark.parametrize("bf16", [False, True])
def test_align_w4_groups(bf16):
    rng = np.random.default_rng(44)
    M, K = 4, 1024
    x = (rng.normal(0, 1, (M, K // 128, 128)) * np.exp2(rng.integers(-140, 120, (M, K // 128, 1)))).reshape(M, K)
    x = x.astype(f32)
    x[0, 5], x[1, 300], x[1, 301], x[2, 700] = np.nan, np.inf, -np.inf, 3e38
    x[3, :128] = np.array([1, 0x80000001, 0x00400000], np.uint32).view(f32).repeat(43)[:128]
    xin = F.to_bf16_bits(x) if bf16 else x
    q, s = ops.align_w4_groups(cuda(xin), x_is_bf16=bf16)
    wq, ws = F.align_w4_groups(F.bf16_bits_to_f32(xin) if bf16 else x)
    assert same(host(q), wq) and same(host(s), ws)


# ------------------------------------------------------------------------------ fused quantize + GEMV
def fused_case(rng, M, K, Ns, edge_rows=False):
    x = (rng.normal(0, 1, (M, K)) * np.exp2(rng.integers(-40, 40, (M, 1)))).astype(f32)
    if edge_rows and M >= 3:
        x[1] = 0.0                          # zero row: q = 0, s = 0
        x[2, K // 3] = np.inf               # inf row: inv = 0, s = inf -> NaN outputs
        if M >= 4:
            x[3, 1] = np.nan
    mats = []
    for i, N in enumerate(Ns):
        W = rng.integers(-128, 128, (N, K), dtype=np.int8)
        sc = rng.uniform(1e-3, 1e-2, N).astype(f32)
        b = rng.normal(0, 1, N).astype(f32) if i % 2 else None
        act, out = [(ACT_NONE, OUT_FP32), (ACT_SILU, OUT_FP32), (ACT_GELU, OUT_BF16), (ACT_RELU, OUT_INT8)][i % 4]
        mats.append((W, sc, b, act, out, f32(3.0) if out == OUT_INT8 else None))
    return x, mats


@pytest.mark.parametrize("K", [16, 48, 496, 1024, 2048, 3072, 4112, 6912, 9216])
@pytest.mark.parametrize("M", [1, 4])
def test_fused_quant_gemm_matches_separate_ops(K, M):
    rng = np.random.default_rng(K * 10 + M)
    ngroups = {16: 2, 48: 4, 496: 3, 1024: 3, 2048: 1, 3072: 2, 4112: 4, 6912: 2, 9216: 3}[K]
    x, mats = fused_case(rng, M, K, [48, 96, 32, 160][:ngroups], edge_rows=True)
    outs = ops.quant_gemm_rowcol(cuda(x), [(cuda(W), cuda(sc), None if b is None else cuda(b), a, o, osc)
                                           for W, sc, b, a, o, osc in mats], return_q=True)
    q, s = F.quant_rows(x)
    assert same(host(outs[0]), q) and same(host(outs[1]), s)
    for (W, sc, b, a, o, osc), y in zip(mats, outs[2:]):
        want = G.gemm_rowcol(q, s, W, sc, b, act=a, out=o, out_scale=osc)
        assert same(host(y), want), mismatch(host(y), want)


def q8_tie_rows(rng, M, K):
    """Rows whose elements sit on q8 ties (x * inv = k + 1/2 up to one rounding) and at the
    extremes: maxima from 2^-118 (the smallest fast-path maximum) to 2^127, subnormal and zero
    elements, +-amax, and values just inside the maximum."""
    rows = []
    for i in range(M):
        amax = f32(np.ldexp(rng.uniform(1, 2), int(rng.integers(-118, 127)))) if i > 1 else \
            [np.uint32(0x04800000).view(f32), np.uint32(0x7F7FFFFF).view(f32)][i]
        inv = F.fmul(F.Q127, F.recip_f(np.array([amax], f32)))[0]
        with np.errstate(all="ignore"):
            ties = ((rng.integers(-127, 127, K) + f32(0.5)) / inv).astype(f32)
            near = (amax * rng.uniform(-1, 1, K)).astype(f32)
        x = np.where(rng.random(K) < 0.5, ties, near).astype(f32)
        x[~np.isfinite(x)] = 0.0
        x = np.clip(x, -amax, amax).astype(f32)
        x[rng.integers(0, K, 3)] = np.uint32(rng.integers(1, 1 << 23)).view(f32)   # subnormals
        x[0], x[-1] = amax, -amax if K > 1 else amax
        x[rng.integers(0, K, 2)] = -0.0
        rows.append(x)
    return np.stack(rows)


@pytest.mark.parametrize("K", [16, 1024, 2048, 3072])
def test_fused_quantizer_on_q8_ties_and_row_extremes(K):
    """The fast q8 form (rint by the 1.5 * 2^23 rounding constant, no clamp) on the values where a
    wrong rounding or clamp would show: exact ties, +-amax, the smallest and largest fast-path
    maxima; the fused kernel's quantized row and the standalone quantizer against the oracle."""
    rng = np.random.default_rng(K + 77)
    x = q8_tie_rows(rng, 6, K)
    q, s = F.quant_rows(x)
    qg, sg = ops.quant_rows(cuda(x))
    assert same(host(qg), q) and same(host(sg), s)
    W = rng.integers(-128, 128, (96, K), dtype=np.int8)
    sc = rng.uniform(1e-3, 1e-2, 96).astype(f32)
    for m in range(x.shape[0]):
        outs = ops.quant_gemm_rowcol(cuda(x[m:m + 1]), [(cuda(W), cuda(sc))], return_q=True)
        assert same(host(outs[0]), q[m:m + 1]) and same(host(outs[1]), s[m:m + 1]), m
        assert same(host(outs[2]), G.gemm_rowcol(q[m:m + 1], s[m:m + 1], W, sc)), m


@pytest.mark.parametrize("Ns", [[64, 32, 32], [48, 96], [128, 64, 32, 32], [96, 32, 160, 32]])
@pytest.mark.parametrize("K,M", [(1024, 1), (2048, 4), (16, 1)])
def test_fused_equal_row_pieces(Ns, K, M):
    """Matrices of unequal height cut into equal row pieces (their greatest common height, at most 8
    pieces; one grid slice each): every piece's weights, scales, bias and output rows are offset
    from its matrix's, for every output format and with biases and activations."""
    rng = np.random.default_rng(sum(Ns) + K + M)
    x, mats = fused_case(rng, M, K, Ns, edge_rows=True)
    outs = ops.quant_gemm_rowcol(cuda(x), [(cuda(W), cuda(sc), None if b is None else cuda(b), a, o, osc)
                                           for W, sc, b, a, o, osc in mats])
    q, s = F.quant_rows(x)
    for (W, sc, b, a, o, osc), y in zip(mats, outs):
        want = G.gemm_rowcol(q, s, W, sc, b, act=a, out=o, out_scale=osc)
        assert same(host(y), want), (Ns, mismatch(host(y), want))


@pytest.mark.parametrize("Ns,K", [([3072, 3072], 1024), ([2992, 2992], 1024), ([2560, 2560, 512], 512),
                                   ([3000 - 8, 3000 - 8], 768)])
def test_fused_six_rows_per_wave(Ns, K):
    """Launches of 5000-6500 rows at K <= 1024 run six weight rows per wave (the row sums reduced as
    eight with two zero rows, 24 rows per workgroup): full and partial last row blocks."""
    rng = np.random.default_rng(sum(Ns) + K)
    x = rng.normal(0, 1, (1, K)).astype(f32)
    Ws = [rng.integers(-128, 128, (N, K), dtype=np.int8) for N in Ns]
    scs = [rng.uniform(1e-3, 1e-2, N).astype(f32) for N in Ns]
    outs = ops.quant_gemm_rowcol(cuda(x), [(cuda(W), cuda(sc)) for W, sc in zip(Ws, scs)])
    q, s = F.quant_rows(x)
    for W, sc, y in zip(Ws, scs, outs):
        assert same(host(y), G.gemm_rowcol(q, s, W, sc)), (Ns, mismatch(host(y), G.gemm_rowcol(q, s, W, sc)))


def test_fused_qwen3_layer_groups_full_size():
    """q/k/v (2048 + 1024 + 1024 rows) and gate/up (2 x 3072 rows) at K = 1024, and the head."""
    rng = np.random.default_rng(123)
    for Ns in ([2048, 1024, 1024], [3072, 3072], [151936]):
        x = rng.normal(0, 1, (1, 1024)).astype(f32)
        Ws = [rng.integers(-127, 128, (N, 1024), dtype=np.int8) for N in Ns]
        scs = [rng.uniform(1e-3, 1e-2, N).astype(f32) for N in Ns]
        outs = ops.quant_gemm_rowcol(cuda(x), [(cuda(W), cuda(sc)) for W, sc in zip(Ws, scs)])
        q, s = F.quant_rows(x)
        for W, sc, y in zip(Ws, scs, outs):
            want = oracle_rowcol_blocked(q, s, W, sc, rows=37984)
            assert same(host(y), want), (Ns, mismatch(host(y), want))


def test_fused_refuses_aliased_outputs():
    rng = np.random.default_rng(5)
    x = cuda(rng.normal(0, 1, (1, 64)).astype(f32))
    W = cuda(rng.integers(-128, 128, (32, 64), dtype=np.int8))
    sc = cuda(np.ones(32, f32))
    y = torch.zeros((1, 32), device="cuda")
    descs = (ops._lib.W8A8Out * 2)(ops._lib.W8A8Out(W.data_ptr(), sc.data_ptr(), None, y.data_ptr(), 128, 32, 0, 0, 0),
                                   ops._lib.W8A8Out(W.data_ptr(), sc.data_ptr(), None, y.data_ptr(), 128, 32, 0, 0, 0))
    rc = ops._lib.lib().tars_quant_gemm_w8a8(x.data_ptr(), 256, None, 0, None, 1, 64, descs, 2, None)
    assert rc == ops._lib.E_OVERLAP
    assert (host(y) == 0).all()
