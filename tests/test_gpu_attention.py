"""tars_attention (opentars_amd.ops.attention) against the oracle's three ops per head, bit for bit:
fdot_nt of the head's q rows with its K head's rows, the causal softmax, fdot_nn with the V rows
(the reference's lowering, tars_mini/llm.py:736-746), and the last head's scores and
probabilities in the shared rows. The shapes cover both forms of the kernel: the split form (up to
4 query rows per K / V head group: Qwen3 decode with 2 query heads per K / V head, Gemma-style 4,
2- to 4-row chunks, long contexts) and one workgroup per head (5 rows, or probabilities past the
split form's LDS). Needs a gfx950 GPU."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from attention_data import plant_attention_specials
from oracle import golden as G
from oracle import numerics as F
from oracle import rowops as R
from opentars_amd import ops
from opentars_amd.contract import OUT_BF16, OUT_FP32, OUT_INT8

pytestmark = pytest.mark.gpu
f32 = np.float32


def bits(a) -> np.ndarray:
    a = np.asarray(a)
    return a.view(np.uint32) if a.dtype == f32 else a.view(np.uint16) if a.itemsize == 2 else a.view(np.uint8)


def oracle_attention(q, kc, vval, heads, kv_heads, hd, causal_k, out, osc):
    """Per head in order: scores, causal softmax, P V, converted; the last head's scores and
    probabilities (what the shared buffers hold at the end)."""
    M, nk = q.shape[0], kc.shape[0]
    grp = heads // kv_heads
    valid = [min(nk, causal_k + m) if causal_k > 0 else nk for m in range(M)]
    att = []
    for h in range(heads):
        kv = h // grp
        s = R.fdot_nt(q[:, h * hd:(h + 1) * hd], kc[:, kv * hd:(kv + 1) * hd])
        p = R.softmax_rows_causal(s, valid)
        att.append(G.convert(R.fdot_nn(p, vval[:, kv * hd:(kv + 1) * hd]), out, osc))
    return np.concatenate(att, axis=1), s, p


def layer(seed, heads, kv_heads, hd, M, t0, v_fp16, specials):
    rng = np.random.default_rng(seed)
    nk = (t0 + M + 15) // 16 * 16
    q = rng.normal(0, 0.3, (M, heads * hd)).astype(f32)
    kc = rng.normal(0, 1, (nk, kv_heads * hd)).astype(f32)
    vv = rng.normal(0, 1, (nk, kv_heads * hd)).astype(f32)
    if specials:
        plant_attention_specials(rng, q, kc, vv, kv_heads, hd, v_fp16)
    vdev = vv.astype(np.float16).view(np.uint16) if v_fp16 else vv
    vval = F.from_fp16_bits(vdev) if v_fp16 else vv
    return q, kc, vdev, vval, nk


def run_case(heads, kv_heads, hd, M, t0, v_fp16, out, specials=False):
    q, kc, vdev, vval, nk = layer(heads * 1000 + hd + M * 7 + t0, heads, kv_heads, hd, M, t0, v_fp16, specials)
    osc = f32(4.0) if out == OUT_INT8 else None
    sc = torch.full((M, nk), float("nan"), device="cuda")
    pr = torch.full((M, nk), float("nan"), device="cuda")
    got = ops.attention(q, kc, vdev, heads, kv_heads, causal_k=t0 + 1, v_fp16=v_fp16, out=out, out_scale=osc,
                        sc=sc, pr=pr)
    want, s_last, p_last = oracle_attention(q, kc, vval, heads, kv_heads, hd, t0 + 1, out, osc)
    g, w = bits(got), bits(want)
    bad = np.argwhere(g != w)
    assert len(bad) == 0, f"att: {len(bad)} differ, first at {tuple(bad[0])}: {g[tuple(bad[0])]:#x} vs {w[tuple(bad[0])]:#x}"
    assert np.array_equal(bits(sc.cpu().numpy()), bits(s_last)), "last head's scores"
    assert np.array_equal(bits(pr.cpu().numpy()), bits(p_last)), "last head's probabilities"


CASES = [
    (16, 8, 128, 1, 250, False, OUT_FP32),   # Qwen3-0.6B decode: split, 2 query heads per K / V head
    (4, 1, 256, 1, 37, True, OUT_FP32),      # head size 256, fp16 V, 4 query heads per K / V head
    (8, 4, 64, 2, 100, False, OUT_BF16),     # a 2-row chunk: 4 query rows per group
    (6, 6, 128, 3, 60, False, OUT_INT8),     # 3 rows, no sharing
    (2, 1, 128, 4, 500, False, OUT_FP32),    # 4 rows: the group split back to single heads
    (2, 1, 64, 5, 30, False, OUT_FP32),      # 5 rows: one workgroup per head
    (2, 1, 64, 1, 2000, True, OUT_FP32),     # 2016 keys: 128 keys per scores workgroup
    (2, 2, 128, 1, 4070, False, OUT_FP32),   # 4080 keys, the most either form takes
    (4, 2, 128, 2, 3000, False, OUT_FP32),   # probabilities past the split form's LDS: one per head
    (3, 3, 64, 1, 0, False, OUT_FP32),       # the first position: one valid key of 16
]


@pytest.mark.parametrize("heads,kv_heads,hd,M,t0,v_fp16,out", CASES)
def test_attention_matches_the_oracle(heads, kv_heads, hd, M, t0, v_fp16, out):
    run_case(heads, kv_heads, hd, M, t0, v_fp16, out)


@pytest.mark.parametrize("heads,kv_heads,hd,M,t0,v_fp16", [
    (16, 8, 128, 1, 250, False),
    (4, 2, 128, 2, 40, False),
    (2, 1, 64, 1, 300, True),
    (2, 1, 256, 1, 20, False),
    (2, 1, 64, 5, 30, False),
])
def test_attention_with_values_the_flushes_change(heads, kv_heads, hd, M, t0, v_fp16):
    run_case(heads, kv_heads, hd, M, t0, v_fp16, OUT_FP32, specials=True)


def test_attention_twice_in_a_row_and_without_the_shared_rows():
    """Two calls on one stream share the device scratch: the second (fewer keys, other heads)
    must not see the first's scores; sc / pr left out."""
    for heads, kv_heads, t0 in ((16, 8, 250), (4, 2, 40)):
        q, kc, vdev, vval, nk = layer(t0, heads, kv_heads, 128, 1, t0, False, False)
        got = ops.attention(q, kc, vdev, heads, kv_heads, causal_k=t0 + 1)
        want = oracle_attention(q, kc, vval, heads, kv_heads, 128, t0 + 1, OUT_FP32, None)[0]
        assert np.array_equal(bits(got), bits(want))


def test_attention_on_two_streams_at_once():
    """Calls on two streams overlap in time: each stream's split form has its own scores scratch,
    so every call's output matches the oracle (one shared scratch would mix their scores)."""
    data = []
    for i, (heads, kv_heads, t0) in enumerate(((16, 8, 250), (16, 8, 170))):
        q, kc, vdev, vval, nk = layer(700 + i, heads, kv_heads, 128, 1, t0, False, False)
        want = oracle_attention(q, kc, vval, heads, kv_heads, 128, t0 + 1, OUT_FP32, None)[0]
        dev = [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (q, kc, vdev)]
        data.append((dev, want, heads, kv_heads, t0))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[], []]
    torch.cuda.synchronize()
    for rep in range(16):
        for j in (0, 1):
            (q, kc, v), _, heads, kv_heads, t0 = data[j]
            with torch.cuda.stream(streams[j]):
                att = torch.empty((1, heads * 128), dtype=torch.float32, device="cuda")
                ops.attention(q, kc, v, heads, kv_heads, causal_k=t0 + 1, att=att)
                outs[j].append(att)
    torch.cuda.synchronize()
    for j in (0, 1):
        for rep, att in enumerate(outs[j]):
            assert np.array_equal(bits(att.cpu().numpy()), bits(data[j][1])), f"stream {j}, call {rep}"


def test_attention_refusals():
    q = torch.zeros((1, 256), device="cuda")
    kc = torch.zeros((32, 128), device="cuda")
    with pytest.raises(ops.TarsError):
        ops.attention(q, kc, kc, 2, 1, att=q)                   # the output is the q rows
    with pytest.raises(ValueError):
        ops.attention(q, kc, kc, 3, 1)                          # 3 heads over 256 columns
    with pytest.raises(ops.TarsError):
        ops.attention(torch.zeros((1, 96), device="cuda"), torch.zeros((32, 48), device="cuda"),
                      torch.zeros((32, 48), device="cuda"), 2, 1)   # head size 48
