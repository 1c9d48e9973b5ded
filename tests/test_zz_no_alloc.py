"""tars_attention_noalloc (the attention entry point that allocates nothing: its scores scratch is
a static device array) against tars_attention through the C ABI, bit for bit: two calls in a row
on one stream, the second with fewer heads and keys (the shared array keeps the first call's
scores, which the second must not see), and the refusal of a shape past the array. Needs a gfx950
GPU."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from opentars_amd import _lib

pytestmark = pytest.mark.gpu


def call(fn, q, kc, vc, att, sc, pr, heads, kv_heads, hd, M, nk, t0):
    grp = heads // kv_heads
    arr = lambda vals: (ctypes.c_void_p * heads)(*vals)
    qp = arr([q.data_ptr() + 4 * h * hd for h in range(heads)])
    kp = arr([kc.data_ptr() + 4 * (h // grp) * hd for h in range(heads)])
    vp = arr([vc.data_ptr() + 4 * (h // grp) * hd for h in range(heads)])
    ap = arr([att.data_ptr() + 4 * h * hd for h in range(heads)])
    return fn(qp, 4 * heads * hd, kp, 4 * kv_heads * hd, vp, 4 * kv_heads * hd, 0, ap, 4 * heads * hd, 0, 0,
              sc.data_ptr(), 4 * nk, pr.data_ptr(), 4 * nk, heads, M, nk, hd, t0 + 1,
              torch.cuda.current_stream().cuda_stream)


def layer(seed, heads, kv_heads, hd, M, t0):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    nk = (t0 + M + 15) // 16 * 16
    q = torch.randn((M, heads * hd), device="cuda", generator=g) * 0.3
    kc = torch.randn((nk, kv_heads * hd), device="cuda", generator=g)
    vc = torch.randn((nk, kv_heads * hd), device="cuda", generator=g)
    return q, kc, vc, nk


def outputs(M, heads, hd, nk):
    return (torch.full((M, heads * hd), float("nan"), device="cuda"), torch.full((M, nk), float("nan"), device="cuda"),
            torch.full((M, nk), float("nan"), device="cuda"))


def test_noalloc_attention_matches_the_allocating_entry_point():
    lib = _lib.lib()
    for seed, (heads, kv_heads, hd, M, t0) in enumerate(((16, 8, 128, 1, 700), (4, 2, 128, 2, 60))):
        q, kc, vc, nk = layer(seed, heads, kv_heads, hd, M, t0)
        want, want_sc, want_pr = outputs(M, heads, hd, nk)
        got, got_sc, got_pr = outputs(M, heads, hd, nk)
        assert call(lib.tars_attention, q, kc, vc, want, want_sc, want_pr, heads, kv_heads, hd, M, nk, t0) == 0
        assert call(lib.tars_attention_noalloc, q, kc, vc, got, got_sc, got_pr, heads, kv_heads, hd, M, nk, t0) == 0, \
            _lib.last_error()
        torch.cuda.synchronize()
        for g, w in ((got, want), (got_sc, want_sc), (got_pr, want_pr)):
            assert torch.equal(g.view(torch.int32), w.view(torch.int32)), (heads, M, t0)


def test_noalloc_attention_refuses_a_shape_past_the_static_array():
    lib = _lib.lib()
    heads, kv_heads, hd, M, t0 = 32, 32, 64, 3, 4000           # 32 * 3 * 4016 floats > 262144
    q, kc, vc, nk = layer(9, heads, kv_heads, hd, M, t0)
    att, sc, pr = outputs(M, heads, hd, nk)
    assert call(lib.tars_attention_noalloc, q, kc, vc, att, sc, pr, heads, kv_heads, hd, M, nk, t0) == _lib.E_RANGE
    torch.cuda.synchronize()
    assert torch.isnan(att).all()                               # nothing written
