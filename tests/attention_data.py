"""Attention inputs shared by the GPU attention tests: values whose fp32 flushes change a result."""
from __future__ import annotations

import numpy as np


def plant_attention_specials(rng, q, kc, vv, kv_heads, hd, v_fp16):
    """Values whose flushes change a result: subnormal K and V elements, K and V columns of tiny
    normals (their products with q or with a probability are subnormal), an infinite q element
    against a subnormal K element (the flushed product is NaN, the unflushed one infinite), and two
    equal K rows whose V values cancel to a subnormal partial sum (2^-100 (1 - (1 - 2^-23)) p).
    The tiny K column 9 is the first step of its 16-lane chain (the chain starts subnormal); the tiny
    K column 25 is the second step of the same lane's chain and the V column 6 turns tiny halfway
    down the keys, so there a normal partial sum absorbs the subnormal products (the unflushed fast
    path's case)."""
    nk = kc.shape[0]
    sub = lambda n: (rng.integers(1, 1 << 23, n, dtype=np.uint32) | (rng.integers(0, 2, n, dtype=np.uint32) << 31)).view(np.float32)
    for kv in range(kv_heads):
        c0 = kv * hd
        kc[rng.integers(0, nk, 6), c0 + rng.integers(0, hd, 6)] = sub(6)
        kc[:, c0 + 9] = rng.normal(0, 1, nk).astype(np.float32) * np.float32(2.0 ** -70)
        q[:, c0 + 9] = np.float32(2.0 ** -60)
        kc[:, c0 + 25] = rng.normal(0, 1, nk).astype(np.float32) * np.float32(2.0 ** -70)
        q[:, c0 + 25] = np.float32(2.0 ** -60)
        if not v_fp16:
            vv[rng.integers(0, nk, 6), c0 + rng.integers(0, hd, 6)] = sub(6)
            vv[:, c0 + 5] = rng.normal(0, 1, nk).astype(np.float32) * np.float32(2.0 ** -124)
            vv[nk // 2:, c0 + 6] = rng.normal(0, 1, nk - nk // 2).astype(np.float32) * np.float32(2.0 ** -124)
            vv[0, c0 + 3], vv[1, c0 + 3] = np.float32(2.0 ** -100), -np.float32(2.0 ** -100) * np.float32(1 - 2.0 ** -23)
        kc[1, c0:c0 + hd] = kc[0, c0:c0 + hd]
    q[0, 7] = np.inf
    kc[nk // 2, 7] = sub(1)[0]
