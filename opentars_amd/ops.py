"""The golden model's matrix ops on MI355X, with the golden model's op signatures.

Each function runs the HIP kernels through the C ABI (libopentars_amd.so) and returns results
bit-identical to the golden model (tars_mini/golden.py, tars_mini/numerics.py):

  quant_rows(x)                          numerics.quant_rows            numerics.py:383-390
  gemm_rowcol(q, srow, W, scol, ...)     Machine._gemm (QM_ROWCOL etc.) golden.py:326-349
  gemm_rowcol_ksplit(q, srow, Ws, scol)  lin_k blocks + ELT_ADD chain   llm.py:303-321, 627-635
  align_w4_groups(x)                     numerics.align_w4_groups       numerics.py:55-98
  gemm_w4(x, Wp, ws, ...)                Machine._gemm_w4               golden.py:295-324
  softmax_rows(x) / softmax_rows_causal  Machine._row (ROW_SOFTMAX)     numerics.py:328-333, 362-371
  layernorm_rows / rmsnorm_rows /        Machine._row (norms)           numerics.py:341-358, 374-380
    l2norm_rows(x, gamma, beta, eps)
  relu(x, act)                           Machine._relu                  golden.py:351-356
  elt(op, a, b, ...)                     Machine._elt                   golden.py:393-418
  rope_rows(x, tab, rows_per_pos, rot)   Machine._rope                  numerics.py:412-424
  fdot_nt(a, b) / fdot_nn(a, b)          Machine._fdot                  numerics.py:393-409
  embed_rows(table, ids, scale)          the runtime's embedding lookup tars_board.py:298-314

Inputs are torch tensors on the GPU (results stay there, stream-ordered on the current stream),
or numpy arrays (copied in; results come back as numpy after a synchronize, which is what
golden-style callers expect). 2-D operands may be row-strided views whose rows are contiguous.
There is no CPU path: without the built library or a GPU every call raises.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import numpy as np
import torch

from . import _lib
from .contract import (ACT_NONE, DT_BF16, DT_FP32, ESIZE, OUT_BF16, OUT_FP16, OUT_FP32, OUT_INT8, W4_GROUP)


class TarsError(RuntimeError):
    """A call the contract rejects: .code is the library status (E_FIELD, E_ALIGN, ...)."""

    def __init__(self, code: int, message: str):
        self.code = code
        self.name = _lib.STATUS_NAMES.get(code, str(code))
        super().__init__(f"{self.name}: {message}")


class ContractError(TarsError):
    """An output overlapping an input (the golden model's ContractError, golden.py:18-19, 473-479)."""


def _check(rc: int) -> None:
    if rc == _lib.OK:
        return
    msg = _lib.last_error()
    if rc == _lib.E_OVERLAP:
        raise ContractError(rc, msg)
    raise TarsError(rc, msg)


def _device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("opentars_amd needs a ROCm GPU (gfx950); there is no CPU fallback")
    return torch.device("cuda", torch.cuda.current_device())


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


_NP_TO_TORCH = {np.dtype(np.int8): torch.int8, np.dtype(np.uint8): torch.uint8,
                np.dtype(np.float32): torch.float32, np.dtype(np.int16): torch.int16,
                np.dtype(np.uint16): torch.int16, np.dtype(np.int32): torch.int32}


def _to_dev(a, dtype: torch.dtype | None = None) -> torch.Tensor:
    """A torch device tensor for `a` (numpy arrays are copied; uint16 bits travel as int16)."""
    if isinstance(a, torch.Tensor):
        if not a.is_cuda:
            raise ValueError("torch inputs must already live on the GPU")
        return a
    arr = np.ascontiguousarray(a)
    if arr.dtype == np.uint16:
        arr = arr.view(np.int16)
    t = torch.from_numpy(arr).to(_device())
    return t if dtype is None else t.view(dtype)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _ld(t: torch.Tensor) -> int:
    """Row stride in bytes of a 2-D tensor whose rows are contiguous."""
    if t.dim() != 2 or (t.shape[1] > 1 and t.stride(1) != 1):
        raise ValueError("expected a 2-D tensor with contiguous rows")
    return t.stride(0) * t.element_size()


def _vec(t: torch.Tensor, n: int, what: str) -> torch.Tensor:
    if t.dim() != 1 or t.numel() != n or (n > 1 and t.stride(0) != 1):
        raise ValueError(f"{what} must be a contiguous vector of {n} elements")
    return t


def _numpy_mode(*args) -> bool:
    return any(isinstance(a, np.ndarray) for a in args)


def _out_dtype(out: int) -> torch.dtype:
    return {OUT_FP32: torch.float32, OUT_BF16: torch.bfloat16, OUT_INT8: torch.int8,
            OUT_FP16: torch.int16}.get(out, torch.uint8)


def _f32_bits(v) -> int:
    return int(np.asarray(v, np.float32).reshape(()).view(np.uint32))


def _finish(numpy_mode: bool, *ts: torch.Tensor):
    if not numpy_mode:
        return ts if len(ts) > 1 else ts[0]
    torch.cuda.synchronize()
    outs = []
    for t in ts:
        if t.dtype == torch.bfloat16:
            outs.append(t.view(torch.int16).cpu().numpy().view(np.uint16))
        elif t.dtype == torch.int16:                       # binary16 bits
            outs.append(t.cpu().numpy().view(np.uint16))
        else:
            outs.append(t.cpu().numpy())
    return tuple(outs) if len(outs) > 1 else outs[0]


def quant_rows(x, q: torch.Tensor | None = None, s: torch.Tensor | None = None):
    """Per-token INT8: (q int8 [M, K], s fp32 [M]) with amax = max|x|, q = q8(x, 127 * recip(amax)),
    s = amax * fp32(1/127) (numerics.py:383-390)."""
    npm = _numpy_mode(x)
    xt = _to_dev(x)
    if xt.dtype != torch.float32 or xt.dim() != 2:
        raise ValueError("quant_rows needs fp32 [M, K]")
    M, K = xt.shape
    q = torch.empty((M, K), dtype=torch.int8, device=xt.device) if q is None else q
    s = torch.empty((M,), dtype=torch.float32, device=xt.device) if s is None else s
    _vec(s, M, "s")
    _check(_lib.lib().tars_quant_rows(xt.data_ptr(), _ld(xt), q.data_ptr(), _ld(q), s.data_ptr(), M, K, _stream()))
    return _finish(npm, q, s)


def gemm_rowcol(q, srow, W, scol, bias=None, act: int = ACT_NONE, out: int = OUT_FP32,
                out_scale=None, y: torch.Tensor | None = None):
    """W8A8 with the golden epilogue: convert(act(((i2f(q @ W^T) * srow) * scol) + bias)).
    srow None: no row scale (QM_CHANNEL); scol of one element: one scale for all (QM_TENSOR)."""
    npm = _numpy_mode(q, srow, W, scol, bias)
    qt, Wt, st = _to_dev(q, torch.int8), _to_dev(W, torch.int8), _to_dev(scol, torch.float32)
    rt = None if srow is None else _to_dev(srow, torch.float32)
    bt = None if bias is None else _to_dev(bias, torch.float32)
    M, K = qt.shape
    N = Wt.shape[0]
    if Wt.dim() != 2 or Wt.shape[1] != K or not Wt.is_contiguous():
        raise ValueError("W must be a dense [N, K] int8 matrix")
    if rt is not None:
        _vec(rt, M, "srow")
    if bt is not None:
        _vec(bt, N, "bias")
    _vec(st, st.numel(), "scol")
    y = torch.empty((M, N), dtype=_out_dtype(out), device=qt.device) if y is None else y
    osb = _f32_bits(out_scale) if out == OUT_INT8 else 0
    _check(_lib.lib().tars_gemm_w8a8(qt.data_ptr(), _ld(qt), _ptr(rt), Wt.data_ptr(), st.data_ptr(), st.numel(),
                                     _ptr(bt), y.data_ptr(), _ld(y), M, N, K, act, out, osb, _stream()))
    return _finish(npm, y)


def quant_gemm_rowcol(x, mats: Sequence, return_q: bool = False):
    """Fused per-token quantization + W8A8 for up to 4 matrices sharing it (q/k/v, gate/up):
    each entry of `mats` is (W, scol) or (W, scol, bias, act, out, out_scale). Returns the list of
    outputs (and (q, s) first when return_q). Bit-identical to quant_rows + gemm_rowcol per matrix
    (llm.py:711-731: one ROW_QUANT feeding several QM_ROWCOL GEMMs)."""
    flat = [x] + [a for m in mats for a in m[:3]]
    npm = _numpy_mode(*flat)
    xt = _to_dev(x, torch.float32)
    if xt.dtype != torch.float32 or xt.dim() != 2:
        raise ValueError("x must be fp32 [M, K]")
    M, K = xt.shape
    if not 1 <= len(mats) <= 4:
        raise ValueError("1 to 4 matrices")
    descs, ys, keep = (_lib.W8A8Out * len(mats))(), [], []
    for i, m in enumerate(mats):
        W, scol = m[0], m[1]
        bias = m[2] if len(m) > 2 else None
        act = m[3] if len(m) > 3 else ACT_NONE
        out = m[4] if len(m) > 4 else OUT_FP32
        osc = m[5] if len(m) > 5 else None
        Wt, st = _to_dev(W, torch.int8), _to_dev(scol, torch.float32)
        bt = None if bias is None else _to_dev(bias, torch.float32)
        N = Wt.shape[0]
        if Wt.dim() != 2 or Wt.shape[1] != K or not Wt.is_contiguous():
            raise ValueError("W must be a dense [N, K] int8 matrix")
        _vec(st, N, "scol")
        if bt is not None:
            _vec(bt, N, "bias")
        y = torch.empty((M, N), dtype=_out_dtype(out), device=xt.device)
        keep += [Wt, st, bt]
        ys.append(y)
        descs[i] = _lib.W8A8Out(Wt.data_ptr(), st.data_ptr(), _ptr(bt), y.data_ptr(), _ld(y), N, act, out,
                                _f32_bits(osc) if out == OUT_INT8 else 0)
    q = torch.empty((M, K), dtype=torch.int8, device=xt.device) if return_q else None
    s = torch.empty((M,), dtype=torch.float32, device=xt.device) if return_q else None
    _check(_lib.lib().tars_quant_gemm_w8a8(xt.data_ptr(), _ld(xt), _ptr(q), K if q is not None else 0, _ptr(s),
                                           M, K, descs, len(mats), _stream()))
    res = ([q, s] if return_q else []) + ys
    out_ = _finish(npm, *res)
    return list(out_) if isinstance(out_, tuple) else [out_]


def gemm_rowcol_ksplit(q, srow, blocks: Sequence, scol, y: torch.Tensor | None = None):
    """K split into blocks W_i [N, K_i] over consecutive column ranges of q, sharing srow and scol:
    per-block W8A8 partials in fp32, added in block order (llm.py:627-635, golden.py:411-412)."""
    npm = _numpy_mode(q, srow, scol, *blocks)
    qt, st = _to_dev(q, torch.int8), _to_dev(scol, torch.float32)
    rt = None if srow is None else _to_dev(srow, torch.float32)
    Ws = [_to_dev(w, torch.int8) for w in blocks]
    M = qt.shape[0]
    N = Ws[0].shape[0]
    for w in Ws:
        if w.dim() != 2 or w.shape[0] != N or not w.is_contiguous():
            raise ValueError("every block must be a dense [N, K_i] int8 matrix")
    if sum(w.shape[1] for w in Ws) != qt.shape[1]:
        raise ValueError("the blocks must cover q's columns")
    if rt is not None:
        _vec(rt, M, "srow")
    _vec(st, N, "scol")
    y = torch.empty((M, N), dtype=torch.float32, device=qt.device) if y is None else y
    nb = len(Ws)
    ptrs = (ctypes.c_void_p * nb)(*[w.data_ptr() for w in Ws])
    ks = (ctypes.c_int32 * nb)(*[w.shape[1] for w in Ws])
    _check(_lib.lib().tars_gemm_w8a8_ksplit(qt.data_ptr(), _ld(qt), _ptr(rt), ptrs, ks, nb, st.data_ptr(),
                                            y.data_ptr(), _ld(y), M, N, _stream()))
    return _finish(npm, y)


def _w4_act(x, x_is_bf16: bool) -> tuple[torch.Tensor, int]:
    if isinstance(x, torch.Tensor) and x.dtype == torch.bfloat16:
        return x, DT_BF16
    if x_is_bf16:
        return _to_dev(x, torch.int16), DT_BF16
    xt = _to_dev(x, torch.float32)
    if xt.dtype != torch.float32:
        raise ValueError("W4A16 activations are fp32 or bf16")
    return xt, DT_FP32


def align_w4_groups(x, x_is_bf16: bool = False):
    """Block-FP alignment: (int16 mantissas [M, K], fp32 group scales [M, K/128]) (numerics.py:55-98)."""
    npm = _numpy_mode(x)
    xt, dt = _w4_act(x, x_is_bf16)
    M, K = xt.shape
    q = torch.empty((M, K), dtype=torch.int16, device=xt.device)
    s = torch.empty((M, max(K // W4_GROUP, 1)), dtype=torch.float32, device=xt.device)
    _check(_lib.lib().tars_align_w4(xt.data_ptr(), _ld(xt), dt, q.data_ptr(), _ld(q), s.data_ptr(), _ld(s),
                                    M, K, _stream()))
    return _finish(npm, q, s)


def gemm_w4(x, Wp, ws, bias=None, act: int = ACT_NONE, out: int = OUT_FP32, out_scale=None,
            y: torch.Tensor | None = None, x_is_bf16: bool = False):
    """W4A16 (golden.py:295-324): x fp32/bf16 [M, K]; Wp uint8 [N, K/2] (low nibble = even k);
    ws binary16 bits [N, K/128]; four fp32 banks over the group terms, then bias, act, convert."""
    npm = _numpy_mode(x, Wp, ws, bias)
    xt, dt = _w4_act(x, x_is_bf16)
    Wt = _to_dev(Wp, torch.uint8)
    wst = _to_dev(ws)
    if wst.dtype not in (torch.int16, torch.float16) and not (hasattr(torch, "uint16") and wst.dtype == torch.uint16):
        raise ValueError("ws must hold binary16 bits")
    bt = None if bias is None else _to_dev(bias, torch.float32)
    M, K = xt.shape
    N = Wt.shape[0]
    if Wt.dim() != 2 or Wt.shape[1] * 2 != K or not Wt.is_contiguous():
        raise ValueError("Wp must be a dense [N, K/2] uint8 matrix")
    if tuple(wst.shape) != (N, K // W4_GROUP) or not wst.is_contiguous():
        raise ValueError("ws must be a dense [N, K/128] matrix")
    if bt is not None:
        _vec(bt, N, "bias")
    y = torch.empty((M, N), dtype=_out_dtype(out), device=xt.device) if y is None else y
    osb = _f32_bits(out_scale) if out == OUT_INT8 else 0
    _check(_lib.lib().tars_gemm_w4a16(xt.data_ptr(), _ld(xt), dt, Wt.data_ptr(), wst.data_ptr(), _ptr(bt),
                                      y.data_ptr(), _ld(y), M, N, K, act, out, osb, _stream()))
    return _finish(npm, y)


# ---------------------------------------------------------------- fp32 row / elementwise / dot ops
ROW_SOFTMAX, ROW_LAYERNORM, ROW_RMSNORM, ROW_L2NORM = 0, 1, 2, 3
ELT_MUL, ELT_ADD, ELT_MULADD, ELT_SUB = 0, 1, 2, 3
BM_DENSE, BM_ROW, BM_COL, BM_SCALAR = 0, 1, 2, 3


def _f32_rows(x, what: str) -> torch.Tensor:
    t = _to_dev(x)
    if t.dtype != torch.float32 or t.dim() != 2:
        raise ValueError(f"{what} must be fp32 [M, N]")
    return t


def _half_rows(x, what: str) -> torch.Tensor:
    """binary16 rows as int16 bits (numpy uint16 / torch float16 or int16)."""
    t = _to_dev(x)
    if t.dtype == torch.float16:
        t = t.view(torch.int16)
    if t.dtype != torch.int16 or t.dim() != 2:
        raise ValueError(f"{what} must be binary16 [rows, cols]")
    return t


def _out(y, M: int, N: int, out: int, like: torch.Tensor) -> torch.Tensor:
    return torch.empty((M, N), dtype=_out_dtype(out), device=like.device) if y is None else y


def _row_op(x, fn: int, gamma=None, beta=None, eps=0.0, causal_k: int = 0, valid=None, out: int = OUT_FP32,
            out_scale=None, y=None):
    npm = _numpy_mode(x, gamma, beta, valid)
    xt = _f32_rows(x, "x")
    M, N = xt.shape
    gt = None if gamma is None else _vec(_to_dev(gamma, torch.float32), N, "gamma")
    bt = None if beta is None else _vec(_to_dev(beta, torch.float32), N, "beta")
    vt = None if valid is None else _vec(_to_dev(np.asarray(valid, np.int32) if not isinstance(valid, torch.Tensor)
                                                 else valid, torch.int32), M, "valid")
    y = _out(y, M, N, out, xt)
    eb = _f32_bits(eps) if fn != ROW_SOFTMAX else 0
    osb = _f32_bits(out_scale) if out == OUT_INT8 else 0
    _check(_lib.lib().tars_row_op(xt.data_ptr(), _ld(xt), fn, _ptr(gt), _ptr(bt), eb, causal_k, _ptr(vt),
                                  y.data_ptr(), _ld(y), out, osb, M, N, _stream()))
    return _finish(npm, y)


def softmax_rows(x, out: int = OUT_FP32, out_scale=None, y=None, causal_k: int = 0):
    """mx = row max; e = exp(x + -mx); y = e * recip(sum16(e)) (numerics.py:328-333). causal_k > 0:
    row m sees its first min(N, causal_k + m) elements (the ROW_SOFTMAX descriptor's K rule,
    golden.py:366-367)."""
    return _row_op(x, ROW_SOFTMAX, causal_k=causal_k, out=out, out_scale=out_scale, y=y)


def softmax_rows_causal(x, valid, out: int = OUT_FP32, out_scale=None, y=None):
    """Softmax over the first valid[m] (1..N) elements of row m; the rest +0 (numerics.py:362-371)."""
    return _row_op(x, ROW_SOFTMAX, valid=valid, out=out, out_scale=out_scale, y=y)


def layernorm_rows(x, gamma, beta, eps, out: int = OUT_FP32, out_scale=None, y=None):
    """numerics.py:341-350."""
    return _row_op(x, ROW_LAYERNORM, gamma, beta, eps, out=out, out_scale=out_scale, y=y)


def rmsnorm_rows(x, gamma, beta, eps, out: int = OUT_FP32, out_scale=None, y=None):
    """numerics.py:353-358."""
    return _row_op(x, ROW_RMSNORM, gamma, beta, eps, out=out, out_scale=out_scale, y=y)


def l2norm_rows(x, gamma, beta, eps, out: int = OUT_FP32, out_scale=None, y=None):
    """numerics.py:374-380."""
    return _row_op(x, ROW_L2NORM, gamma, beta, eps, out=out, out_scale=out_scale, y=y)


def relu(x, act: int, out: int = OUT_FP32, out_scale=None, y=None):
    """act(x) converted to the output format (golden.py:351-356)."""
    npm = _numpy_mode(x)
    xt = _f32_rows(x, "x")
    M, N = xt.shape
    y = _out(y, M, N, out, xt)
    osb = _f32_bits(out_scale) if out == OUT_INT8 else 0
    _check(_lib.lib().tars_relu(xt.data_ptr(), _ld(xt), act, y.data_ptr(), _ld(y), out, osb, M, N, _stream()))
    return _finish(npm, y)


def elt(op: int, a, b, bmode: int = BM_DENSE, c=None, act: int = ACT_NONE, out: int = OUT_FP32, out_scale=None,
        y=None, a_fp16: bool = False, a_row: bool = False, shape: tuple | None = None):
    """y = act(a) * b | act(a) + b | act(a) + -b | c + act(a) * b (golden.py:393-418). a: fp32
    [M, N] (a_fp16: binary16 bits; a_row: one row [1, N] for every m); b: fp32 [M, N] (DENSE) or a
    vector of N (ROW), M (COL) or 1 (SCALAR) values; c: MULADD's addend [M, N] in the output's
    float format; y may be a or c itself (in place). shape=(M, N) when a is a broadcast row."""
    npm = _numpy_mode(a, b, c)
    at = _half_rows(a, "a") if a_fp16 else _f32_rows(a, "a")
    M, N = shape if shape is not None else at.shape
    bt = _to_dev(b, torch.float32)
    if bmode == BM_DENSE:
        if bt.dim() != 2:
            raise ValueError("a dense b must be [M, N]")
        ldb = _ld(bt)
    else:
        bt = bt.reshape(-1)
        ldb = 0
    ct = None
    if c is not None:
        ct = _half_rows(c, "c") if out == OUT_FP16 else _f32_rows(c, "c")
    y = _out(y, M, N, out, at)
    osb = _f32_bits(out_scale) if out == OUT_INT8 else 0
    _check(_lib.lib().tars_elt(at.data_ptr(), _ld(at), int(a_fp16), int(a_row), bt.data_ptr(), ldb, bmode,
                               _ptr(ct), 0 if ct is None else _ld(ct), op, act, y.data_ptr(), _ld(y), out, osb, M, N,
                               _stream()))
    return _finish(npm, y)


def rope_rows(x, tab, rows_per_pos: int, rot: int, out: int = OUT_FP32, out_scale=None, y=None):
    """Rotary embedding of the first rot elements of each row, table row m // rows_per_pos
    (numerics.py:412-424)."""
    npm = _numpy_mode(x, tab)
    xt = _f32_rows(x, "x")
    tt = _f32_rows(tab, "tab")
    M, N = xt.shape
    if tt.shape[1] != rot or not tt.is_contiguous() or tt.shape[0] < (M - 1) // rows_per_pos + 1:
        raise ValueError("tab must be a dense [positions, rot] fp32 table covering every row")
    y = _out(y, M, N, out, xt)
    osb = _f32_bits(out_scale) if out == OUT_INT8 else 0
    _check(_lib.lib().tars_rope(xt.data_ptr(), _ld(xt), tt.data_ptr(), rows_per_pos, rot, y.data_ptr(), _ld(y), out,
                                osb, M, N, _stream()))
    return _finish(npm, y)


def _fdot(a, b, nn: bool, b_fp16: bool, out: int, out_scale, y):
    npm = _numpy_mode(a, b)
    at = _f32_rows(a, "a")
    bt = _half_rows(b, "b") if b_fp16 else _f32_rows(b, "b")
    M, K = at.shape
    N = bt.shape[1] if nn else bt.shape[0]
    if (bt.shape[0] if nn else bt.shape[1]) != K:
        raise ValueError("a and b disagree on K")
    y = _out(y, M, N, out, at)
    osb = _f32_bits(out_scale) if out == OUT_INT8 else 0
    _check(_lib.lib().tars_fdot(at.data_ptr(), _ld(at), bt.data_ptr(), _ld(bt), int(nn), int(b_fp16), y.data_ptr(),
                                _ld(y), out, osb, M, N, K, _stream()))
    return _finish(npm, y)


def fdot_nt(a, b, out: int = OUT_FP32, out_scale=None, y=None):
    """y[m][n] = sum16 over k of a[m][k] * b[n][k] (numerics.py:393-399)."""
    return _fdot(a, b, False, False, out, out_scale, y)


def fdot_nn(a, b, b_fp16: bool = False, out: int = OUT_FP32, out_scale=None, y=None):
    """y[m][n] = ((+0 + a[m][0] b[0][n]) + a[m][1] b[1][n]) + ... (numerics.py:402-409); b may be
    binary16 bits (the fp16 KV state)."""
    return _fdot(a, b, True, b_fp16, out, out_scale, y)


def attention(q, kcache, vcache, heads: int, kv_heads: int, causal_k: int = 0, v_fp16: bool = False,
              out: int = OUT_FP32, out_scale=None, sc=None, pr=None, att=None):
    """One layer's attention as the reference lowers it (tars_mini/llm.py:736-746): for every query
    head h, with K / V head h // (heads // kv_heads), fdot_nt of its q rows with the K rows, the
    causal softmax (causal_k: the descriptor's K rule; 0 = every key valid), fdot_nn with the V rows
    into its output columns; sc / pr (fp32 [M, nk], optional) receive the last head's scores and
    probabilities, as the shared buffers of the three ops do. q fp32 [M, heads * hd]; kcache fp32
    [nk, kv_heads * hd]; vcache the same, fp32 or binary16 bits (v_fp16). Returns att
    [M, heads * hd] in format out (or fills the given one)."""
    npm = _numpy_mode(q, kcache, vcache)
    qt = _f32_rows(q, "q")
    kt = _f32_rows(kcache, "kcache")
    vt = _half_rows(vcache, "vcache") if v_fp16 else _f32_rows(vcache, "vcache")
    M, nk = qt.shape[0], kt.shape[0]
    if heads < 1 or kv_heads < 1 or heads % kv_heads or qt.shape[1] % heads:
        raise ValueError("heads must be a multiple of kv_heads and divide q's columns")
    hd = qt.shape[1] // heads
    if kt.shape[1] != kv_heads * hd or vt.shape != (nk, kv_heads * hd):
        raise ValueError("kcache and vcache must be [nk, kv_heads * hd]")
    att = _out(att, M, heads * hd, out, qt)
    ve, oe, grp = (2 if v_fp16 else 4), ESIZE[out], heads // kv_heads
    arr = lambda vals: (ctypes.c_void_p * heads)(*vals)
    qp = arr([qt.data_ptr() + 4 * h * hd for h in range(heads)])
    kp = arr([kt.data_ptr() + 4 * (h // grp) * hd for h in range(heads)])
    vp = arr([vt.data_ptr() + ve * (h // grp) * hd for h in range(heads)])
    ap = arr([att.data_ptr() + oe * h * hd for h in range(heads)])
    osb = _f32_bits(out_scale) if out == OUT_INT8 else 0
    _check(_lib.lib().tars_attention(qp, _ld(qt), kp, _ld(kt), vp, _ld(vt), int(v_fp16), ap, _ld(att), out, osb,
                                     _ptr(sc), 0 if sc is None else _ld(sc), _ptr(pr), 0 if pr is None else _ld(pr),
                                     heads, M, nk, hd, causal_k, _stream()))
    return _finish(npm, att)


def embed_rows(table, ids, scale=None, y=None):
    """Rows `ids` of the bf16 table ([rows, cols], uint16 bits; int16 on the device) as fp32, times
    the fp32 `scale` when given: the board runtime's embedding lookup (tars_board.py:298-314),
    done on the device. y: optional fp32 [len(ids), cols] output rows (row-strided view allowed)."""
    nm = _numpy_mode(table)
    t = _to_dev(table)
    if t.dim() != 2 or t.element_size() != 2 or t.is_floating_point():
        raise ValueError("the table is a 2-D array of bf16 bits (uint16 / int16)")
    ids = np.ascontiguousarray(np.asarray(ids, np.int64).reshape(-1))
    if ids.size == 0:
        raise ValueError("no ids")
    if ids.min() < -(1 << 31) or ids.max() >= (1 << 31):
        raise ValueError("ids must fit int32")
    ids32 = ids.astype(np.int32)
    rows, cols = t.shape
    if y is None:
        y = torch.empty((ids.size, cols), dtype=torch.float32, device=t.device)
    if y.shape != (ids.size, cols) or y.dtype != torch.float32:
        raise ValueError("y must be fp32 [len(ids), cols]")
    scaled = scale is not None
    _check(_lib.lib().tars_embed_rows(t.data_ptr(), _ld(t), rows, cols,
                                      ids32.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), ids32.size,
                                      int(scaled), _f32_bits(scale) if scaled else 0, y.data_ptr(), _ld(y),
                                      _stream()))
    return _finish(nm, y)


def set_w8a8_path(path: str) -> str:
    """'auto' | 'gemv' | 'mfma': which W8A8 kernel family runs for M >= 2 (and M = 1). Returns the
    previous setting."""
    codes = {"auto": 0, "gemv": 1, "mfma": 2}
    prev = _lib.lib().tars_set_w8a8_path(codes[path])
    return {v: k for k, v in codes.items()}[prev]


__all__ = ["TarsError", "ContractError", "quant_rows", "gemm_rowcol", "quant_gemm_rowcol", "gemm_rowcol_ksplit",
           "align_w4_groups", "gemm_w4", "embed_rows", "attention", "set_w8a8_path", "ESIZE", "softmax_rows", "softmax_rows_causal",
           "layernorm_rows", "rmsnorm_rows", "l2norm_rows", "relu", "elt", "rope_rows", "fdot_nt", "fdot_nn",
           "ROW_SOFTMAX", "ROW_LAYERNORM", "ROW_RMSNORM", "ROW_L2NORM", "ELT_MUL", "ELT_ADD", "ELT_MULADD",
           "ELT_SUB", "BM_DENSE", "BM_ROW", "BM_COL", "BM_SCALAR"]
