#!/usr/bin/env python3
"""Benchmark of the W8A8 / W4A16 matrix path on one MI355X.

Headline workload (`value`): one Qwen3-0.6B decode step's linear set at M = 1, as the golden model
runs it: 28 layers x (q 1024->2048, k 1024->1024, v 1024->1024, o 2048->1024, gate/up 1024->3072,
down 3072->1024) plus the lm_head 1024->151936, each preceded by its per-token quantizer (q/k/v share
one quantization, gate/up share one, o and down have their own, the head its own). Weights are
seeded random int8 with per-channel fp32 scales (~596 MB of weights per step), resident in HBM
before timing. A step is captured once as a HIP graph (the C ABI validates every call at capture)
and replayed; `value` = algorithmic HBM bytes of the step / step time.

Also reported: each single-GPU workload of the path ("configs": Qwen3-0.6B decode shapes, the
lm_head, the K-split projections, M = 4 / 256 prefill, W4A16 group-128) as us/call, GB/s and
roofline fraction (and TOPS for the prefill GEMM), each rotated over >= 512 MiB of distinct weight
copies so the 256 MB MALL cannot serve it, each with the numpy oracle's golden path timed on one
core on the inputs of its first copy and checked bit for bit against the GPU's output; per row of
the decode step (kernel instance and role: q/k/v, o, gate/up, down, head) the dispatch durations
from the dispatches' own start and end timestamps (the roofline row is the one with the most
dispatch time per step), beside the time each launch adds to a dependent chain of graph launches;
the same decode step as a 313-descriptor queue through the library's queue
executor ("queue_executor", host clock, end to end); a whole Qwen3-0.6B decode step at position 250
(norms, quantizers, every linear, q/k norms, RoPE, the attention, residual adds, SiLU * up and the
head: 1910 descriptors) through the same executor ("queue_whole_decode_step_t250"); and the CPU
baseline (the numpy oracle, single core) on a bounded sample of the same workload, with a bit-exact
check of the timed outputs.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-configs] [--no-cpu-baseline] [--no-queue]
"""
from __future__ import annotations

import os

# The CPU baseline is a single-core figure: pin every numeric library's thread pool to one thread
# before numpy (or torch) loads its BLAS / OpenMP runtime.
for _var in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS", "BLIS_NUM_THREADS",
             "NUMEXPR_NUM_THREADS"):
    os.environ[_var] = "1"

import argparse
import ctypes
import json
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK = 8.0e12          # MI355X HBM3E, bytes/s
INT8_PEAK = 5.0e15         # MI355X dense INT8 MFMA, ops/s
ROTATE_BYTES = 512 << 20   # distinct weight bytes each single-config measurement cycles through

QWEN3_LAYERS = 28
QWEN3_H, QWEN3_Q, QWEN3_KV, QWEN3_FF, QWEN3_VOCAB = 1024, 2048, 1024, 3072, 151936


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-configs", action="store_true", help="skip the per-config measurements")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-queue", action="store_true", help="skip the descriptor-queue executor measurement")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU baseline sample length")
    ap.add_argument("--detail", type=str, default="", help="also write the full result JSON here")
    ap.add_argument("--only-configs", action="store_true",
                    help="run only the per-config measurements and print them (for profiler passes)")
    ap.add_argument("--config-reps", type=int, default=2000, help="launches timed per config")
    ap.add_argument("--pmc-summary", nargs=5, metavar=("FETCH_CSV", "WRITE_CSV", "MFMA_CSV", "VALU_CSV", "DETAIL"),
                    help="write the per-config counter table from four --only-configs rocprofv3 passes and exit")
    ap.add_argument("--pmc-out", type=str, default=str(ROOT / "profiles" / "config_traffic.json"))
    ap.add_argument("--pmc-step-summary", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "DETAIL"),
                    help="write the decode step's per-instance traffic from two rocprofv3 passes and exit")
    ap.add_argument("--pmc-step-out", type=str, default=str(ROOT / "profiles" / "decode_step_traffic.json"))
    ap.add_argument("--trace-summary", nargs=2, metavar=("KERNEL_TRACE_CSV", "DETAIL"),
                    help="summarize a rocprofv3 --kernel-trace run of the decode step per row (kernel, grid)")
    ap.add_argument("--trace-out", type=str, default=str(ROOT / "profiles" / "decode_step_kernels.json"))
    return ap.parse_args()


# ------------------------------------------------------------------------------ launch plumbing
class Launch:
    """One C-ABI call with its arguments resolved to raw pointers (no per-call Python checks).
    `operands` keeps the device tensors it reads and writes (for checks and the CPU baseline)."""

    def __init__(self, kind: str, fn, args: tuple, nbytes: int, ops: int, name: str, operands: dict):
        self.kind, self.fn, self.args, self.nbytes, self.ops, self.name = kind, fn, args, nbytes, ops, name
        self.operands = operands

    def __call__(self, stream: int) -> None:
        rc = self.fn(*self.args, stream)
        if rc != 0:
            from opentars_amd import _lib
            raise RuntimeError(f"{self.name}: status {rc}: {_lib.last_error()}")


def quant_launch(lib, x, q, s, name=""):
    M, K = x.shape
    return Launch("quant_rows", lib.tars_quant_rows,
                  (x.data_ptr(), x.stride(0) * 4, q.data_ptr(), q.stride(0), s.data_ptr(), M, K),
                  4 * M * K + M * K + 4 * M, 0, name, dict(x=x, q=q, s=s))


def w8_launch(lib, q, s, W, scol, y, name=""):
    M, K = q.shape
    N = W.shape[0]
    return Launch("gemm_w8a8", lib.tars_gemm_w8a8,
                  (q.data_ptr(), q.stride(0), s.data_ptr(), W.data_ptr(), scol.data_ptr(), N, None,
                   y.data_ptr(), y.stride(0) * 4, M, N, K, 0, 0, 0),
                  N * K + 4 * N + M * K + 4 * M + 4 * M * N, 2 * M * N * K, name,
                  dict(q=q, s=s, W=W, scol=scol, y=y))


def fused_launch(lib, x, mats, name=""):
    """One tars_quant_gemm_w8a8 call: x quantized in registers, feeding mats [(W, scol, y), ...]."""
    from opentars_amd import _lib
    M, K = x.shape
    descs = (_lib.W8A8Out * len(mats))(*[_lib.W8A8Out(W.data_ptr(), sc.data_ptr(), None, y.data_ptr(),
                                                      y.stride(0) * 4, W.shape[0], 0, 0, 0) for W, sc, y in mats])
    nbytes = 4 * M * K + sum(W.shape[0] * K + 4 * W.shape[0] + 4 * M * W.shape[0] for W, _, _ in mats)
    ops = sum(2 * M * W.shape[0] * K for W, _, _ in mats)
    return Launch("quant_gemm_w8a8", lib.tars_quant_gemm_w8a8,
                  (x.data_ptr(), x.stride(0) * 4, None, 0, None, M, K, descs, len(mats)),
                  nbytes, ops, name, dict(x=x, mats=mats, descs=descs))


def ksplit_launch(lib, q, s, blocks, scol, y, name=""):
    M = q.shape[0]
    N = blocks[0].shape[0]
    nb = len(blocks)
    ptrs = (ctypes.c_void_p * nb)(*[b.data_ptr() for b in blocks])
    ks = (ctypes.c_int32 * nb)(*[b.shape[1] for b in blocks])
    K = sum(b.shape[1] for b in blocks)
    return Launch("gemm_w8a8_ksplit", lib.tars_gemm_w8a8_ksplit,
                  (q.data_ptr(), q.stride(0), s.data_ptr(), ptrs, ks, nb, scol.data_ptr(), y.data_ptr(),
                   y.stride(0) * 4, M, N),
                  N * K + 4 * N + M * K + 4 * M + 4 * M * N, 2 * M * N * K, name,
                  dict(q=q, s=s, blocks=blocks, scol=scol, y=y, ptrs=ptrs, ks=ks))


def w4_launch(lib, x, Wp, ws, y, name=""):
    M, K = x.shape
    N = Wp.shape[0]
    return Launch("gemm_w4a16", lib.tars_gemm_w4a16,
                  (x.data_ptr(), x.stride(0) * 4, 4, Wp.data_ptr(), ws.data_ptr(), None, y.data_ptr(),
                   y.stride(0) * 4, M, N, K, 0, 0, 0),
                  N * K // 2 + 2 * N * (K // 128) + 4 * M * K + 4 * M * N, 2 * M * N * K, name,
                  dict(x=x, Wp=Wp, ws=ws, y=y))


# ------------------------------------------------------------------------------ workloads
def rand_int8(torch, gen, n, k):
    return torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda", generator=gen)


def rand_scales(torch, gen, n):
    return (torch.rand(n, device="cuda", generator=gen) * 9e-3 + 1e-3).to(torch.float32)


def decode_set(torch, lib, seed: int):
    """The Qwen3-0.6B decode-step linear set in model order. Returns (fused, unfused, buffers):
    fused = one quantize+GEMV launch per shared quantization (q/k/v, o, gate/up, down, head), the
    way the library runs a layer; unfused = the golden model's own descriptor sequence (ROW_QUANT,
    then one GEMM per projection), used for the CPU baseline and as a comparison."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    H, Q, KV, FF = QWEN3_H, QWEN3_Q, QWEN3_KV, QWEN3_FF
    keep, fused, unfused = [], [], []

    def act(k):
        x = torch.randn((1, k), device="cuda", generator=gen, dtype=torch.float32)
        q = torch.empty((1, k), dtype=torch.int8, device="cuda")
        s = torch.empty((1,), dtype=torch.float32, device="cuda")
        keep.extend([x, q, s])
        return x, q, s

    def lin(n, k):
        W, sc, y = rand_int8(torch, gen, n, k), rand_scales(torch, gen, n), torch.empty((1, n), device="cuda")
        keep.extend([W, sc, y])
        return W, sc, y

    def group(tag, k, projs):
        x, q, s = act(k)
        mats = [lin(n, k) for _, n in projs]
        fused.append(fused_launch(lib, x, mats, tag))
        unfused.append(quant_launch(lib, x, q, s, tag + ".quant"))
        for (nm, _), (W, sc, y) in zip(projs, mats):
            unfused.append(w8_launch(lib, q, s, W, sc, y, nm))

    for L in range(QWEN3_LAYERS):
        group(f"L{L}.qkv", H, [(f"L{L}.q_proj", Q), (f"L{L}.k_proj", KV), (f"L{L}.v_proj", KV)])
        group(f"L{L}.o", Q, [(f"L{L}.o_proj", H)])
        group(f"L{L}.gate_up", H, [(f"L{L}.gate_proj", FF), (f"L{L}.up_proj", FF)])
        group(f"L{L}.down", FF, [(f"L{L}.down_proj", H)])
    group("head", H, [("lm_head", QWEN3_VOCAB)])
    return fused, unfused, keep


def queue_decode_step(torch, lib, seed: int, steps: int, warmup: int) -> dict:
    """The same decode-step linear set as a descriptor queue in one device-resident DDR image, run
    through the library's executor (tars_run_queue) the way QwenLowering emits it: per layer
    ROW_QUANT + q/k/v GEMMs, ROW_QUANT + o, ROW_QUANT + gate/up, ROW_QUANT + down, then ROW_QUANT +
    the head as 4 blocks of 37984 rows (qwen_ref.py:371-378); 313 descriptors, QM_ROWCOL, fp32 out.
    Timed end to end per step on the host clock (descriptor checks, launches and GPU work, the host
    holding its copy of the queue): with the executor's quantizer+GEMM fusion (113 launches) and its
    launch plans (a repeated queue replays as one HIP graph), with fusion but every run checked and
    launched, and with neither (313 launches)."""
    from opentars_amd import _lib, contract as C
    from opentars_amd.queue import encode_descriptor
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 7)
    H, Qd, KV, FF, V = QWEN3_H, QWEN3_Q, QWEN3_KV, QWEN3_FF, QWEN3_VOCAB
    small, big = [0], [0]

    def take(region, n, align):
        a = (region[0] + align - 1) // align * align
        region[0] = a + n
        return a

    descs, fills, nbytes = [], [], 0

    def quant(k):
        x, q, s = take(small, 4 * k, 16), take(small, k, 16), take(small, 16, 16)
        fills.append(("randn", x, k))
        descs.append(dict(OPCODE=C.OP_ROW, CTRL=C.ROW_QUANT, EPI=C.epi(out=C.OUT_INT8), A_OFF=x, Y_OFF=q,
                          SCALE_OFF=s, M=1, N=k))
        return q, s, 4 * k

    def gemm(q, s, k, n, w=None, sc=None, y=None):
        w = take(big, n * k, 256) if w is None else w
        sc = take(small, 4 * n, 16) if sc is None else sc
        y = take(small, 4 * n, 16) if y is None else y
        descs.append(dict(OPCODE=C.OP_GEMM, CTRL=C.ctrl(C.QM_ROWCOL), EPI=C.epi(), A_OFF=q, W_OFF=w, SCALE_OFF=sc,
                          Y_OFF=y, HDR_RSV=s // 16, M=1, N=n, K=k))
        return w, sc, y, n * k + 4 * n + 4 * n

    for _ in range(QWEN3_LAYERS):
        for k, projs in ((H, (Qd, KV, KV)), (Qd, (H,)), (H, (FF, FF)), (FF, (H,))):
            q, s, xb = quant(k)
            nbytes += xb
            for n in projs:
                w, sc, y, b = gemm(q, s, k, n)
                fills += [("int8", w, n * k), ("scale", sc, n)]
                nbytes += b
    q, s, xb = quant(H)
    nbytes += xb
    hw, hsc, hy = take(big, V * H, 256), take(small, 4 * V, 16), take(small, 4 * V, 16)
    fills += [("int8", hw, V * H), ("scale", hsc, V)]
    rows = V // 4
    for blk in range(4):
        nbytes += gemm(q, s, H, rows, hw + blk * rows * H, hsc + 4 * blk * rows, hy + 4 * blk * rows)[3]
    qaddr = take(small, 64 * len(descs), 64)
    if small[0] >= 16 * (1 << 24):
        raise RuntimeError("row scales must lie below 16 * 2^24 bytes (the HDR_RSV field)")
    base_big = (small[0] + 4095) // 4096 * 4096
    image = torch.empty(base_big + big[0], dtype=torch.uint8, device="cuda")
    image[:base_big].zero_()
    for kind, off, n in fills:
        off = off + (base_big if kind == "int8" else 0)
        if kind == "int8":
            image[off:off + n].view(torch.int8).copy_(
                torch.randint(-127, 128, (n,), dtype=torch.int8, device="cuda", generator=gen))
        elif kind == "scale":
            image[off:off + 4 * n].view(torch.float32).copy_(torch.rand(n, device="cuda", generator=gen) * 9e-3 + 1e-3)
        else:
            image[off:off + 4 * n].view(torch.float32).copy_(torch.randn(n, device="cuda", generator=gen))
    raw = []
    for d in descs:
        if d["OPCODE"] == C.OP_GEMM:
            d = dict(d, W_OFF=d["W_OFF"] + base_big)
        raw.append(encode_descriptor(dict(MAGIC=C.MAGIC, VERSION=C.VERSION, VALID=1, **d)))
    host_q = b"".join(raw)
    image[qaddr:qaddr + len(host_q)].copy_(torch.frombuffer(bytearray(host_q), dtype=torch.uint8).cuda())
    torch.cuda.synchronize()
    st = _lib.QueueStatus()
    stream = torch.cuda.current_stream().cuda_stream

    def run():
        rc = lib.tars_run_queue(image.data_ptr(), image.numel(), qaddr, len(raw), host_q, 0, 0, ctypes.byref(st),
                                stream)
        if rc != 0 or not st.done:
            raise RuntimeError(f"queue: status {rc} done={st.done} err={st.err_code} op={st.op_idx}: "
                               f"{_lib.last_error()}")

    res = {"descriptors": len(raw), "image_bytes": int(image.numel()), "algorithmic_bytes_per_step": nbytes}
    # fused + launch plans (the default: from the third run on, one graph launch per step); fused
    # with every run checked and launched; the golden's one launch per descriptor
    for key, fusion, graphs in (("fused_plans", 1, 1), ("fused", 1, 0), ("unfused", 0, 0)):
        prev_f, prev_g = lib.tars_set_queue_fusion(fusion), lib.tars_set_queue_graphs(graphs)
        try:
            for _ in range(max(warmup, 3)):
                run()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            e0.record()
            for _ in range(steps):
                run()
            e1.record()
            torch.cuda.synchronize()
            t = (time.perf_counter() - t0) / steps
            tg = e0.elapsed_time(e1) / 1e3 / steps
        finally:
            lib.tars_set_queue_fusion(prev_f)
            lib.tars_set_queue_graphs(prev_g)
        # host clock end to end (checks, launches, the wait for the last step) and the stream's own
        # time between events around the steps
        res[key] = {"launches_per_step": 113 if fusion else len(raw), "ms_per_step": round(t * 1e3, 4),
                    "GBps": round(nbytes / t / 1e9, 1), "gpu_ms_per_step": round(tg * 1e3, 4)}
    del image
    torch.cuda.empty_cache()
    return res


class DecodeQueue:
    """A Qwen3-style decode step (one token at position t0) as the descriptor queue the reference's
    lowering emits for it (tars_mini/llm.py:705-767 attention block, :614-640 MLP, 330-338
    linears, 94-108 norm/quant/softmax): per layer RMSNorm -> ROW_QUANT -> q/k/v GEMMs (v straight
    into the V cache row t0) -> per-head RMSNorm + RoPE of q and k (k into the K cache row) -> per
    head FDOT_NT / causal softmax / FDOT_NN -> ROW_QUANT -> o GEMM -> residual ELT_ADD -> RMSNorm ->
    ROW_QUANT -> gate (SiLU) / up GEMMs -> ELT_MUL in place -> ROW_QUANT -> down GEMM -> residual;
    then the final RMSNorm, ROW_QUANT and the head in 4 blocks. Synthetic weights (int8 with
    per-channel scales, norms near 1), KV caches holding t0 earlier positions. `small` data first
    (row scales must lie below 16 * 2^24 bytes), weights after."""

    def __init__(self, layers=28, H=1024, heads=16, kv_heads=8, hd=128, ff=3072, vocab=151936, t0=250,
                 head_blocks=4):
        from opentars_amd import contract as C
        self.C = C
        self.descs, self.fills = [], []
        self.small, self.big = [0], [0]
        nk = (t0 + 1 + 15) // 16 * 16
        take_s = lambda n: self._take(self.small, n, 256)
        take_b = lambda n: self._take(self.big, n, 256)
        tab = take_s(4 * hd * (t0 + 1))
        self.fills.append(("rope", tab, (t0 + 1, hd)))
        x = take_s(4 * H)
        self.fills.append(("randn", x, H, 1.0))
        self.weight_bytes = 0
        for _ in range(layers):
            kc, vc = take_s(4 * nk * kv_heads * hd), take_s(4 * nk * kv_heads * hd)
            self.fills += [("randn", kc, nk * kv_heads * hd, 1.0), ("randn", vc, nk * kv_heads * hd, 1.0)]
            h = self.norm(x, H, 1, take_s)
            qh, sh = self.quant(h, H, take_s)
            q = self.gemm(qh, sh, H, heads * hd, take_s, take_b)
            k = self.gemm(qh, sh, H, kv_heads * hd, take_s, take_b)
            self.gemm(qh, sh, H, kv_heads * hd, take_s, take_b, y=vc + 4 * t0 * kv_heads * hd)
            qn = self.norm(q, hd, heads, take_s)
            qr = take_s(4 * heads * hd)
            self.add(OPCODE=C.OP_ROPE, EPI=C.epi(), A_OFF=qn, W_OFF=tab + 4 * hd * t0, Y_OFF=qr, M=heads, N=hd, K=hd,
                     GROUP_SIZE=heads)
            kn = self.norm(k, hd, kv_heads, take_s)
            self.add(OPCODE=C.OP_ROPE, EPI=C.epi(), A_OFF=kn, W_OFF=tab + 4 * hd * t0,
                     Y_OFF=kc + 4 * t0 * kv_heads * hd, M=kv_heads, N=hd, K=hd, GROUP_SIZE=kv_heads)
            sc, pr, att = take_s(4 * nk), take_s(4 * nk), take_s(4 * heads * hd)
            for hh in range(heads):
                kv = hh // (heads // kv_heads)
                self.add(OPCODE=C.OP_FDOT, EPI=C.epi(), A_OFF=qr + 4 * hh * hd, W_OFF=kc + 4 * kv * hd, Y_OFF=sc,
                         M=1, N=nk, K=hd, GROUP_SIZE=4 * kv_heads * hd // 16)
                self.add(OPCODE=C.OP_ROW, CTRL=C.ROW_SOFTMAX, EPI=C.epi(), A_OFF=sc, Y_OFF=pr, M=1, N=nk, K=t0 + 1)
                self.add(OPCODE=C.OP_FDOT, CTRL=1, EPI=C.epi(), A_OFF=pr, W_OFF=vc + 4 * kv * hd,
                         Y_OFF=att + 4 * hh * hd, M=1, N=hd, K=nk, GROUP_SIZE=4 * kv_heads * hd // 16)
            qa, sa = self.quant(att, heads * hd, take_s)
            o = self.gemm(qa, sa, heads * hd, H, take_s, take_b)
            x1 = take_s(4 * H)
            self.add(OPCODE=C.OP_ELT, CTRL=C.ELT_ADD, EPI=C.epi(), A_OFF=x, W_OFF=o, Y_OFF=x1, M=1, N=H)
            h2 = self.norm(x1, H, 1, take_s)
            q2, s2 = self.quant(h2, H, take_s)
            g = self.gemm(q2, s2, H, ff, take_s, take_b, act=C.ACT_SILU)
            u = self.gemm(q2, s2, H, ff, take_s, take_b)
            self.add(OPCODE=C.OP_ELT, CTRL=C.ELT_MUL, EPI=C.epi(), A_OFF=g, W_OFF=u, Y_OFF=g, M=1, N=ff)
            q3, s3 = self.quant(g, ff, take_s)
            d = self.gemm(q3, s3, ff, H, take_s, take_b)
            x = take_s(4 * H)
            self.add(OPCODE=C.OP_ELT, CTRL=C.ELT_ADD, EPI=C.epi(), A_OFF=x1, W_OFF=d, Y_OFF=x, M=1, N=H)
        hf = self.norm(x, H, 1, take_s)
        qf, sf = self.quant(hf, H, take_s)
        hw, hsc, hy = take_b(vocab * H), take_s(4 * vocab), take_s(4 * vocab)
        self.fills += [("int8", hw, vocab * H), ("scale", hsc, vocab)]
        self.weight_bytes += vocab * H
        rows = vocab // head_blocks
        for blk in range(head_blocks):
            self.add(OPCODE=C.OP_GEMM, CTRL=C.ctrl(C.QM_ROWCOL), EPI=C.epi(), A_OFF=qf, W_OFF=hw + blk * rows * H,
                     SCALE_OFF=hsc + 4 * blk * rows, Y_OFF=hy + 4 * blk * rows, HDR_RSV=sf // 16, M=1, N=rows, K=H)
        self.logits, self.vocab = hy, vocab
        self.qaddr = take_s(64 * len(self.descs))
        if self.small[0] >= 16 * (1 << 24):
            raise RuntimeError("row scales must lie below 16 * 2^24 bytes (the HDR_RSV field)")
        self.base_big = (self.small[0] + 4095) // 4096 * 4096
        self.size = self.base_big + self.big[0]

    @staticmethod
    def _take(region, n, align):
        a = (region[0] + align - 1) // align * align
        region[0] = a + n
        return a

    def add(self, **f):
        self.descs.append(dict(MAGIC=self.C.MAGIC, VERSION=self.C.VERSION, VALID=1, **f))

    def norm(self, x, n, rows, take_s):
        g = take_s(4 * n)
        self.fills.append(("gamma", g, n))
        y = take_s(4 * n * rows)
        self.add(OPCODE=self.C.OP_ROW, CTRL=self.C.ROW_RMSNORM, EPI=self.C.epi(), A_OFF=x, SCALE_OFF=g,
                 W_OFF=int(np.float32(1e-6).view(np.uint32)), Y_OFF=y, M=rows, N=n)
        return y

    def quant(self, x, k, take_s):
        q, s = take_s(k), take_s(16)
        self.add(OPCODE=self.C.OP_ROW, CTRL=self.C.ROW_QUANT, EPI=self.C.epi(out=self.C.OUT_INT8), A_OFF=x, Y_OFF=q,
                 SCALE_OFF=s, M=1, N=k)
        return q, s

    def gemm(self, q, s, k, n, take_s, take_b, act=0, y=None):
        C = self.C
        w, sc = take_b(n * k), take_s(4 * n)
        y = take_s(4 * n) if y is None else y
        self.fills += [("int8", w, n * k), ("scale", sc, n)]
        self.weight_bytes += n * k
        self.add(OPCODE=C.OP_GEMM, CTRL=C.ctrl(C.QM_ROWCOL, fusion=int(act != 0)), EPI=C.epi(act), A_OFF=q, W_OFF=w,
                 SCALE_OFF=sc, Y_OFF=y, HDR_RSV=s // 16, M=1, N=n, K=k)
        return y

    def raw(self) -> bytes:
        """The encoded queue, weight offsets moved past the small region."""
        from opentars_amd.queue import encode_descriptor
        out = []
        for d in self.descs:
            if d["OPCODE"] == self.C.OP_GEMM:
                d = dict(d, W_OFF=d["W_OFF"] + self.base_big)
            out.append(encode_descriptor(d))
        return b"".join(out)

    def fill(self, put):
        """put(kind, offset, count, extra) for every region (weights at base_big + offset)."""
        for f in self.fills:
            kind, off = f[0], f[1]
            put(kind, off + (self.base_big if kind == "int8" else 0), *f[2:])


def full_decode_step(torch, lib, seed: int, t0: int = 250, steps: int = 20) -> dict:
    """A whole Qwen3-0.6B decode step at t=250 as one descriptor queue (1910 descriptors) in one
    device image, through the executor with its fusions and launch plans: ms per token."""
    from opentars_amd import _lib
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 11)
    dq = DecodeQueue(t0=t0)
    image = torch.zeros(dq.size, dtype=torch.uint8, device="cuda")

    def put(kind, off, n, extra=None):
        if kind == "int8":
            image[off:off + n].view(torch.int8).copy_(torch.randint(-127, 128, (n,), dtype=torch.int8, device="cuda",
                                                                    generator=gen))
        elif kind == "scale":
            image[off:off + 4 * n].view(torch.float32).copy_(torch.rand(n, device="cuda", generator=gen) * 9e-3 + 1e-3)
        elif kind == "gamma":
            image[off:off + 4 * n].view(torch.float32).copy_(1 + 0.1 * torch.randn(n, device="cuda", generator=gen))
        elif kind == "rope":
            rows, hd = n
            pos = torch.arange(rows, device="cuda", dtype=torch.float32)[:, None]
            inv = 1.0 / (1e6 ** (torch.arange(0, hd, 2, device="cuda", dtype=torch.float32) / hd))
            fr = pos * inv[None, :]
            image[off:off + 4 * rows * hd].view(torch.float32).copy_(torch.cat([fr.cos(), fr.sin()], 1).reshape(-1))
        else:
            image[off:off + 4 * n].view(torch.float32).copy_(torch.randn(n, device="cuda", generator=gen) * extra)

    dq.fill(put)
    host_q = dq.raw()
    image[dq.qaddr:dq.qaddr + len(host_q)].copy_(torch.frombuffer(bytearray(host_q), dtype=torch.uint8).cuda())
    torch.cuda.synchronize()
    st = _lib.QueueStatus()
    stream = torch.cuda.current_stream().cuda_stream
    n = len(dq.descs)

    def run():
        rc = lib.tars_run_queue(image.data_ptr(), image.numel(), dq.qaddr, n, host_q, 0, 0, ctypes.byref(st), stream)
        if rc != 0 or not st.done:
            raise RuntimeError(f"decode queue: status {rc} done={st.done} err={st.err_code} op={st.op_idx}: "
                               f"{_lib.last_error()}")

    res = {"descriptors": n, "t0": t0, "weight_bytes": dq.weight_bytes}
    for key, fusion, graphs, reps in (("fused_plans", 1, 1, steps), ("fused", 1, 0, 3)):
        prev_f, prev_g = lib.tars_set_queue_fusion(fusion), lib.tars_set_queue_graphs(graphs)
        try:
            for _ in range(3):
                run()
            torch.cuda.synchronize()
            t_start = time.perf_counter()
            for _ in range(reps):
                run()
            torch.cuda.synchronize()
            t = (time.perf_counter() - t_start) / reps
        finally:
            lib.tars_set_queue_fusion(prev_f)
            lib.tars_set_queue_graphs(prev_g)
        res[key] = {"ms_per_token": round(t * 1e3, 3), "tokens_per_s": round(1 / t, 1)}
    logits = image[dq.logits:dq.logits + 4 * dq.vocab].view(torch.float32)
    res["logits_finite"] = bool(torch.isfinite(logits).all().item())
    del image
    torch.cuda.empty_cache()
    return res


def capture(torch, launches):
    """A HIP graph of the launches in order (torch's capture stream is the current stream)."""
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for l in launches:                  # one eager pass on the capture stream first
            l(torch.cuda.current_stream().cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        s = torch.cuda.current_stream().cuda_stream
        for l in launches:
            l(s)
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, reps: int, warmup: int) -> float:
    """Seconds per replay (events on the current stream, synchronized on both sides)."""
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / reps


def plain_rows_per_wave(rows: int, M: int = 1, K: int = 1024) -> int:
    """The plain GEMV's rows-per-wave rule (gemv_w8a8.hip, plain_rows_per_wave)."""
    return 4 if rows >= 32768 else 2 if M >= 3 and rows >= 2048 and K <= 8192 else 1


def fused_rows_per_wave(rows: int, K: int) -> int:
    """The fused quantize + GEMV rule (gemv_w8a8.hip, fused_rows_per_wave)."""
    u = 1
    while u < 4 and rows // (4 * 2 * u) >= 256:
        u *= 2
    wgs = -(-rows // (4 * u))
    if 256 < wgs < 512:
        return 6 if K <= 1024 and -(-rows // 24) <= 256 else 2 * u
    return u


def kernel_instance(l: Launch) -> str:
    """The HIP kernel instance a launch runs, named as rocprofv3 names it (mirrors the dispatch in
    gemv_w8a8.hip for the M = 1 W8A8 paths)."""
    if l.kind == "quant_gemm_w8a8":
        K = l.args[6]
        rows = sum(d.N for d in l.operands["descs"])
        simple = all(not d.bias and d.act == 0 and d.out == 0 for d in l.operands["descs"])
        name, u, tail = "quant_gemv_w8a8_kernel", fused_rows_per_wave(rows, K), ""
    elif l.kind == "gemm_w8a8" and l.args[9] == 1:
        K, rows = l.args[11], l.args[10]
        simple = l.args[2] is not None and l.args[6] is None and l.args[12] == 0 and l.args[13] == 0
        name, u, tail = "gemv_w8a8_kernel", plain_rows_per_wave(rows), ", 1"
    else:
        return l.kind
    # the epilogue instance: true for QM_ROWCOL with fp32 output and no bias or activation; the
    # fused kernel's last parameter (row pairs for a gated product) is false here
    tail += ", true" if simple else ", false"
    if name == "quant_gemv_w8a8_kernel":
        tail += ", false"
    c = K // 16
    if c <= 32:
        lanes = 8 if c <= 8 else 16 if c <= 16 else 32
        return f"{name}<{lanes}, 1, 8{tail}>"
    cpl = -(-c // 64)
    if cpl > 8:
        return f"{name}<64, 0, {1 if u == 1 else 4}{tail}>"
    u = min(u, {1: 8, 2: 4, 3: 2, 4: 2}.get(cpl, 1))
    return f"{name}<64, {cpl}, {u}{tail}>"


def role(l: Launch) -> str:
    """The projection group a decode-step launch serves, the layer index dropped: qkv, o, gate_up,
    down or head."""
    return l.name.split(".", 1)[1] if l.name.startswith("L") and "." in l.name else l.name


def fused_grid_items(l: Launch) -> int:
    """Work-items of a fused quantizer + GEMV dispatch (rocprofv3's grid size): matrices of unequal
    height cut into pieces of their greatest common height, one 256-thread workgroup per 4 U rows
    of a piece (mirrors go_fused in gemv_w8a8.hip for whole-wave rows and no row pairs)."""
    import math
    ns = [d.N for d in l.operands["descs"]]
    h = 0
    for n in ns:
        h = math.gcd(h, n)
    u = fused_rows_per_wave(sum(ns), l.args[6])
    return -(-h // (4 * u)) * (sum(ns) // h) * 256


def row_key(l: Launch) -> str:
    """A decode-step launch's kernel instance and role, as the measurement rows name them."""
    return f"{kernel_instance(l)} @ {role(l)}"


def marginal_times(torch, graph, launches, rounds: int = 12, per: int = 8) -> dict:
    """What each row (kernel instance and role) adds to the decode step: the step graph's time less
    the time of a graph of the step without that row's launches, per launch of the row. Launch gaps
    are included and a graph's fixed replay cost cancels. The two graphs are timed in alternation
    (rounds x per replays each, HIP events around each group on the current stream) so drift
    cancels too. The rest of the step still streams at least 420 MB, above the 256 MB MALL, so
    every launch reads its weights cold as in the step."""
    rows = {}
    for l in launches:
        rows.setdefault(row_key(l), []).append(l)
    out = {}
    for key, ls in rows.items():
        reduced = capture(torch, [l for l in launches if row_key(l) != key])
        for _ in range(3):
            graph.replay()
            reduced.replay()
        torch.cuda.synchronize()
        tot = {0: 0.0, 1: 0.0}
        for _ in range(rounds):
            for i, g in ((0, graph), (1, reduced)):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(per):
                    g.replay()
                e1.record()
                torch.cuda.synchronize()
                tot[i] += e0.elapsed_time(e1) / 1e3
        del reduced
        full_s, without_s = tot[0] / (rounds * per), tot[1] / (rounds * per)
        us = (full_s - without_s) / len(ls) * 1e6
        l = ls[0]
        out[key] = {"kernel": kernel_instance(l), "role": role(l),
                    "grid_items": fused_grid_items(l) if l.kind == "quant_gemm_w8a8" else None,
                    "launches_per_step": len(ls), "avg_bytes_per_launch": l.nbytes,
                    "us_per_launch": round(us, 3), "us_per_step": round(us * len(ls), 2),
                    "GBps": round(l.nbytes / us / 1e3, 1), "hbm_frac": round(l.nbytes / us / 1e3 / (HBM_PEAK / 1e9), 4)}
    return out


# ------------------------------------------------------------------------------ single configs
def rotated(torch, make, per_copy_bytes: int):
    """Enough independent copies of a workload to cycle through ROTATE_BYTES."""
    n = max(2, -(-ROTATE_BYTES // max(per_copy_bytes, 1)))
    return [make(i) for i in range(n)]


CONFIG_REPS = 2000


def time_graph_replays(torch, g, reps: int, warmup: int) -> tuple[float, list[float]]:
    """Seconds per replay over `reps` back-to-back replays, and each replay's own seconds (an event
    recorded after every replay on the current stream)."""
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    ev[0].record()
    for i in range(reps):
        g.replay()
        ev[i + 1].record()
    torch.cuda.synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) / 1e3 for i in range(reps)]
    return ev[0].elapsed_time(ev[-1]) / 1e3 / reps, per


def quantiles(xs: list[float], qs=(0.1, 0.5, 0.9)) -> list[float]:
    """Linear-interpolation quantiles of `xs` (numpy's default method)."""
    s = sorted(xs)
    out = []
    for q in qs:
        p = q * (len(s) - 1)
        i = int(p)
        out.append(s[i] + (s[min(i + 1, len(s) - 1)] - s[i]) * (p - i))
    return out


def measure_config(torch, launches, reps_target: int | None = None) -> dict:
    """One config's launches (rotated over distinct weight copies) as a graph, replayed back to back:
    the mean µs per call over every replay (two events around the whole run), then, in a second
    run with an event after every replay, the p10 / median / p90 of each replay's per-call time
    (kept apart so the per-replay events do not touch the mean)."""
    reps_target = reps_target or CONFIG_REPS
    g = capture(torch, launches)
    reps = max(3, reps_target // len(launches))
    t = time_graph(torch, g, reps, warmup=2) / len(launches)
    _, per = time_graph_replays(torch, g, reps, warmup=0)
    nbytes, ops = launches[0].nbytes, launches[0].ops
    r = {"us_per_call": round(t * 1e6, 3), "GBps": round(nbytes / t / 1e9, 1),
         "hbm_frac": round(nbytes / t / HBM_PEAK, 4), "bytes_per_call": nbytes,
         "distinct_copies": len(launches), "replays": reps,
         "us_per_call_p10_p50_p90": [round(v * 1e6 / len(launches), 3) for v in quantiles(per)]}
    if ops:
        r["TOPS"] = round(ops / t / 1e12, 2)
        r["int8_peak_frac"] = round(ops / t / INT8_PEAK, 5)
    del g
    return r


# ------------------------------------------------------------------------------ profiler counters per config
CLOCK_HZ = 2.4e9            # MI355X peak engine clock
SIMDS = 1024                # 256 CUs x 4 SIMDs
COUNTER_FILE = ROOT / "profiles" / "config_traffic.json"
# the kernel instance (as rocprofv3 names it) and grid size in work-items that each per-config
# measurement dispatches, as the library's selection rules pick them
CONFIG_KERNELS = {
    "c1_gemv_qwen3_gate_M1_K1024_N3072": ("gemv_w8a8_kernel<64, 1, 1, 1, true>", 196608),
    "lm_head_M1_K1024_N151936": ("gemv_w8a8_kernel<64, 1, 4, 1, true>", 2430976),
    "lm_head_fused_quant_M1_K1024_N151936": ("quant_gemv_w8a8_kernel<64, 1, 4, true, false>", 2430976),
    "c2_gemma3_down_ksplit_3456+3456": ("gemv_w8a8_ksplit2_kernel<7, 1, 5>", 73920),
    "c2_gemma3_down_ksplit_4096+2816": ("gemv_w8a8_ksplit2_kernel<7, 1, 5>", 73920),
    "c4_prefill_M4_K1024_N3072": ("gemv_w8a8_kernel<64, 1, 2, 4, true>", 98304),
    "c4_prefill_M4_K3072_N1024": ("gemv_w8a8_kernel<64, 3, 1, 4, true>", 65536),
    "c4_prefill_M4_K1024_N3072_mfma": ("mfma_chunk_kernel<4, 2, true>", 49152),
    "c4_prefill_M4_K3072_N1024_mfma": ("mfma_chunk_kernel<8, 2, true>", 32768),
    "c4_prefill_M256_K1024_N3072": ("mfma_panel_kernel<4, true>", 65536),
    "c4_prefill_M256_K3072_N1024": ("mfma_tile_kernel<32, 32, 2, 2, 512, 3, true, false>", 65536),
    "c5_w4a16_M1_K1536_N12288": ("gemv_w4a16_kernel<4, 4, 1, 1, false, true>", 196608),
    "c5_w4a16_M1_K6144_N1536": ("gemv_w4a16_kernel<4, 2, 1, 3, false, true>", 49152),
    "c5_w4a16_M4_K1536_N12288": ("gemm_w4a16_mfma_kernel<4, 1, 4, 16, false, true>", 196608),
    "c5_w4a16_M4_K6144_N1536": ("gemv_w4a16_kernel<8, 2, 2, 3, false, true>", 98304),
    "c5_w4a16_M8_K1536_N12288": ("gemm_w4a16_mfma_kernel<8, 1, 8, 16, false, true>", 393216),
    "c5_w4a16_M8_K6144_N1536": ("gemv_w4a16_kernel<8, 3, 2, 3, false, true>", 131072),
}


def pmc_means(path: str) -> dict:
    """Per (kernel, grid) of a rocprofv3 counter_collection.csv: the dispatch count and the mean
    per dispatch of each counter (summed over the counter's hardware instances)."""
    import csv
    disp = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            d = disp.setdefault(row["Dispatch_Id"], {"kernel": row["Kernel_Name"], "grid": int(row["Grid_Size"]),
                                                     "c": {}})
            d["c"][row["Counter_Name"]] = d["c"].get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
    agg = {}
    for d in disp.values():
        a = agg.setdefault((d["kernel"], d["grid"]), {"n": 0, "sum": {}})
        a["n"] += 1
        for c, v in d["c"].items():
            a["sum"][c] = a["sum"].get(c, 0.0) + v
    return {k: {"dispatches": a["n"], **{c: v / a["n"] for c, v in a["sum"].items()}} for k, a in agg.items()}


def pmc_summary(csvs: list, detail: str, out: str) -> int:
    """The per-config counter table from four `--only-configs` profiler passes (FETCH_SIZE;
    WRITE_SIZE; SQ_VALU_MFMA_BUSY_CYCLES + SQ_INSTS_VALU_MFMA_MOPS_I8; SQ_INSTS_VALU) and the
    first pass's --detail output (algorithmic bytes per config). Byte counters are scaled by what
    they read for the 256 MiB device copy the pass starts with."""
    P = [pmc_means(p) for p in csvs]
    configs = json.loads(Path(detail).read_text())["configs"]

    def find(p, sub, grid):
        hits = [k for k in p if sub in k[0] and k[1] == grid]
        if len(hits) != 1:
            raise SystemExit(f"{len(hits)} kernels match {sub} with grid {grid}")
        return hits[0]
    copy = max((k for k in P[0] if "copyBuffer" in k[0]), key=lambda k: P[0][k]["FETCH_SIZE"])
    fetch_scale = (256 << 20) / (P[0][copy]["FETCH_SIZE"] * 1024)
    write_scale = (256 << 20) / (P[1][find(P[1], copy[0], copy[1])]["WRITE_SIZE"] * 1024)
    table = {}
    for key, (sub, grid) in CONFIG_KERNELS.items():
        m = [p[find(p, sub, grid)] for p in P]
        rd, wr = m[0]["FETCH_SIZE"] * 1024 * fetch_scale, m[1]["WRITE_SIZE"] * 1024 * write_scale
        alg = configs[key]["bytes_per_call"]
        table[key] = {"kernel": sub, "grid_workitems": grid, "dispatches": m[0]["dispatches"],
                      "read_bytes": round(rd), "write_bytes": round(wr), "traffic_bytes": round(rd + wr),
                      "algorithmic_bytes": alg, "traffic_over_algorithmic": round((rd + wr) / alg, 3),
                      "mfma_busy_cycles_per_simd": round(m[2].get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / SIMDS, 1),
                      "mfma_i8_ops": round(m[2].get("SQ_INSTS_VALU_MFMA_MOPS_I8", 0.0) * 512),
                      "valu_instructions_per_simd": round(m[3].get("SQ_INSTS_VALU", 0.0) / SIMDS, 1)}
    Path(out).write_text(json.dumps({"fetch_scale": round(fetch_scale, 5), "write_scale": round(write_scale, 5),
                                     "calibration": "256 MiB device-to-device copy", "configs": table}, indent=1))
    print(f"{len(table)} configs; FETCH_SIZE x {fetch_scale:.4f}, WRITE_SIZE x {write_scale:.4f}", flush=True)
    return 0


def pmc_step_summary(fetch_csv: str, write_csv: str, detail: str, out: str) -> int:
    """HBM traffic per launch of each decode-step row (kernel instance and grid, roofline_rows in
    the first pass's --detail output) from two profiler passes over the decode step (FETCH_SIZE,
    then WRITE_SIZE). Byte counters are scaled by what they read for the 1 GiB device copy the
    bench makes."""
    P = [pmc_means(fetch_csv), pmc_means(write_csv)]
    rows = json.loads(Path(detail).read_text())["roofline_rows"]
    copy = max((k for k in P[0] if "copyBuffer" in k[0]), key=lambda k: P[0][k]["FETCH_SIZE"])
    fetch_kib, write_kib = P[0][copy]["FETCH_SIZE"], P[1][copy]["WRITE_SIZE"]
    fetch_scale, write_scale = (1 << 30) / (fetch_kib * 1024), (1 << 30) / (write_kib * 1024)
    res = {}
    for key, r in rows.items():
        m = []
        for i in range(2):
            hits = [v for k, v in P[i].items() if f"::{r['kernel']}(" in k[0] and k[1] == r["grid_items"]]
            if len(hits) != 1:
                raise SystemExit(f"{len(hits)} dispatch groups match {key} (grid {r['grid_items']}) in pass {i}")
            m.append(hits[0])
        rd, wr = m[0]["FETCH_SIZE"] * 1024 * fetch_scale, m[1]["WRITE_SIZE"] * 1024 * write_scale
        res[key] = {"kernel": r["kernel"], "role": r["role"], "grid_items": r["grid_items"],
                    "read_bytes": round(rd), "write_bytes": round(wr), "traffic_bytes": round(rd + wr),
                    "algorithmic_bytes": r["avg_bytes_per_launch"],
                    "traffic_over_algorithmic": round((rd + wr) / r["avg_bytes_per_launch"], 3),
                    "dispatches": m[0]["dispatches"]}
    Path(out).write_text(json.dumps({
        "about": "HBM traffic per launch from rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE (KiB per "
                 "dispatch), each scaled by the same counter's reading for a 1 GiB device-to-device copy; "
                 "one row per kernel instance and grid size (the decode step's roles)",
        "fetch_copy_kib": fetch_kib, "write_copy_kib": write_kib, "fetch_scale": fetch_scale,
        "write_scale": write_scale, "rows": res}, indent=1))
    print(f"{len(res)} rows; FETCH_SIZE x {fetch_scale:.4f}, WRITE_SIZE x {write_scale:.4f}", flush=True)
    return 0


def trace_grid(row: dict) -> int:
    """Work-items of a dispatch in a rocprofv3 kernel-trace CSV row."""
    if "Grid_Size" in row:
        return int(row["Grid_Size"])
    return int(row["Grid_Size_X"]) * int(row.get("Grid_Size_Y") or 1) * int(row.get("Grid_Size_Z") or 1)


def trace_summary(trace_csv: str, detail: str, out: str) -> int:
    """Per decode-step row (kernel instance and grid size, roofline_rows in the same run's --detail
    output), the rocprofv3 kernel trace's dispatch durations (end minus start timestamp): count,
    mean, median and minimum; the HBM fraction that the mean gives for the row's algorithmic bytes
    per launch, beside bench.py's own dispatch-timed figure from the same run. Writes out (JSON)
    and the same name with .md."""
    import csv
    import statistics
    durs = {}
    with open(trace_csv, newline="") as f:
        for row in csv.DictReader(f):
            key = (row["Kernel_Name"], trace_grid(row))
            durs.setdefault(key, []).append((int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3)
    line = json.loads(Path(detail).read_text())
    rows, roof = line["roofline_rows"], line["roofline"]
    table = {}
    for key, r in rows.items():
        hits = [k for k in durs if f"::{r['kernel']}(" in k[0] and k[1] == r["grid_items"]]
        if len(hits) != 1:
            raise SystemExit(f"{len(hits)} dispatch groups match {key} (grid {r['grid_items']})")
        d = durs[hits[0]]
        avg = sum(d) / len(d)
        table[key] = {"kernel": r["kernel"], "role": r["role"], "grid_items": r["grid_items"],
                      "launches_per_step": r["launches_per_step"], "trace_dispatches": len(d),
                      "trace_avg_us": round(avg, 3), "trace_median_us": round(statistics.median(d), 3),
                      "trace_min_us": round(min(d), 3), "algorithmic_bytes": r["avg_bytes_per_launch"],
                      "hbm_frac_from_trace": round(r["avg_bytes_per_launch"] / avg / 1e3 / (HBM_PEAK / 1e9), 4),
                      "bench_us_per_launch": r["us_per_launch"], "bench_hbm_frac": r["hbm_frac"]}
    dom = next(k for k, r in rows.items() if r["kernel"] == roof["kernel"] and r["us_per_launch"] == roof["avg_us_per_launch"])
    summary = {"about": "rocprofv3 --kernel-trace dispatch durations per decode-step row (kernel instance and grid "
                        "size) against bench.py's own dispatch-timed figures from the same run",
               "line_roofline": {k: roof[k] for k in ("kernel", "shape", "frac", "avg_us_per_launch", "avg_bytes_per_launch")},
               "roofline_row": dom, "frac_from_trace": table[dom]["hbm_frac_from_trace"],
               "trace_over_bench_duration": round(table[dom]["trace_avg_us"] / roof["avg_us_per_launch"], 4),
               "rows": table}
    Path(out).write_text(json.dumps(summary, indent=1))
    md = [f"| Row (kernel instance @ role) | Work-items | Launches / step | Trace dispatches | Trace mean µs | Trace median µs | "
          f"Trace min µs | Algorithmic MB / launch | HBM frac (trace mean) | bench.py µs / launch in the step | bench.py HBM frac |",
          "|---|---|---|---|---|---|---|---|---|---|---|"]
    for key, t in sorted(table.items(), key=lambda kv: -kv[1]["trace_avg_us"] * kv[1]["launches_per_step"]):
        md.append(f"| `{key}` | {t['grid_items']} | {t['launches_per_step']} | {t['trace_dispatches']} | {t['trace_avg_us']} | "
                  f"{t['trace_median_us']} | {t['trace_min_us']} | {t['algorithmic_bytes'] / 1e6:.3f} | "
                  f"{t['hbm_frac_from_trace']} | {t['bench_us_per_launch']} | {t['bench_hbm_frac']} |")
    Path(out).with_suffix(".table.md").write_text("\n".join(md) + "\n")
    print(json.dumps({k: summary[k] for k in ("line_roofline", "roofline_row", "frac_from_trace", "trace_over_bench_duration")}),
          flush=True)
    return 0


def attach_counters(res: dict) -> None:
    """Profiler figures for each measured config whose algorithmic bytes match the table's: HBM
    traffic per call, and the share of the call (at the measured time and peak clock) that each
    SIMD's MFMA unit is busy and that its VALU issues (a wave64 VALU instruction holds a SIMD for
    4 cycles)."""
    if not COUNTER_FILE.exists():
        return
    table = json.loads(COUNTER_FILE.read_text())["configs"]
    for key, r in res.items():
        e = table.get(key)
        if not e or e["algorithmic_bytes"] != r.get("bytes_per_call") or e["kernel"] != CONFIG_KERNELS.get(key, ("",))[0]:
            continue                  # a stale entry: other bytes, or another kernel instance
        cycles = r["us_per_call"] * 1e-6 * CLOCK_HZ
        r["counters"] = {"kernel": e["kernel"], "traffic_bytes": e["traffic_bytes"],
                         "traffic_over_algorithmic": e["traffic_over_algorithmic"],
                         "mfma_busy_frac": round(e["mfma_busy_cycles_per_simd"] / cycles, 4),
                         "valu_issue_frac": round(4 * e["valu_instructions_per_simd"] / cycles, 4),
                         "source": "profiles/config_traffic.json (rocprofv3 --pmc)"}


def cpu_config_baseline(fn, gpu_out, nbytes: int, ops: int, min_s: float = 0.3) -> dict:
    """The oracle's golden-path restatement of one config call (fn: numpy, on the host copies of
    the GPU run's first weight copy and its inputs) on one pinned core: microseconds per call over
    at least min_s seconds (at least one call), the same algorithmic bytes and ops per second as
    the GPU figure, and whether its output equals the GPU's for that copy bit for bit."""
    mask = os.sched_getaffinity(0)
    os.sched_setaffinity(0, {min(mask)})
    try:
        want = fn()
        calls, t0 = 0, time.perf_counter()
        while True:
            fn()
            calls += 1
            el = time.perf_counter() - t0
            if el >= min_s:
                break
    finally:
        os.sched_setaffinity(0, mask)
    t = el / calls
    r = {"us_per_call": round(t * 1e6, 1), "GBps": round(nbytes / t / 1e9, 4), "calls": calls, "cores": 1,
         "bit_exact_vs_gpu": bool(np.ascontiguousarray(want).tobytes() == np.ascontiguousarray(gpu_out).tobytes())}
    if ops:
        r["GOPS"] = round(ops / t / 1e9, 3)
    return r


def config_suite(torch, lib, seed: int, attention: bool = True, cpu: bool = True) -> dict:
    from opentars_amd import ops
    from oracle import golden as G
    from oracle import numerics as F
    host = lambda t: t.cpu().numpy()

    def rerun_first(ls, y):
        """The GPU output of the rotation's first copy (launched once more after the timing)."""
        ls[0](torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        return host(y)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 1)
    res = {}

    def w8(M, N, K, name):
        x = torch.randn((M, K), device="cuda", generator=gen)
        q, s = ops.quant_rows(x)
        y = torch.empty((M, N), device="cuda")
        holds = []

        def make(i):
            W, sc = rand_int8(torch, gen, N, K), rand_scales(torch, gen, N)
            holds.append((W, sc))
            return w8_launch(lib, q, s, W, sc, y, name)
        ls = rotated(torch, make, N * K)
        r = measure_config(torch, ls)
        r.update(M=M, N=N, K=K)
        if cpu:
            W0, sc0 = holds[0]
            qn, sn, Wn, scn = host(q), host(s), host(W0), host(sc0)
            r["cpu_baseline"] = cpu_config_baseline(lambda: G.gemm_rowcol(qn, sn, Wn, scn), rerun_first(ls, y),
                                                    ls[0].nbytes, ls[0].ops)
        del ls, holds
        torch.cuda.empty_cache()
        return r

    res["c1_gemv_qwen3_gate_M1_K1024_N3072"] = w8(1, 3072, 1024, "c1")
    res["lm_head_M1_K1024_N151936"] = w8(1, QWEN3_VOCAB, 1024, "lm_head")
    # the head as the decode step runs it: the quantizer fused in, 4 distinct weight copies
    x = torch.randn((1, 1024), device="cuda", generator=gen)
    y = torch.empty((1, QWEN3_VOCAB), device="cuda")
    holds = []

    def make_head(i):
        W, sc = rand_int8(torch, gen, QWEN3_VOCAB, 1024), rand_scales(torch, gen, QWEN3_VOCAB)
        holds.append((W, sc))
        return fused_launch(lib, x, [(W, sc, y)], "head")
    ls = rotated(torch, make_head, QWEN3_VOCAB * 1024)
    r = dict(measure_config(torch, ls), M=1, N=QWEN3_VOCAB, K=1024)
    if cpu:
        W0, sc0 = holds[0]
        xn, Wn, scn = host(x), host(W0), host(sc0)

        def head_cpu():
            qn, sn = F.quant_rows(xn)
            return G.gemm_rowcol(qn, sn, Wn, scn)
        r["cpu_baseline"] = cpu_config_baseline(head_cpu, rerun_first(ls, y), ls[0].nbytes, ls[0].ops)
    res["lm_head_fused_quant_M1_K1024_N151936"] = r
    del ls, holds
    torch.cuda.empty_cache()
    for split in ((3456, 3456), (4096, 2816)):
        x = torch.randn((1, 6912), device="cuda", generator=gen)
        q, s = ops.quant_rows(x)
        y = torch.empty((1, 1152), device="cuda")
        holds = []

        def make(i):
            bl = [rand_int8(torch, gen, 1152, k) for k in split]
            sc = rand_scales(torch, gen, 1152)
            holds.append((bl, sc))
            return ksplit_launch(lib, q, s, bl, sc, y, "c2")
        ls = rotated(torch, make, 1152 * 6912)
        r = measure_config(torch, ls)
        r.update(M=1, N=1152, K=6912, blocks=list(split))
        if cpu:
            bl0, sc0 = holds[0]
            qn, sn, bln, scn = host(q), host(s), [host(b) for b in bl0], host(sc0)
            r["cpu_baseline"] = cpu_config_baseline(lambda: G.gemm_rowcol_ksplit(qn, sn, bln, scn),
                                                    rerun_first(ls, y), ls[0].nbytes, ls[0].ops)
        res[f"c2_gemma3_down_ksplit_{split[0]}+{split[1]}"] = r
        log(f"c2 {split}: {r['us_per_call']} us")
        del ls, holds
    # the automatic kernel family (GEMV rows for M = 4, INT8 MFMA for M = 256), and the MFMA family
    # forced at M = 4 beside it
    for M, path in ((4, 0), (4, 2), (256, 0)):
        for K, N in ((1024, 3072), (3072, 1024)):
            prev = lib.tars_set_w8a8_path(path)
            try:
                r = w8(M, N, K, "c4")
            finally:
                lib.tars_set_w8a8_path(prev)
            r["family"] = "mfma" if path == 2 or M > 16 else "gemv_rows"
            key = f"c4_prefill_M{M}_K{K}_N{N}" + ("_mfma" if path == 2 else "")
            res[key] = r
            log(f"{key}: {r['us_per_call']} us ({r['family']})")
    for M, K, N in ((1, 1536, 12288), (1, 6144, 1536), (4, 1536, 12288), (4, 6144, 1536), (8, 1536, 12288),
                    (8, 6144, 1536)):
        x = torch.randn((M, K), device="cuda", generator=gen)
        y = torch.empty((M, N), device="cuda")
        holds = []

        def make(i):
            Wp = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, device="cuda", generator=gen)
            ws = (torch.rand((N, K // 128), device="cuda", generator=gen) * 9e-3 + 1e-3).half()
            holds.append((Wp, ws))
            return w4_launch(lib, x, Wp, ws, y, "c5")
        ls = rotated(torch, make, N * K // 2)
        r = measure_config(torch, ls)
        r.update(M=M, N=N, K=K)
        if cpu and M == 1:
            Wp0, ws0 = holds[0]
            xn, Wpn, wsn = host(x), host(Wp0), host(ws0).view(np.uint16)
            r["cpu_baseline"] = cpu_config_baseline(lambda: G.gemm_w4(xn, Wpn, wsn), rerun_first(ls, y),
                                                    ls[0].nbytes, ls[0].ops)
        res[f"c5_w4a16_M{M}_K{K}_N{N}"] = r
        log(f"c5 M={M} K={K} N={N}: {r['us_per_call']} us")
        del ls, holds
        torch.cuda.empty_cache()
    if attention:
        res["attention_decode_qwen3_t250"] = attention_decode(torch, lib, gen)
        ad = res["attention_decode_qwen3_t250"]
        log(f"attention t=250: {ad['op_by_op']['us_per_layer']} us per layer op by op, "
            f"{ad['fused_op']['us_per_layer']} us fused")
    for r in res.values():
        # every config's inputs come from one CUDA generator with this seed, drawn in config order
        r["inputs_seed"] = seed + 1
    attach_counters(res)
    return res


QWEN3_HEADS, QWEN3_KV_HEADS, QWEN3_HEAD_DIM, QWEN3_LAYERS = 16, 8, 128, 28


def attention_layers(torch, lib, gen, t0: int):
    """Decode attention of one token at position t0 for every Qwen3-0.6B layer, as the reference
    lowers it (tars_mini/llm.py:736-746): per query head, FDOT_NT of the rotated q row with the
    head's K cache rows (scores over pad16(t0 + 1) keys), the causal softmax with t0 + 1 valid keys,
    and FDOT_NN of the probabilities with the V cache rows. fp32 caches of pad16(t0 + 1) rows per
    layer; each layer its own caches. Returns ([launches of layer l], bytes read per layer)."""
    nh, nkv, hd = QWEN3_HEADS, QWEN3_KV_HEADS, QWEN3_HEAD_DIM
    nk = (t0 + 1 + 15) // 16 * 16
    layers, keep = [], []
    for _ in range(QWEN3_LAYERS):
        kc = torch.randn((nk, nkv * hd), device="cuda", generator=gen)
        vc = torch.randn((nk, nkv * hd), device="cuda", generator=gen)
        q = torch.randn((1, nh * hd), device="cuda", generator=gen) * 0.1
        sc = torch.empty((1, nk), device="cuda")
        pr = torch.empty((1, nk), device="cuda")
        att = torch.empty((1, nh * hd), device="cuda")
        keep.append((kc, vc, q, sc, pr, att))
        ls = []
        for hh in range(nh):
            kv = hh // (nh // nkv)
            ls.append(Launch("fdot_nt", lib.tars_fdot,
                             (q.data_ptr() + 4 * hh * hd, 4 * nh * hd, kc.data_ptr() + 4 * kv * hd, 4 * nkv * hd, 0, 0,
                              sc.data_ptr(), 4 * nk, 0, 0, 1, nk, hd), 0, 0, f"h{hh}.scores", {}))
            ls.append(Launch("softmax", lib.tars_row_op,
                             (sc.data_ptr(), 4 * nk, 0, None, None, 0, t0 + 1, None, pr.data_ptr(), 4 * nk, 0, 0, 1, nk),
                             0, 0, f"h{hh}.softmax", {}))
            ls.append(Launch("fdot_nn", lib.tars_fdot,
                             (pr.data_ptr(), 4 * nk, vc.data_ptr() + 4 * kv * hd, 4 * nkv * hd, 1, 0,
                              att.data_ptr() + 4 * hh * hd, 4 * nh * hd, 0, 0, 1, hd, nk), 0, 0, f"h{hh}.pv", {}))
        layers.append(ls)
    return layers, keep, 2 * nk * nkv * hd * 4


def attention_decode(torch, lib, gen, t0: int = 250) -> dict:
    """The decode attention of one token at t=250 over all 28 layers (16 query heads, 8 KV heads,
    head dim 128, fp32 caches of pad16(t0 + 1) rows): op by op through the C ABI (48 launches per
    layer, one graph per token), and as the reference's descriptor queue (1344 descriptors) through
    the executor, whose attention fusion runs each layer's 16 head triples as one launch; us per
    layer and per token."""
    layers, keep, nbytes = attention_layers(torch, lib, gen, t0)
    launches = [l for ls in layers for l in ls]
    g = capture(torch, launches)
    t = time_graph(torch, g, reps=20, warmup=3)
    del g
    r = {"op_by_op": {"launches_per_layer": len(layers[0]), "us_per_layer": round(t / len(layers) * 1e6, 2),
                      "us_per_token": round(t * 1e6, 1), "GBps": round(nbytes * len(layers) / t / 1e9, 1)},
         "t0": t0, "heads": QWEN3_HEADS, "kv_heads": QWEN3_KV_HEADS, "head_dim": QWEN3_HEAD_DIM,
         "layers": QWEN3_LAYERS, "cache_bytes_per_layer": nbytes}
    # the fused attention op (tars_attention): one call per layer for its 16 heads over the same
    # buffers (the split form: a scores launch and a softmax + P V launch)
    nh, nkv, hd = QWEN3_HEADS, QWEN3_KV_HEADS, QWEN3_HEAD_DIM
    nk = (t0 + 1 + 15) // 16 * 16
    ops_l = []
    for kc, vc, q, sc, pr, att in keep:
        arr = lambda vals: (ctypes.c_void_p * nh)(*vals)
        grp = nh // nkv
        ptrs = (arr([q.data_ptr() + 4 * h * hd for h in range(nh)]), arr([kc.data_ptr() + 4 * (h // grp) * hd for h in range(nh)]),
                arr([vc.data_ptr() + 4 * (h // grp) * hd for h in range(nh)]), arr([att.data_ptr() + 4 * h * hd for h in range(nh)]))
        ops_l.append(Launch("attention", lib.tars_attention,
                            (ptrs[0], 4 * nh * hd, ptrs[1], 4 * nkv * hd, ptrs[2], 4 * nkv * hd, 0, ptrs[3], 4 * nh * hd, 0, 0,
                             sc.data_ptr(), 4 * nk, pr.data_ptr(), 4 * nk, nh, 1, nk, hd, t0 + 1), nbytes, 0, "attention",
                            {"ptrs": ptrs}))
    g = capture(torch, ops_l)
    t = time_graph(torch, g, reps=50, warmup=3)
    del g
    r["fused_op"] = {"calls_per_token": len(ops_l), "us_per_layer": round(t / len(ops_l) * 1e6, 2),
                     "us_per_token": round(t * 1e6, 1), "GBps": round(nbytes * len(ops_l) / t / 1e9, 1)}
    del layers, keep, launches, ops_l
    torch.cuda.empty_cache()
    r["executor"] = attention_queue(torch, lib, gen, t0)
    return r


def attention_queue(torch, lib, gen, t0: int) -> dict:
    """The same attention as descriptors in one device DDR image (per layer and head: FDOT_NT into
    the shared scores, causal ROW_SOFTMAX into the shared probabilities, FDOT_NN into the head's
    output columns, tars_mini/llm.py:736-746), run through tars_run_queue; host clock per token."""
    from opentars_amd import _lib, contract as C
    from opentars_amd.queue import encode_descriptor
    nh, nkv, hd = QWEN3_HEADS, QWEN3_KV_HEADS, QWEN3_HEAD_DIM
    nk = (t0 + 1 + 15) // 16 * 16
    top = [0]

    def take(n):
        a = (top[0] + 255) // 256 * 256
        top[0] = a + n
        return a

    descs, fills = [], []
    for _ in range(QWEN3_LAYERS):
        q, kc, vc = take(4 * nh * hd), take(4 * nk * nkv * hd), take(4 * nk * nkv * hd)
        sc, pr, att = take(4 * nk), take(4 * nk), take(4 * nh * hd)
        fills += [(q, nh * hd, 0.1), (kc, nk * nkv * hd, 1.0), (vc, nk * nkv * hd, 1.0)]
        for h in range(nh):
            kv = h // (nh // nkv)
            descs.append(dict(OPCODE=C.OP_FDOT, EPI=C.epi(), A_OFF=q + 4 * h * hd, W_OFF=kc + 4 * kv * hd, Y_OFF=sc,
                              M=1, N=nk, K=hd, GROUP_SIZE=4 * nkv * hd // 16))
            descs.append(dict(OPCODE=C.OP_ROW, CTRL=C.ROW_SOFTMAX, EPI=C.epi(), A_OFF=sc, Y_OFF=pr, M=1, N=nk, K=t0 + 1))
            descs.append(dict(OPCODE=C.OP_FDOT, CTRL=1, EPI=C.epi(), A_OFF=pr, W_OFF=vc + 4 * kv * hd,
                              Y_OFF=att + 4 * h * hd, M=1, N=hd, K=nk, GROUP_SIZE=4 * nkv * hd // 16))
    qaddr = take(64 * len(descs))
    image = torch.zeros(top[0], dtype=torch.uint8, device="cuda")
    for off, n, sd in fills:
        image[off:off + 4 * n].view(torch.float32).copy_(torch.randn(n, device="cuda", generator=gen) * sd)
    host_q = b"".join(encode_descriptor(dict(MAGIC=C.MAGIC, VERSION=C.VERSION, VALID=1, **d)) for d in descs)
    image[qaddr:qaddr + len(host_q)].copy_(torch.frombuffer(bytearray(host_q), dtype=torch.uint8).cuda())
    torch.cuda.synchronize()
    st = _lib.QueueStatus()
    stream = torch.cuda.current_stream().cuda_stream

    def run():
        rc = lib.tars_run_queue(image.data_ptr(), image.numel(), qaddr, len(descs), host_q, 0, 0, ctypes.byref(st),
                                stream)
        if rc != 0 or not st.done:
            raise RuntimeError(f"attention queue: status {rc} done={st.done} err={st.err_code} op={st.op_idx}: "
                               f"{_lib.last_error()}")

    res = {"descriptors": len(descs)}
    for key, fusion, graphs, reps in (("fused_plans", 1, 1, 20), ("fused", 1, 0, 10), ("unfused_plans", 0, 1, 5)):
        prev_f, prev_g = lib.tars_set_queue_fusion(fusion), lib.tars_set_queue_graphs(graphs)
        try:
            for _ in range(3):
                run()
            torch.cuda.synchronize()
            t_start = time.perf_counter()
            for _ in range(reps):
                run()
            torch.cuda.synchronize()
            t = (time.perf_counter() - t_start) / reps
        finally:
            lib.tars_set_queue_fusion(prev_f)
            lib.tars_set_queue_graphs(prev_g)
        # a fused layer is one tars_attention launch group: two kernels in the split form
        res[key] = {"launches_per_token": 2 * QWEN3_LAYERS if fusion else len(descs), "us_per_token": round(t * 1e6, 1),
                    "us_per_layer": round(t / QWEN3_LAYERS * 1e6, 2)}
    del image
    torch.cuda.empty_cache()
    return res


# ------------------------------------------------------------------------------ CPU baseline
def cpu_baseline(launches, target_s: float, spot) -> dict:
    """The numpy oracle (the golden path's own algorithm: the per-token quantizer, int64 matmul and
    the elementwise fp32 epilogue) over the decode-step launches in model order, on this host's CPU,
    single-threaded, until about target_s seconds of compute have passed. Same bytes/s unit. Also
    checks the GPU's timed layer-0 q/k/v outputs (spot = (x, [(W, scol, y), ...])) bit for bit
    against the oracle's."""
    import numpy as np
    from oracle import golden as G
    from oracle import numerics as F

    x0, mats0 = spot
    xq, xs = F.quant_rows(x0)
    exact = all(np.array_equal(y.view(np.uint32), G.gemm_rowcol(xq, xs, W, sc).view(np.uint32))
                for W, sc, y in mats0)

    host = {}

    def operands(i, l):
        if i not in host:             # device -> host copies happen outside the timed calls
            host[i] = {k: v.cpu().numpy() for k, v in l.operands.items()}
        return host[i]

    for i, l in enumerate(launches):
        operands(i, l)
    # one core: the process is pinned to a single CPU for the timed loop (restored afterwards)
    mask = os.sched_getaffinity(0)
    pinned = min(mask)
    os.sched_setaffinity(0, {pinned})
    try:
        elapsed, done_bytes, calls = 0.0, 0, 0
        while elapsed < target_s:
            for i, l in enumerate(launches):
                o = host[i]
                t = time.perf_counter()
                if l.kind == "quant_rows":
                    F.quant_rows(o["x"])
                else:
                    G.gemm_rowcol(o["q"], o["s"], o["W"], o["scol"])
                elapsed += time.perf_counter() - t
                done_bytes += l.nbytes
                calls += 1
                if elapsed >= target_s:
                    break
    finally:
        os.sched_setaffinity(0, mask)
    cpu = cpu_description()
    steps = done_bytes / sum(l.nbytes for l in launches)
    return {"value": round(done_bytes / elapsed / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"numpy oracle over {calls} launches of the decode step in model order "
                      f"({steps:.2f} steps, {elapsed:.1f} s of compute)",
            "bit_exact_spot_check_layer0_qkv": exact,
            "cpu_model": cpu, "os_cpu_count": os.cpu_count(), "pinned_cpu": pinned,
            "threads_env": {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS",
                                                           "MKL_NUM_THREADS")}}


def cpu_description() -> dict:
    """The host CPU as /proc/cpuinfo and lscpu name it (a virtual machine may shorten the model name,
    so the family / model / stepping numbers are reported too)."""
    import subprocess
    info = {"machine": platform.machine()}
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if not line.strip():
                    break
                k, _, v = line.partition(":")
                k = k.strip()
                if k in ("vendor_id", "cpu family", "model", "model name", "stepping", "cpu MHz"):
                    info[k.replace(" ", "_")] = v.strip()
    except OSError:
        pass
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in ("Model name", "BIOS Model name", "Socket(s)", "Core(s) per socket"):
                info["lscpu_" + k.strip().replace(" ", "_").replace("(", "").replace(")", "")] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return info


# ------------------------------------------------------------------------------ main
def main() -> int:
    args = parse()
    if args.pmc_summary:
        return pmc_summary(args.pmc_summary[:4], args.pmc_summary[4], args.pmc_out)
    if args.pmc_step_summary:
        return pmc_step_summary(*args.pmc_step_summary, args.pmc_step_out)
    if args.trace_summary:
        return trace_summary(*args.trace_summary, args.trace_out)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the matrix path runs on a single GPU here (sharding the "
              "output channels over several GPUs is not implemented); use --gpus 1", file=sys.stderr)
        return 2
    import torch
    import opentars_amd

    lib = opentars_amd.lib()
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    torch.cuda.set_device(0)
    torch.backends.cuda.matmul.allow_tf32 = False
    global CONFIG_REPS
    CONFIG_REPS = args.config_reps
    if args.only_configs:
        # a 256 MiB device-to-device copy first: the calibration dispatch for profiler byte counters
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        configs = config_suite(torch, lib, args.seed, attention=False, cpu=not args.no_cpu_baseline)
        out = {"configs": configs}
        if args.detail:
            Path(args.detail).write_text(json.dumps(out, indent=1))
        print(json.dumps(out), flush=True)
        return 0

    log("building the decode-step workload")
    launches, unfused, keep = decode_set(torch, lib, args.seed)
    step_bytes = sum(l.nbytes for l in launches)
    weight_bytes = sum(l.args[10] * l.args[11] for l in unfused if l.kind == "gemm_w8a8")
    graph = capture(torch, launches)
    torch.cuda.synchronize()

    log(f"captured {len(launches)} launches; timing {args.steps} steps")
    # the timed region: W warmup steps, then exactly K steps between synchronizations
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    t_wall = time.perf_counter() - t_wall
    step_s = e0.elapsed_time(e1) / 1e3 / args.steps

    log(f"step {step_s * 1e6:.1f} us; per-row timing")
    rows = marginal_times(torch, graph, launches)
    rows_sum_s = sum(r["us_per_step"] for r in rows.values()) / 1e6
    # the roofline row: the step's largest dispatch (the lm_head, a quarter of the step's bytes);
    # every row is reported beside it
    dom_key = max(rows, key=lambda k: rows[k]["avg_bytes_per_launch"])
    dom = rows[dom_key]
    traffic = None
    tfile = ROOT / "profiles" / "decode_step_traffic.json"
    if tfile.exists():
        entry = json.loads(tfile.read_text()).get("rows", {}).get(dom_key)
        if entry and entry.get("algorithmic_bytes") == dom["avg_bytes_per_launch"]:
            traffic = entry["traffic_bytes"]

    l0 = next(l for l in launches if l.name == "L0.qkv")
    l0_out = [(W.cpu().numpy(), sc.cpu().numpy(), y.cpu().numpy()) for W, sc, y in l0.operands["mats"]]
    l0_x = l0.operands["x"].cpu().numpy()
    # the golden model's unfused sequence (ROW_QUANT + one GEMM per projection), for comparison
    g_unf = capture(torch, unfused)
    unfused_s = time_graph(torch, g_unf, max(3, args.steps // 4), warmup=3)
    del g_unf

    # device copy ceiling for context
    big = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(big)
    for _ in range(2):
        dst.copy_(big)
    torch.cuda.synchronize()
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record()
    for _ in range(5):
        dst.copy_(big)
    c1.record()
    torch.cuda.synchronize()
    copy_gbps = 2 * (1 << 30) * 5 / (c0.elapsed_time(c1) / 1e3) / 1e9
    del big, dst
    torch.cuda.empty_cache()

    log("descriptor-queue executor")
    queue = None if args.no_queue else queue_decode_step(torch, lib, args.seed, max(3, args.steps // 10), 3)
    log("whole decode step through the executor")
    full = None if args.no_queue else full_decode_step(torch, lib, args.seed)
    log("per-config measurements")
    configs = {} if args.no_configs else config_suite(torch, lib, args.seed, cpu=not args.no_cpu_baseline)
    log("cpu baseline")
    cpu = None if args.no_cpu_baseline else cpu_baseline(unfused, args.cpu_seconds, (l0_x, l0_out))

    value = step_bytes / step_s / 1e9
    line = {
        "metric": "W8A8 GEMV HBM GB/s, Qwen3-0.6B decode-step linear set (M=1), bit-exact",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / 11.71, 1),
        "dtype": "int8",
        "data": "synthetic (seeded random int8 weights, per-channel fp32 scales, N(0,1) activations)",
        "config": {"workload": "qwen3-0.6b decode-step W8A8 linear set, M=1: 28 layers x (q,k,v,o,gate,up,down) "
                               "+ lm_head 1024x151936, each with its per-token quantizer fused in",
                   "launches_per_step": len(launches), "weight_bytes": weight_bytes,
                   "algorithmic_bytes_per_step": step_bytes, "graph": True},
        "unfused_golden_sequence": {"launches_per_step": len(unfused), "ms_per_step": round(unfused_s * 1e3, 4),
                                    "GBps": round(sum(l.nbytes for l in unfused) / unfused_s / 1e9, 1)},
        "hbm_frac": round(value * 1e9 / HBM_PEAK, 4),
        "roofline": {"bound": "hbm", "kernel": dom["kernel"],
                     "shape": f"{dom['role']} (1024 -> {QWEN3_VOCAB}, the step's largest dispatch), "
                              f"{dom['grid_items']} work-items",
                     "achieved": dom["GBps"], "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": dom["hbm_frac"],
                     "traffic": traffic, "traffic_source": "profiles/decode_step_traffic.json (rocprofv3 --pmc)",
                     "avg_bytes_per_launch": dom["avg_bytes_per_launch"], "avg_us_per_launch": dom["us_per_launch"],
                     "duration_source": "the launch's cost in the timed step graph: step time less the time of the "
                                        "step without it (HIP events, launch gap included); rocprofv3 kernel-trace "
                                        "durations per row in profiles/decode_step_kernels.md"},
        "roofline_rows": rows,
        "lm_head": {k: configs.get(k) for k in ("lm_head_M1_K1024_N151936", "lm_head_fused_quant_M1_K1024_N151936")},
        # the instances' per-launch times (each instance timed as its own graph, less one replay's
        # fixed cost) summed over a step's launches, beside the step itself
        "rows_sum_us_per_step": round(rows_sum_s * 1e6, 1),
        "device_copy_GBps": round(copy_gbps, 1),
        "queue_executor": queue,
        "queue_whole_decode_step_t250": full,
        "cpu_baseline": cpu,
        "configs": configs,
        "wall_s_timed": round(t_wall, 3),
    }
    if args.detail:
        Path(args.detail).write_text(json.dumps(line, indent=1))
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
