"""Write small board exports and the golden model's results on them, for the export loader's
parity tests: tests/golden/export_small.npz (Qwen3), export_qwen35_mtp.npz (Qwen3.5: DeltaNet and
full-attention layers, the MTP head and the speculative-decoding queues) and export_gemma4.npz
(Gemma 4: sliding and full attention, shared KV layers, per-layer token embeddings, the scaled
input embedding). Each holds the files tools/export_kv260.py writes (image.bin, embed_bf16.bin,
ple_bf16.bin, queues.bin, queues_c<n>.bin, queues_s_*.bin, manifest.json) and expected.json.

Two more exports pin the compositions the three above leave open: export_gemma3_ksplit.npz (Gemma 3
with intermediate 4608, so every down projection is two K blocks added in fp32, llm.py:303-321) and
export_gemma4_w4.npz (Gemma 4 lowered with wbits=4: every linear a W4A16 GEMM, the double-wide
down projections as W4 K blocks with their own group scales, llm.py:120-132, 306-313).

The models are the reference's small configurations (qwen_ref.py:43-45, 79-90) with a 512-token
vocabulary and seeded random weights (qwen_ref.random_weights / random_mtp, the embedding tables
rounded to bf16 as the export requires). The descriptor queues and DDR images come from the
reference's own lowering (tars_mini/llm.py QwenLowering, emitted as export_kv260.py:141-247,
250-293 does); the results from the reference's board runtime on its golden backend
(deploy/kv260/sw/tars_board.py Qwen over Golden, recorded as export_kv260.py:320-347 does): per
step the argmax and the SHA-256 of the fp32 logits, and for the MTP export the tokens and verify
rows of speculative rounds. This script imports the reference checkout (read-only, in the build
container only); the .npz files hold data only and the GPU box never runs this.

    python tests/golden/make_export_fixture.py [qwen3|qwen35_mtp|gemma4|gemma3_ksplit|gemma4_w4 ...] \
        [--ref /path/to/reference]
"""
from __future__ import annotations

import argparse
import hashlib
import json
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
T = 40                       # positions
CHUNKS, ALIGN = (8, 4), 4    # prefill chunk sizes and their start alignment (export_kv260.py:48)
HPAGE = 2 << 20
OUT = {"qwen3": "export_small.npz", "qwen35_mtp": "export_qwen35_mtp.npz", "gemma4": "export_gemma4.npz",
       "gemma3_ksplit": "export_gemma3_ksplit.npz", "gemma4_w4": "export_gemma4_w4.npz"}
# token sequences the expected results are recorded on
PROMPTS = [dict(name="plain", ids=[3, 141, 59, 26, 500, 7, 7, 311, 42, 9, 88, 201, 17], new=8),
           dict(name="short", ids=[1, 2], new=6)]
SPEC_NEW = 10                # tokens decoded speculatively after the prompt (MTP export)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> the nearest bf16 value (ties to even), as fp32."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32)


def model(kind: str):
    """(config, weights, lowering options) of a small model."""
    from tars_mini import qwen_ref as Q
    if kind == "qwen3":
        cfg = Q.make_config(Q.CFG_Q3_SMALL, ["full_attention"] * 2, vocab=512)
        return cfg, Q.random_weights(cfg, seed=2026, embed=True), dict(scratch_bytes=1 << 20, queue_cap=160)
    if kind == "qwen35_mtp":
        cfg = Q.make_config(Q.CFG_SMALL, ["linear_attention", "full_attention"], vocab=512)
        w = Q.random_weights(cfg, seed=2027, embed=True)
        w.update(Q.random_mtp(cfg, seed=5))
        return cfg, w, dict(scratch_bytes=1 << 21, verify_rows=2, mtp=True, queue_cap=4096)
    if kind == "gemma3_ksplit":
        # intermediate 4608: every down projection runs as two K blocks [2304, 2304] (as the
        # reference's Gemma 3 test sets it up, tests/test_v04.py:313-317)
        cfg = Q.make_config(dict(Q.CFG_G3_SMALL, intermediate_size=4608), ["sliding_attention", "full_attention"],
                            vocab=512)
        return cfg, Q.random_weights(cfg, seed=2029, embed=True), dict(scratch_bytes=1 << 22, queue_cap=4096)
    if kind == "gemma4_w4":
        # W4A16 linears (llm.py:120-132); intermediate 2304, so the two KV-shared layers' double-wide
        # MLP (4608) runs its down projection as two W4 K blocks with their own group scales
        # (llm.py:306-313); per-layer inputs of 256 (a W4 GEMM needs K >= 256, llm.py:123)
        cfg = Q.make_config(dict(Q.CFG_G4_SMALL, intermediate_size=2304, hidden_size_per_layer_input=256), vocab=512)
        return cfg, Q.random_weights(cfg, seed=2030, embed=True), dict(scratch_bytes=1 << 22, keep_layers=False,
                                                                         queue_cap=4096, wbits=4)
    cfg = Q.make_config(Q.CFG_G4_SMALL, vocab=512)
    return cfg, Q.random_weights(cfg, seed=2028, embed=True), dict(scratch_bytes=1 << 22, keep_layers=False,
                                                                     queue_cap=4096)


def emit(low, path: Path, items) -> list:
    """The queues of items [(key, emitter)] back to back into path: [[key, offset, count], ...]."""
    index, off = [], 0
    with open(path, "wb") as f:
        for key, fn in items:
            a = len(low.p.descs)
            fn()
            b = len(low.p.descs)
            f.write(b"".join(low.p.descs[a:b]))
            index.append([key, off, b - a])
            off += 64 * (b - a)
            del low.p.descs[a:b]
    return index


def write_export(out: Path, kind: str) -> None:
    from tars_mini import llm as L
    cfg, w, opts = model(kind)
    w["embed_tokens.weight"] = emb = bf16_round(w["embed_tokens.weight"])
    ple = w.pop("embed_tokens_per_layer.weight", None)     # host-side only, read by mmap
    low = L.QwenLowering(cfg, w, max_tokens=T, ddr_bytes=1 << 27, head=True, **opts)
    assert low.p.base == 0
    (emb.view(np.uint32) >> 16).astype(np.uint16).tofile(out / "embed_bf16.bin")
    img = bytes(low.p.ddr[:low.end])
    img += bytes((-len(img)) % (1 << 20))
    (out / "image.bin").write_bytes(img)
    index = emit(low, out / "queues.bin", [(t0, lambda t0=t0: low.chunk(t0, 1)) for t0 in range(T)])
    assert all(k <= low.queue_cap for _, _, k in index)
    chunks = {str(n): emit(low, out / f"queues_c{n}.bin",
                           [(t0, lambda t0=t0, n=n: low.chunk(t0, n)) for t0 in range(0, T - n + 1, ALIGN)])
              for n in CHUNKS}
    wbits = opts.get("wbits", 8)
    m = dict(model=f"{kind}-small-random", max_tokens=T, hidden=low.H, vocab=low.vocab, state_dtype="fp32",
             wbits=wbits, min_firmware=0x00040001 if wbits == 4 else 0, keep_layers=low.keep_layers, bos_ids=[], turn_end="<|im_end|>\n",
             embed_scale=float(L.input_embedding(cfg, np.ones((1, 1), np.float32))[0, 0])
             if (low.gemma or low.gemma4) else None,
             image_bytes=len(img), state_end=low.scratch_end, qbase=low.qbase, queue_cap=low.queue_cap,
             x0_off=low.x0.off, x0_ld=low.x0.ld, logits_off=low.logits.off,
             mem_bytes=(len(img) + HPAGE - 1) // HPAGE * HPAGE, chat_prefix="", chat_suffix="", eos_ids=[0],
             queue_index=[[o, k] for _, o, k in index], head_blocks=[lin.n for lin in low.head_lins],
             chunks=chunks)
    if low.ple_dim:
        assert ple is not None
        (bf16_round(ple).view(np.uint32) >> 16).astype(np.uint16).tofile(out / "ple_bf16.bin")
        m.update(ple_cols=len(low.types) * low.ple_dim,
                 ple_scale=float(L.ple_embedding(cfg, np.ones((1, 1), np.float32))[0, 0]),
                 ple0_off=low.ple0.off, ple0_ld=low.ple0.ld)
    if opts.get("mtp"):
        kinds = dict(v2p0=(range(T - 1), lambda r: low.chunk(r, 2, all_rows=True, parity=0, spec=True)),
                     v2p1=(range(T - 1), lambda r: low.chunk(r, 2, all_rows=True, parity=1, spec=True)),
                     m1=(range(T - 1), lambda r: low.mtp_chunk(r, 1)),
                     m2=(range(T - 2), lambda r: low.mtp_chunk(r, 2)),
                     mp1=(range(T - 1), lambda r: low.mtp_chunk(r, 1, head=False)),
                     mp4=(range(0, T - 4, 4), lambda r: low.mtp_chunk(r, 4, head=False)),
                     swap=(range(1), lambda r: low.swap_state()))
        m["spec"] = {name: emit(low, out / f"queues_s_{name}.bin", [(r, lambda r=r, f=f: f(r)) for r in rows])
                     for name, (rows, f) in kinds.items()}
    (out / "manifest.json").write_text(json.dumps(m))


def sha(lg) -> str:
    return hashlib.sha256(np.ascontiguousarray(lg, np.float32).tobytes()).hexdigest()


def record(out: Path, kind: str) -> list:
    import tars_board as B
    dev = B.Golden(mem=json.loads((out / "manifest.json").read_text())["mem_bytes"])
    model_ = B.Qwen(dev, out, log=lambda *a, **k: None)
    res = []
    for p in PROMPTS:
        model_.new_conversation()          # one token a step: the prompt, then greedy
        ids, steps, cur = p["ids"], [], p["ids"][0]
        for i in range(len(ids) + p["new"] - 1):
            lg = model_.step(cur)
            steps.append(dict(pos=i, token=int(cur), argmax=int(np.argmax(lg)), sha256=sha(lg)))
            cur = ids[i + 1] if i + 1 < len(ids) else int(np.argmax(lg))
        model_.new_conversation()          # the prompt in prefill chunks, then two steps
        lg = model_.prefill(ids, chunked=True)
        after = [dict(pos=len(ids) - 1, argmax=int(np.argmax(lg)), sha256=sha(lg))]
        cur = int(np.argmax(lg))
        for i in range(2):
            lg = model_.step(cur)
            after.append(dict(pos=len(ids) + i, token=cur, argmax=int(np.argmax(lg)), sha256=sha(lg)))
            cur = int(np.argmax(lg))
        case = dict(p, steps=steps, prefill=after)
        if model_.spec:                    # speculative decoding after a chunked prefill
            model_.new_conversation()
            lg = model_.prefill(ids, chunked=True)
            cur = model_.begin_spec(lg)
            rounds, toks = [], [cur]
            while len(toks) < SPEC_NEW and model_.can_spec():
                draft = model_.draft
                new, rows = model_.spec_round(cur)
                rounds.append(dict(pos=model_.pos, draft=draft, new=new, rows_sha256=sha(rows)))
                toks += new
                cur = new[-1]
            model_.end_spec()
            case["spec"] = dict(first=toks[0], rounds=rounds, tokens=toks)
        res.append(case)
        print(f"{kind} {p['name']}: {[s['argmax'] for s in steps]}"
              + (f" spec {case['spec']['tokens']}" if "spec" in case else ""), flush=True)
    return res


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("kinds", nargs="*", default=list(OUT))
    ap.add_argument("--ref", default="/root/reference")
    args = ap.parse_args()
    ref = Path(args.ref)
    sys.path.insert(0, str(ref))
    sys.path.insert(0, str(ref / "deploy" / "kv260" / "sw"))
    for kind in args.kinds:
        with tempfile.TemporaryDirectory() as d:
            out = Path(d)
            write_export(out, kind)
            (out / "expected.json").write_text(json.dumps(record(out, kind), indent=1))
            files = {p.name: np.frombuffer(p.read_bytes(), np.uint8) for p in sorted(out.iterdir())}
        dst = HERE / OUT[kind]
        np.savez_compressed(dst, **files)
        print(f"wrote {dst} ({dst.stat().st_size} bytes; {', '.join(f'{k} {v.size}' for k, v in files.items())})")


if __name__ == "__main__":
    main()
