"""Write tests/golden/export_small.npz: a small board export (the files tools/export_kv260.py
writes: image.bin, embed_bf16.bin, queues.bin, queues_c<n>.bin, manifest.json) and the golden
model's results on it (expected.json), for the export loader's parity tests.

The model is the reference's small Qwen3 configuration (qwen_ref.py:43-45: hidden 256, 4 query
heads / 2 KV heads x 64, MLP 512) with 2 layers, a 512-token vocabulary and seeded random weights
(qwen_ref.random_weights, its embedding rounded to bf16 as the export requires). Its descriptor
queues and DDR image come from the reference's own lowering (tars_mini/llm.py QwenLowering: one
queue per position and the prefill chunk queues, as export_kv260.py:141-247, 273-293 emits them);
the results from the reference's board runtime on its golden backend
(deploy/kv260/sw/tars_board.py Qwen over Golden, as export_kv260.py:320-347 records them): per step
the argmax and the SHA-256 of the fp32 logits. This script imports the reference checkout
(read-only, in the build container only); the .npz holds data only and the GPU box never runs
this.

    python tests/golden/make_export_fixture.py [/path/to/reference]
"""
from __future__ import annotations

import hashlib
import json
import sys
import tempfile
from pathlib import Path

import numpy as np

REF = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
OUT = Path(__file__).resolve().parent / "export_small.npz"

T = 40                       # positions
CHUNKS, ALIGN = (8, 4), 4    # prefill chunk sizes and their start alignment (export_kv260.py:48)
HPAGE = 2 << 20
# token sequences the expected results are recorded on
PROMPTS = [dict(name="plain", ids=[3, 141, 59, 26, 500, 7, 7, 311, 42, 9, 88, 201, 17], new=8),
           dict(name="short", ids=[1, 2], new=6)]


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> the nearest bf16 value (ties to even), as fp32."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32)


def write_export(out: Path) -> None:
    from tars_mini import llm as L
    from tars_mini import qwen_ref as Q
    cfg = Q.make_config(Q.CFG_Q3_SMALL, ["full_attention"] * 2, vocab=512)
    w = Q.random_weights(cfg, seed=2026, embed=True)
    emb = bf16_round(w["embed_tokens.weight"])
    w["embed_tokens.weight"] = emb
    low = L.QwenLowering(cfg, w, max_tokens=T, ddr_bytes=1 << 26, head=True, queue_cap=96,
                         scratch_bytes=1 << 20)
    assert low.p.base == 0
    (emb.view(np.uint32) >> 16).astype(np.uint16).tofile(out / "embed_bf16.bin")
    img = bytes(low.p.ddr[:low.end])
    img += bytes((-len(img)) % (1 << 20))
    (out / "image.bin").write_bytes(img)
    mem_bytes = (len(img) + HPAGE - 1) // HPAGE * HPAGE
    index, off = [], 0
    with open(out / "queues.bin", "wb") as f:
        for t0 in range(T):
            a = len(low.p.descs)
            low.chunk(t0, 1)
            b = len(low.p.descs)
            assert b - a <= low.queue_cap
            f.write(b"".join(low.p.descs[a:b]))
            index.append([off, b - a])
            off += 64 * (b - a)
            del low.p.descs[a:b]
    chunks = {}
    for n in CHUNKS:
        cidx, off = [], 0
        with open(out / f"queues_c{n}.bin", "wb") as f:
            for t0 in range(0, T - n + 1, ALIGN):
                a = len(low.p.descs)
                low.chunk(t0, n)
                b = len(low.p.descs)
                f.write(b"".join(low.p.descs[a:b]))
                cidx.append([t0, off, b - a])
                off += 64 * (b - a)
                del low.p.descs[a:b]
        chunks[str(n)] = cidx
    m = dict(model="qwen3-small-2l-random", max_tokens=T, hidden=low.H, vocab=low.vocab, state_dtype="fp32",
             wbits=8, min_firmware=0, keep_layers=low.keep_layers, bos_ids=[], turn_end="<|im_end|>\n",
             embed_scale=None, image_bytes=len(img), state_end=low.scratch_end, qbase=low.qbase,
             queue_cap=low.queue_cap, x0_off=low.x0.off, x0_ld=low.x0.ld, logits_off=low.logits.off,
             mem_bytes=mem_bytes, chat_prefix="", chat_suffix="", eos_ids=[0], queue_index=index,
             head_blocks=[lin.n for lin in low.head_lins], chunks=chunks)
    (out / "manifest.json").write_text(json.dumps(m))


def record(out: Path) -> list:
    import tars_board as B
    dev = B.Golden(mem=json.loads((out / "manifest.json").read_text())["mem_bytes"])
    model = B.Qwen(dev, out, log=lambda *a, **k: None)
    sha = lambda lg: hashlib.sha256(np.ascontiguousarray(lg, np.float32).tobytes()).hexdigest()
    res = []
    for p in PROMPTS:
        model.new_conversation()          # one token a step: the prompt, then greedy
        ids, steps, cur = p["ids"], [], p["ids"][0]
        for i in range(len(ids) + p["new"] - 1):
            lg = model.step(cur)
            steps.append(dict(pos=i, token=int(cur), argmax=int(np.argmax(lg)), sha256=sha(lg)))
            cur = ids[i + 1] if i + 1 < len(ids) else int(np.argmax(lg))
        model.new_conversation()          # the prompt in prefill chunks, then two steps
        lg = model.prefill(ids, chunked=True)
        after = [dict(pos=len(ids) - 1, argmax=int(np.argmax(lg)), sha256=sha(lg))]
        cur = int(np.argmax(lg))
        for i in range(2):
            lg = model.step(cur)
            after.append(dict(pos=len(ids) + i, token=cur, argmax=int(np.argmax(lg)), sha256=sha(lg)))
            cur = int(np.argmax(lg))
        res.append(dict(p, steps=steps, prefill=after))
        print(f"{p['name']}: {[s['argmax'] for s in steps]}", flush=True)
    return res


def main() -> None:
    sys.path.insert(0, str(REF))
    sys.path.insert(0, str(REF / "deploy" / "kv260" / "sw"))
    with tempfile.TemporaryDirectory() as d:
        out = Path(d)
        write_export(out)
        (out / "expected.json").write_text(json.dumps(record(out), indent=1))
        files = {p.name: np.frombuffer(p.read_bytes(), np.uint8) for p in sorted(out.iterdir())}
    np.savez_compressed(OUT, **files)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes; {', '.join(f'{k} {v.size}' for k, v in files.items())})")


if __name__ == "__main__":
    main()
