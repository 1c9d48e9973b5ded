"""Build libopentars_amd.so in-tree with hipcc for gfx950.

    python -m opentars_amd.build            # or __graft_entry__.build()

Flags that matter for bit-exactness:
  -ffp-contract=off      no multiply-add fusion anywhere: every fp32 step rounds on its own
  (no -ffast-math, no -fgpu-flush-denormals-to-zero): fp32 subnormals are preserved by the
                         hardware and flushed explicitly after each step, as the reference does
  -packed-fp32-ops off   scalar fp32 instructions only
Latency:
  -amdgpu-kernarg-preload-count=16   leading scalar kernel arguments arrive in SGPRs at wave launch
                         (a kernel whose first loads need them issues those loads without a
                         kernel-argument round trip; a compatibility prologue loads them itself
                         where the firmware does not preload)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libopentars_amd.so"
OBJ = PKG / "_build"
SOURCES = ["abi.hip", "queue.hip", "quant_rows.hip", "gemv_w8a8.hip", "gemm_w8a8_mfma.hip", "w4a16.hip",
           "rowops.hip", "embed.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build opentars_amd")


def flags() -> list[str]:
    return [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
            "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-mllvm", "-amdgpu-kernarg-preload-count=16",
            "-Wall", "-Wno-unused-function", "-I", str(PKG.parent / "include")]


_NOISE = "is not a recognized feature for this target"  # the host pass does not know the GPU feature


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in proc.stderr.splitlines() if _NOISE not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source into one shared library next to this file (always rebuilds).

    Each source compiles to its own object in parallel (each carries its own kernels' code
    objects), then one link step writes the library."""
    from concurrent.futures import ThreadPoolExecutor

    OBJ.mkdir(exist_ok=True)
    cc = hipcc()
    objs = [OBJ / (Path(s).stem + ".o") for s in SOURCES]
    cmds = [[cc, *flags(), "-c", str(CSRC / s), "-o", str(o)] for s, o in zip(SOURCES, objs)]
    jobs = jobs or max(1, min(len(cmds), os.cpu_count() or 1, 16))
    with ThreadPoolExecutor(jobs) as pool:
        list(pool.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
