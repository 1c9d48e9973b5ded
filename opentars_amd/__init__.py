"""opentars_amd: the openTARS golden model's quantized matrix path on MI355X (gfx950).

HIP kernels behind a C ABI (include/opentars_amd.h, libopentars_amd.so) and Python ops with the
golden model's signatures (opentars_amd.ops). Bit-exact against the golden arithmetic.
"""
from __future__ import annotations

from . import contract
from ._lib import LIB_PATH, LibraryMissing, lib, version

__all__ = ["contract", "LIB_PATH", "LibraryMissing", "lib", "version", "ops"]


def __getattr__(name):
    if name == "ops":                      # torch is imported only when the ops are used
        import importlib
        return importlib.import_module(f"{__name__}.ops")
    raise AttributeError(name)
