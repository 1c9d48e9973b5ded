"""ctypes binding of libopentars_amd.so (the C ABI declared in include/opentars_amd.h).

The library is built in-tree by opentars_amd.build. Loading fails loudly when it is missing:
there is no CPU fallback anywhere in the package.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_int, c_int32, c_int64, c_uint32, c_uint64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libopentars_amd.so"

# Status codes (include/opentars_amd.h)
OK, E_FIELD, E_ALIGN, E_RANGE, E_OVERLAP, E_ARG, E_DEVICE = 0, -6, -7, -8, -9, -10, -11
STATUS_NAMES = {OK: "OK", E_FIELD: "E_FIELD", E_ALIGN: "E_ALIGN", E_RANGE: "E_RANGE",
                E_OVERLAP: "E_OVERLAP", E_ARG: "E_ARG", E_DEVICE: "E_DEVICE"}


class W8A8Out(ctypes.Structure):
    """tars_w8a8_out: one weight matrix fed by a shared quantized activation."""
    _fields_ = [("W", c_void_p), ("scol", c_void_p), ("bias", c_void_p), ("Y", c_void_p),
                ("ldy", c_int64), ("N", c_int32), ("act", c_int32), ("out", c_int32),
                ("out_scale_bits", c_uint32)]


class QueueStatus(ctypes.Structure):
    """tars_queue_status: the end state of a descriptor-queue run."""
    _fields_ = [("done", c_int32), ("err_code", c_int32), ("op_idx", c_int32), ("host_op", c_int32)]


# Every exported entry point: name -> (restype, argtypes)
SIGNATURES = {
    "tars_quant_rows": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int32, c_int32, c_void_p]),
    "tars_gemm_w8a8": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int32, c_void_p,
                               c_void_p, c_int64, c_int32, c_int32, c_int32, c_int32, c_int32, c_uint32,
                               c_void_p]),
    "tars_quant_gemm_w8a8": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int32, c_int32,
                                     ctypes.POINTER(W8A8Out), c_int32, c_void_p]),
    "tars_gemm_w8a8_ksplit": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int32, c_void_p,
                                      c_void_p, c_int64, c_int32, c_int32, c_void_p]),
    "tars_align_w4": (c_int, [c_void_p, c_int64, c_int32, c_void_p, c_int64, c_void_p, c_int64, c_int32,
                              c_int32, c_void_p]),
    "tars_gemm_w4a16": (c_int, [c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                c_int32, c_int32, c_int32, c_int32, c_int32, c_uint32, c_void_p]),
    "tars_version": (c_char_p, []),
    "tars_last_error": (c_char_p, []),
    "tars_set_w8a8_path": (c_int, [c_int]),
    "tars_run_queue": (c_int, [c_void_p, c_uint64, c_uint64, c_int32, c_char_p, c_int32, c_int32,
                               POINTER(QueueStatus), c_void_p]),
    "tars_check_descriptor": (c_int, [c_char_p, c_uint64, c_int32, c_int32, POINTER(c_int32), POINTER(c_int32)]),
    "tars_decode_descriptor": (c_int, [c_char_p, POINTER(c_uint64)]),
    "tars_descriptor_crc": (c_uint32, [c_char_p]),
    "tars_encode_descriptor": (c_int, [POINTER(c_uint64), c_int32, c_void_p]),
    "tars_set_queue_fusion": (c_int, [c_int]),
    "tars_set_queue_graphs": (c_int, [c_int]),
    "tars_row_op": (c_int, [c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_uint32, c_int32, c_void_p, c_void_p,
                            c_int64, c_int32, c_uint32, c_int32, c_int32, c_void_p]),
    "tars_elt": (c_int, [c_void_p, c_int64, c_int32, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int64, c_int32,
                         c_int32, c_void_p, c_int64, c_int32, c_uint32, c_int32, c_int32, c_void_p]),
    "tars_rope": (c_int, [c_void_p, c_int64, c_void_p, c_int32, c_int32, c_void_p, c_int64, c_int32, c_uint32, c_int32,
                          c_int32, c_void_p]),
    "tars_relu": (c_int, [c_void_p, c_int64, c_int32, c_void_p, c_int64, c_int32, c_uint32, c_int32, c_int32, c_void_p]),
    "tars_fdot": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int32, c_int32, c_void_p, c_int64, c_int32, c_uint32,
                          c_int32, c_int32, c_int32, c_void_p]),
    "tars_queue_fusion_counts": (c_int, [POINTER(c_int64), c_int32, c_int32]),
    "tars_embed_rows": (c_int, [c_void_p, c_int64, c_int64, c_int32, POINTER(c_int32), c_int32, c_int32, c_uint32,
                                c_void_p, c_int64, c_void_p]),
    "tars_attention": (c_int, [POINTER(c_void_p), c_int64, POINTER(c_void_p), c_int64, POINTER(c_void_p), c_int64,
                               c_int32, POINTER(c_void_p), c_int64, c_int32, c_uint32, c_void_p, c_int64, c_void_p,
                               c_int64, c_int32, c_int32, c_int32, c_int32, c_int32, c_void_p]),
    "tars_attention_noalloc": (c_int, [POINTER(c_void_p), c_int64, POINTER(c_void_p), c_int64, POINTER(c_void_p),
                                       c_int64, c_int32, POINTER(c_void_p), c_int64, c_int32, c_uint32, c_void_p,
                                       c_int64, c_void_p, c_int64, c_int32, c_int32, c_int32, c_int32, c_int32,
                                       c_void_p]),
}

_lib: ctypes.CDLL | None = None


class LibraryMissing(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """The loaded library (loaded once). Raises LibraryMissing when it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise LibraryMissing(f"{LIB_PATH} is not built; run `python -m opentars_amd.build` "
                                 "(the HIP path has no fallback)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, args
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().tars_last_error().decode()


def version() -> str:
    return lib().tars_version().decode()
