"""ctypes binding of lib/libq4nx_hip.so (declared in include/q4nx_hip.h).

There is no CPU fallback: if the library is missing or does not export a symbol, the
import of the op fails with an error that says how to build it.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("Q4NX_LIB", Path(__file__).resolve().parent / "lib" / "libq4nx_hip.so"))

c_p = C.c_void_p
c_i = C.c_int
c_i64 = C.c_int64
c_sz = C.c_size_t
c_f = C.c_float
c_d = C.c_double

# name -> (restype, argtypes); mirrors include/q4nx_hip.h
SIGNATURES: dict[str, tuple] = {
    "q4nx_abi_version": (c_i, []),
    "q4nx_last_error": (C.c_char_p, []),
    "q4nx_dequant_q4": (c_i, [c_p, c_p, c_i, c_i, c_i, c_i, c_p]),
    "q4nx_dequant_q8": (c_i, [c_p, c_p, c_i, c_i, c_i, c_i, c_p]),
    "q4nx_gemv_ws_bytes": (c_sz, [c_i, c_i, c_i, c_i]),
    "q4nx_gemv_q4": (c_i, [c_p, c_p, c_p, c_i, c_i, c_i, c_i64, c_i64, c_p, c_p, c_sz, c_p]),
    "q4nx_gemv_q8": (c_i, [c_p, c_p, c_p, c_i, c_i, c_i, c_i64, c_i64, c_p, c_p, c_sz, c_p]),
    "q4nx_gemv_ex": (c_i, [c_i, c_p, c_i, c_i, c_p, c_i64, c_p, c_f, c_p, c_i, c_p, c_i64, c_p,
                           c_p, c_p, c_p, c_sz, c_p]),
    "q4nx_set_split_tiles": (c_i, [c_i]),
    "q4nx_set_gemv_ksplit": (c_i, [c_i]),
    "q4nx_gemm_ws_bytes": (c_sz, [c_i, c_i, c_i, c_i]),
    "q4nx_gemm": (c_i, [c_i, c_p, c_i, c_i, c_p, c_i64, c_i, c_p, c_i64, c_p, c_p, c_sz, c_p]),
    "q4nx_set_gemm_ksplit": (c_i, [c_i]),
    "q4nx_set_mfma_rows": (c_i, [c_i, c_i]),
    "q4nx_rmsnorm": (c_i, [c_p, c_i, c_p, c_p, c_p, c_i, c_i, c_f, c_p]),
    "q4nx_rope": (c_i, [c_p, c_p, c_p, c_i, c_i, c_i, c_p, c_p, c_i, c_p]),
    "q4nx_rope_table_host": (c_i, [c_p, c_i, c_i, c_d]),
    "q4nx_swiglu": (c_i, [c_p, c_p, c_i, c_p, c_p, c_i, c_i, c_p]),
    "q4nx_qkv_rope_ws_bytes": (c_sz, [c_i, c_i, c_i, c_i]),
    "q4nx_qkv_rope": (c_i, [c_p, c_p, c_p, c_i, c_i, c_i, c_p, c_i64, c_p, c_f, c_p, c_i, c_p,
                            c_p, c_i, c_p, c_p, c_p, c_i64, c_i64, c_p, c_p, c_p, c_sz, c_p]),
    "q4nx_gate_up_ws_bytes": (c_sz, [c_i, c_i, c_i]),
    "q4nx_gate_up_swiglu": (c_i, [c_p, c_p, c_i, c_i, c_p, c_i64, c_p, c_f, c_p, c_i, c_p,
                                  c_i64, c_p, c_p, c_p, c_sz, c_p]),
    "q4nx_layer_tail_ws_bytes": (c_sz, [c_i, c_i, c_i, c_i]),
    "q4nx_layer_tail": (c_i, [c_p, c_p, c_p, c_p, c_i, c_i, c_i, c_p, c_p, c_p, c_p, c_f, c_p, c_i,
                              c_p, c_sz, c_p]),
    "q4nx_ws_check": (c_i, [c_p, c_p]),
    "q4nx_gqa_decode_ws_bytes": (c_sz, [c_i, c_i, c_i, c_i]),
    "q4nx_set_attn_mfma": (c_i, [c_i]),
    "q4nx_gqa_decode": (c_i, [c_p, c_p, c_p, c_p, c_p, c_i, c_i, c_i, c_i, c_p, c_i, c_i64,
                              c_i64, c_f, c_i, c_p, c_sz, c_p]),
    "q4nx_gqa_decode_splits": (c_i, [c_i, c_i, c_i, c_i]),
    "q4nx_gqa_decode_records_splits": (c_i, [c_i, c_i, c_i, c_i]),
    "q4nx_gqa_decode_records": (c_i, [c_p, c_p, c_p, c_i, c_i, c_i, c_i, c_p, c_i, c_i64,
                                      c_i64, c_f, c_i, c_p, c_sz, c_p]),
    "q4nx_gemv_attn_q4": (c_i, [c_p, c_i, c_p, c_i, c_i, c_i, c_p, c_p, c_p, c_p]),
    "q4nx_round_bf16": (c_i, [c_p, c_p, c_i64, c_p]),
    "q4nx_embed_q8": (c_i, [c_p, c_p, c_p, c_p, c_i, c_i, c_i, c_p]),
    "q4nx_argmax": (c_i, [c_p, c_i, c_i, c_i64, c_p, c_p, c_p]),
    "q4nx_decode_advance": (c_i, [c_p, c_i, c_p, c_p, c_p, c_p, c_p, c_i, c_i, c_p]),
}

_lib = None


class Q4NXError(RuntimeError):
    """A non-zero return code from the HIP library, with its message."""

    def __init__(self, rc: int, msg: str):
        super().__init__(f"[{rc}] {msg}")
        self.rc = rc


def lib():
    """The loaded library. Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP extension first "
                f"(python -m llmnputest_amd.build, or __graft_entry__.build())")
        h = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)        # AttributeError if the symbol is not exported
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise Q4NXError(rc, lib().q4nx_last_error().decode(errors="replace"))


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
