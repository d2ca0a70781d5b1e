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


class Policy(C.Structure):
    """q4nx_policy: which kernel family takes a call and how its work is split (passed per
    call; the library keeps no state). Fields default to q4nx_policy_init's values."""
    _fields_ = [
        ("mfma_rows_q4", c_i),          # q4 rows from which the matrix cores take a call; 0 never
        ("mfma_rows_q8", c_i),          # the same for q8
        ("rowblock", c_i),              # one-row calls on the row-block kernels
        ("gemv_ksplit", c_i),           # general VALU GEMV: K parts per group, 0 automatic
        ("gemv_tiles_per_wave", c_i),   # K-tiles per wave (general and row-block), 0 automatic
        ("gemm_ksplit", c_i),           # matrix-core contraction: K parts, 0 automatic
        ("attn_mfma", c_i),             # attention on the matrix cores
    ]

    def __init__(self, **fields):
        super().__init__()
        lib().q4nx_policy_init(C.byref(self))
        for k, v in fields.items():
            if k not in dict(self._fields_):
                raise AttributeError(f"q4nx_policy has no field {k}")
            setattr(self, k, int(v))

    def replace(self, **fields) -> "Policy":
        d = {k: getattr(self, k) for k, _ in self._fields_}
        d.update(fields)
        return Policy(**d)

    def __repr__(self) -> str:
        return "Policy(" + ", ".join(f"{k}={getattr(self, k)}" for k, _ in self._fields_) + ")"


c_pol = C.POINTER(Policy)

# name -> (restype, argtypes); mirrors include/q4nx_hip.h
SIGNATURES: dict[str, tuple] = {
    "q4nx_abi_version": (c_i, []),
    "q4nx_last_error": (C.c_char_p, []),
    "q4nx_dequant_q4": (c_i, [c_p, c_p, c_i, c_i, c_i, c_i, c_p]),
    "q4nx_dequant_q8": (c_i, [c_p, c_p, c_i, c_i, c_i, c_i, c_p]),
    "q4nx_policy_init": (None, [c_p]),
    "q4nx_gemv_ws_bytes": (c_sz, [c_i, c_i, c_i, c_i, c_pol]),
    "q4nx_gemv_q4": (c_i, [c_p, c_p, c_p, c_i, c_i, c_i, c_i64, c_i64, c_p, c_p, c_sz, c_pol, c_p]),
    "q4nx_gemv_q8": (c_i, [c_p, c_p, c_p, c_i, c_i, c_i, c_i64, c_i64, c_p, c_p, c_sz, c_pol, c_p]),
    "q4nx_gemv_ex": (c_i, [c_i, c_p, c_i, c_i, c_p, c_i64, c_p, c_f, c_p, c_i, c_p, c_i64, c_p,
                           c_p, c_p, c_p, c_sz, c_pol, c_p]),
    "q4nx_gemm_ws_bytes": (c_sz, [c_i, c_i, c_i, c_i, c_pol]),
    "q4nx_gemm": (c_i, [c_i, c_p, c_i, c_i, c_p, c_i64, c_i, c_p, c_i64, c_p, c_p, c_sz, c_pol,
                        c_p]),
    "q4nx_rmsnorm": (c_i, [c_p, c_i, c_p, c_p, c_p, c_i, c_i, c_f, c_p]),
    "q4nx_rope": (c_i, [c_p, c_p, c_p, c_i, c_i, c_i, c_p, c_p, c_i, c_p]),
    "q4nx_rope_table_host": (c_i, [c_p, c_i, c_i, c_d]),
    "q4nx_swiglu": (c_i, [c_p, c_p, c_i, c_p, c_p, c_i, c_i, c_p]),
    "q4nx_qkv_rope_ws_bytes": (c_sz, [c_i, c_i, c_i, c_i, c_pol]),
    "q4nx_qkv_rope": (c_i, [c_p, c_p, c_p, c_i, c_i, c_i, c_p, c_i64, c_p, c_f, c_p, c_i, c_p,
                            c_p, c_i, c_p, c_p, c_p, c_i64, c_i64, c_p, c_p, c_p, c_sz, c_pol,
                            c_p]),
    "q4nx_gate_up_ws_bytes": (c_sz, [c_i, c_i, c_i, c_pol]),
    "q4nx_gate_up_swiglu": (c_i, [c_p, c_p, c_i, c_i, c_p, c_i64, c_p, c_f, c_p, c_i, c_p,
                                  c_i64, c_p, c_p, c_p, c_sz, c_pol, c_p]),
    "q4nx_gqa_decode_ws_bytes": (c_sz, [c_i, c_i, c_i, c_i, c_pol]),
    "q4nx_gqa_decode": (c_i, [c_p, c_p, c_p, c_p, c_p, c_i, c_i, c_i, c_i, c_p, c_i, c_i64,
                              c_i64, c_f, c_i, c_p, c_sz, c_pol, c_p]),
    "q4nx_gqa_decode_static": (c_i, [c_p, c_p, c_p, c_p, c_p, c_i, c_i, c_i, c_i, c_p, c_i,
                                     c_i64, c_i64, c_f, c_i, c_pol, c_p]),
    "q4nx_gqa_decode_splits": (c_i, [c_i, c_i, c_i, c_i, c_pol]),
    "q4nx_gqa_decode_records_splits": (c_i, [c_i, c_i, c_i, c_i, c_pol]),
    "q4nx_gqa_decode_records": (c_i, [c_p, c_p, c_p, c_i, c_i, c_i, c_i, c_p, c_i, c_i64,
                                      c_i64, c_f, c_i, c_p, c_sz, c_pol, c_p]),
    "q4nx_gemv_attn_q4": (c_i, [c_p, c_i, c_p, c_i, c_i, c_i, c_p, c_p, c_p, c_p]),
    "q4nx_gemv_q4_null": (c_i, [c_p, c_p, c_p, c_i, c_i, c_p]),
    "q4nx_stream_read": (c_i, [c_p, c_sz, c_p, c_p]),
    "q4nx_round_bf16": (c_i, [c_p, c_p, c_i64, c_p]),
    "q4nx_embed": (c_i, [c_i, c_p, c_p, c_p, c_p, c_i, c_i, c_i, c_p]),
    "q4nx_argmax": (c_i, [c_p, c_i, c_i, c_i64, c_p, c_p, c_p]),
    "q4nx_decode_advance": (c_i, [c_p, c_i, c_p, c_p, c_p, c_p, c_p, c_i, c_i, c_p]),
    "q4nx_decode_advance_embed": (c_i, [c_p, c_i, c_p, c_p, c_p, c_p, c_p, c_i, c_i, c_i, c_p,
                                        c_i, c_i, c_p, c_p, c_p]),
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
