"""ctypes binding of oracle/liboracle_cpu.so (cpu_oracle.c) and of the reference's own CPU
GEMV binary oracle/_ref/cpu_baseline. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py)."""

from __future__ import annotations

import ctypes as C
import os
import re
import subprocess
import tempfile
from pathlib import Path

import numpy as np

from . import q4nx_oracle as qo

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle_cpu.so"
REF_BASELINE = HERE / "_ref" / "cpu_baseline"

_lib = None


def build() -> None:
    """Build liboracle_cpu.so (and _ref/cpu_baseline when the reference is mounted)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        h = C.CDLL(str(LIB))
        h.oracle_gemv.restype = C.c_int
        h.oracle_gemv.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int,
                                  C.c_void_p, C.c_int]
        h.cpu_q8_gemv.restype = C.c_int
        h.cpu_q8_gemv.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_int]
        h.cpu_gqa_decode.restype = C.c_int
        h.cpu_gqa_decode.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                     C.c_int, C.c_int, C.c_int, C.c_float, C.c_int]
        _lib = h
    return _lib


def host_threads() -> int:
    return len(os.sched_getaffinity(0))


def gemv(raw: np.ndarray, kind: str, x_bf16: np.ndarray, n_t: int, k_t: int,
         threads: int | None = None) -> np.ndarray:
    """float64 GEMV from tile bytes (same values as q4nx_oracle.gemv(acc=float64))."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = qo.bf16_to_f32(np.asarray(x_bf16))
    squeeze = x.ndim == 1
    x2 = np.ascontiguousarray(x.reshape(-1, k_t * 256), dtype=np.float32)
    y = np.empty((x2.shape[0], n_t * 32), np.float64)
    rc = lib().oracle_gemv(raw.ctypes.data, 4 if kind == "q4" else 8, n_t, k_t, x2.ctypes.data,
                           x2.shape[0], y.ctypes.data, threads or host_threads())
    if rc != 0:
        raise ValueError("oracle_gemv: bad arguments")
    return y[0] if squeeze else y


def run_ref_baseline(raw: np.ndarray, n_t: int, k_t: int, threads: int, iters: int) -> dict:
    """Run the reference's cpu_baseline on these q4 tile bytes (written to a temp file).

    Its activation is fixed at x[i] = ((i*37 % 101) - 50)/50 (cpu_baseline.cpp:143); it
    prints STREAM and GEMV milliseconds and y[0..3]."""
    if not REF_BASELINE.exists():
        raise FileNotFoundError(REF_BASELINE)
    with tempfile.NamedTemporaryFile(suffix=".q4tiles", delete=False) as f:
        f.write(np.ascontiguousarray(raw, np.uint8).tobytes())
        path = f.name
    try:
        out = subprocess.run([str(REF_BASELINE), path, "0", str(n_t), str(k_t), str(threads),
                              str(iters)], capture_output=True, text=True, check=True).stdout
    finally:
        os.unlink(path)
    res = {"threads": int(re.search(r"threads\s+(\d+)", out).group(1))}
    m = re.search(r"STREAM\s+([\d.]+) ms\s+([\d.]+) GB/s", out)
    res["stream_ms"], res["stream_gbs"] = float(m.group(1)), float(m.group(2))
    m = re.search(r"GEMV\s+([\d.]+) ms\s+([\d.]+) GB/s", out)
    res["gemv_ms"], res["gemv_gbs"] = float(m.group(1)), float(m.group(2))
    res["y0_3"] = [float(v) for v in re.search(r"y\[0\.\.3\]\s+(.*)", out).group(1).split()]
    return res


def ref_baseline_x(k: int) -> np.ndarray:
    """The reference baseline's activation, float32 (cpu_baseline.cpp:143)."""
    i = np.arange(k)
    return (((i * 37) % 101) - 50).astype(np.float32) / np.float32(50.0)


def q8_baseline_gemv(raw: np.ndarray, x_bf16: np.ndarray, n_t: int, k_t: int,
                     threads: int | None = None) -> np.ndarray:
    """fp32 y = W x for one token from q8 tile bytes: the AVX2 CPU baseline
    (cpu_q8_baseline.c, the method of designs/granite_gemv/cpu_baseline.cpp on the q8
    tile)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    if raw.size != n_t * k_t * qo.Q8_TILE_BYTES:
        raise ValueError("raw does not hold n_t x k_t q8 tiles")
    x = np.ascontiguousarray(qo.bf16_to_f32(np.asarray(x_bf16)).reshape(k_t * 256),
                             dtype=np.float32)
    y = np.empty(n_t * 32, np.float32)
    rc = lib().cpu_q8_gemv(raw.ctypes.data, n_t, k_t, x.ctypes.data, y.ctypes.data,
                           threads or host_threads())
    if rc != 0:
        raise ValueError("cpu_q8_gemv: bad arguments")
    return y


def gqa_decode(q: np.ndarray, k_bits: np.ndarray, v_bits: np.ndarray, length: int,
               scale: float = 0.125, threads: int | None = None) -> np.ndarray:
    """fp32 GQA decode attention of one token on the CPU (cpu_attn.c, AVX2, one thread per
    core over the query heads): q fp32 [Hq, 64]; K/V bf16 bits [Hkv, L, 64], positions
    [0, length). Returns fp32 [Hq, 64]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k_bits, dtype=np.uint16)
    v = np.ascontiguousarray(v_bits, dtype=np.uint16)
    hq, hkv, lstride = q.shape[0], k.shape[0], k.shape[1]
    if q.shape[1] != 64 or k.shape != v.shape or k.shape[2] != 64 or not 0 < length <= lstride:
        raise ValueError("q [Hq, 64], K/V [Hkv, L, 64], 0 < length <= L")
    out = np.empty((hq, 64), np.float32)
    rc = lib().cpu_gqa_decode(q.ctypes.data, k.ctypes.data, v.ctypes.data, out.ctypes.data, hq,
                              hkv, int(length), lstride, float(scale), threads or host_threads())
    if rc != 0:
        raise ValueError(f"cpu_gqa_decode: error {rc}")
    return out
