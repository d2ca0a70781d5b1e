"""Oracle for the q4nx tile format, dequantisation and the q4/q8 GEMV.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Each function restates a reference
function from its source text; bf16 is handled as uint16 bits because the reference's
`ml_dtypes` dependency (tools/q4nx.py:44) is not installed here.

Pins (tests/test_oracle_format.py):
  * bf16 RNE against torch.bfloat16 casts on edge values;
  * dequant against a scalar triple loop over (rb, k, r) written from the format text
    (tools/q4nx.py:10-18), independent of `meta_index`;
  * pack -> dequant round trips with known codes and scales;
  * GEMV against fp64 matmul, one-hot (exact column) and ones (row sums);
  * q4 GEMV against the reference's own cpu_baseline.cpp, compiled from its source into
    oracle/_ref/ (oracle/Makefile), on the same tile bytes.
"""

from __future__ import annotations

import numpy as np

GROUP = 32
TILE_ROWS = 32
TILE_K = 256
ROW_BLOCK = 16
N_WEIGHTS = 8192
Q4_TILE_BYTES = 5120
Q8_TILE_BYTES = 8704
LOW_NIBBLE_IS_EVEN = True      # tools/q4nx.py:56


# ------------------------------------------------------------------ bf16 (RNE) as bits

def bf16_round(a) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even; NaN stays NaN (quiet).

    The reference rounds with ml_dtypes' `astype(bfloat16)`, which is RNE
    (tools/q4nx.py:101, 111)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(a), ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_to_f32(b) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round_f32(a) -> np.ndarray:
    """Round to bf16 and return the value as float32."""
    return bf16_to_f32(bf16_round(a))


# ------------------------------------------------------------------ tile addressing

def meta_index() -> np.ndarray:
    """Metadata index of each of the 8192 weight positions: kb*32 + rb*16 + r
    (tools/q4nx.py:89-94)."""
    i = np.arange(N_WEIGHTS)
    rb, rest = divmod(i, 4096)
    k, r = divmod(rest, ROW_BLOCK)
    return (k // GROUP) * TILE_ROWS + rb * ROW_BLOCK + r


def unpack_nibbles(nib: np.ndarray) -> np.ndarray:
    """uint8[..., 4096] -> uint8[..., 8192] codes in weight-index order
    (tools/q4nx.py:80-86): weight i is byte i>>1, low nibble when i is even."""
    nib = np.asarray(nib, dtype=np.uint8)
    out = np.empty(nib.shape[:-1] + (N_WEIGHTS,), dtype=np.uint8)
    lo, hi = nib & 0x0F, nib >> 4
    first, second = (lo, hi) if LOW_NIBBLE_IS_EVEN else (hi, lo)
    out[..., 0::2], out[..., 1::2] = first, second
    return out


def q4_tiles_f32(b: np.ndarray) -> np.ndarray:
    """[T, 5120] uint8 -> [T, 8192] float32 in weight-index order: w = code*d + m,
    one float32 rounding (tools/q4nx.py:127-137)."""
    b = np.asarray(b, dtype=np.uint8).reshape(-1, Q4_TILE_BYTES)
    d = bf16_to_f32(b[:, 0:512].copy().view(np.uint16))
    m = bf16_to_f32(b[:, 512:1024].copy().view(np.uint16))
    codes = unpack_nibbles(b[:, 1024:]).astype(np.float32)
    g = meta_index()
    return codes * d[:, g] + m[:, g]


def q8_tiles_f32(b: np.ndarray) -> np.ndarray:
    """[T, 8704] uint8 -> [T, 8192] float32: w = int8 * s, exact (tools/q4nx.py:140-143)."""
    b = np.asarray(b, dtype=np.uint8).reshape(-1, Q8_TILE_BYTES)
    s = bf16_to_f32(b[:, 0:512].copy().view(np.uint16))
    return b[:, 512:].view(np.int8).astype(np.float32) * s[:, meta_index()]


def dequant_q4_bf16(b: np.ndarray) -> np.ndarray:
    """[T, 5120] -> bf16 bits [T, 8192]: `dequant_q4` per tile (tools/q4nx.py:97-101)."""
    return bf16_round(q4_tiles_f32(b))


def dequant_q8_bf16(b: np.ndarray) -> np.ndarray:
    """[T, 8704] -> bf16 bits [T, 8192]: `dequant_q8` per tile (tools/q4nx.py:104-111)."""
    return bf16_round(q8_tiles_f32(b))


def untile(flat: np.ndarray, n_t: int, k_t: int) -> np.ndarray:
    """[n_t*k_t, 8192] -> [n_t*32, k_t*256], undoing the row-block interleave
    (tools/q4nx.py:146-149): row = tr*32 + rb*16 + r, column = kt*256 + k."""
    m = flat.reshape(n_t, k_t, 2, TILE_K, ROW_BLOCK).transpose(0, 2, 4, 1, 3)
    return m.reshape(n_t * TILE_ROWS, k_t * TILE_K)


def dequant_matrix(raw: np.ndarray, kind: str, n_t: int, k_t: int) -> np.ndarray:
    """Whole tensor -> float32 [N, K] (`Q4NX.tensor`, tools/q4nx.py:176-197)."""
    b = np.asarray(raw, dtype=np.uint8)
    flat = q4_tiles_f32(b) if kind == "q4" else q8_tiles_f32(b)
    return untile(flat, n_t, k_t)


# ------------------------------------------------------------------ brute force

def dequant_tile_bruteforce(tile: np.ndarray, kind: str) -> np.ndarray:
    """float32 [32, 256] natural view of one tile, by a scalar loop over (rb, k, r)
    written straight from the format description (tools/q4nx.py:10-18) and the kernel
    comments (designs/q4nx_unpack/q4nx_unpack.cc:12-19, designs/lm_head/lm_head.h:21-29).
    Slow; for a few tiles only."""
    t = [int(v) for v in np.asarray(tile, dtype=np.uint8)]
    le16 = lambda off: bf16_to_f32(np.array([t[off] | (t[off + 1] << 8)], np.uint16))[0]
    out = np.empty((32, 256), np.float32)
    for rb in range(2):
        for k in range(256):
            for r in range(16):
                g = (k // 32) * 32 + rb * 16 + r
                if kind == "q4":
                    d = le16(2 * g)
                    m = le16(512 + 2 * g)
                    i = rb * 4096 + k * 16 + r
                    byte = t[1024 + (i >> 1)]
                    code = (byte & 0xF) if (i % 2 == 0) else (byte >> 4)
                    out[rb * 16 + r, k] = np.float32(np.float32(code) * d + m)
                else:
                    s = le16(2 * g)
                    b = t[512 + rb * 4096 + k * 16 + r]
                    code = b - 256 if b >= 128 else b
                    out[rb * 16 + r, k] = np.float32(code) * s
    return out


# ------------------------------------------------------------------ GEMV

def gemv(raw: np.ndarray, kind: str, x_bf16: np.ndarray, n_t: int, k_t: int,
         chunk: int = 256, acc=np.float32) -> np.ndarray:
    """y = W @ x for every token row of x, from the same tile bytes.

    float32 (default) restates `reference()` in designs/granite_gemv/granite_gemv.py:256-271
    and designs/lm_head/lm_head.py:129-144: un-tile, dequantise to float32, matmul in
    float32, chunked over tile-rows. `acc=np.float64` gives the tighter fp64 oracle.
    x_bf16: uint16 bits [K] or [B, K]; returns [N] or [B, N].
    """
    tb = Q4_TILE_BYTES if kind == "q4" else Q8_TILE_BYTES
    b_all = np.asarray(raw, dtype=np.uint8).reshape(n_t * k_t, tb)
    x = bf16_to_f32(np.asarray(x_bf16)).astype(acc)
    squeeze = x.ndim == 1
    x2 = x.reshape(-1, k_t * TILE_K)
    out = np.empty((x2.shape[0], n_t * TILE_ROWS), acc)
    for lo in range(0, n_t, chunk):
        n = min(chunk, n_t - lo)
        w = dequant_matrix(b_all[lo * k_t:(lo + n) * k_t], kind, n, k_t).astype(acc)
        out[:, lo * TILE_ROWS:(lo + n) * TILE_ROWS] = x2 @ w.T
    return out[0] if squeeze else out


def metrics(got, ref) -> tuple[float, float]:
    """(max|got-ref| / max|ref|, cosine), both in float64 (granite_gemv.py:326-335)."""
    g = np.asarray(got, np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    if not r.size:
        return 0.0, 1.0
    scale = np.abs(r).max()
    if not np.isfinite(scale) or scale == 0.0:
        scale = 1.0
    g, r = g / scale, r / scale          # scale-free: tiny or huge outputs compare alike
    rel = float(np.abs(g - r).max())
    den = np.linalg.norm(g) * np.linalg.norm(r)
    cos = float(g @ r / den) if den > 0 else float(np.array_equal(g, r))
    return rel, cos
