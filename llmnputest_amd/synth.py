"""Seeded synthetic inputs in the q4nx tile format (no real model files are available).

The generators follow the workload definitions of the decode hot path:

* q4 (GGUF Q4_1) tiles: codes uniform in 0..15 packed two per byte, per-(row, 32-K group)
  bf16 scale d = bf16(|N(0,1)| * 0.02) and minimum m = bf16(-8 * d). -8*d is exact in
  bf16, so "zero-point 8" and the reference's Q4_1 form w = code*d + m coincide
  (tools/q4nx.py:17-26 gives the Q4_1 semantics).
* q8 tiles: int8 codes uniform in [-127, 127], one bf16 scale per (row, 32-K group)
  s = bf16(|N(0,1)| * 0.01) (the stored format carries 256 scales per tile,
  tools/q4nx.py:8, 104-111; a per-256-K scale is the special case of 8 equal groups).
* activations: bf16(N(0,1)).

bf16 values are carried as raw uint16 bits everywhere on the host.
"""

from __future__ import annotations

import numpy as np

from .q4nx import Q4_TILE_BYTES, Q8_TILE_BYTES, TILE_K, TILE_ROWS, tiled_shape


def f32_to_bf16_bits(a) -> np.ndarray:
    """Round float32 to bfloat16 (round-to-nearest-even), returned as uint16 bits."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        rounded = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)
    return rounded


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def random_bf16(rng: np.random.Generator, shape, scale: float = 1.0) -> np.ndarray:
    """bf16(N(0,1) * scale) as uint16 bits."""
    return f32_to_bf16_bits(rng.standard_normal(shape).astype(np.float32) * np.float32(scale))


def q4_tiles(rng: np.random.Generator, n: int, k: int, d_scale: float = 0.02) -> np.ndarray:
    """uint8[n/32, k/256, 5120] of q4 tiles with zero-point-8 Q4_1 metadata."""
    tr, kt = tiled_shape(n, k)
    t = tr * kt
    out = np.empty((t, Q4_TILE_BYTES), dtype=np.uint8)
    out[:, 1024:] = rng.integers(0, 256, size=(t, 4096), dtype=np.uint8)
    d = f32_to_bf16_bits(np.abs(rng.standard_normal((t, 256))).astype(np.float32) * np.float32(d_scale))
    m = f32_to_bf16_bits(bf16_bits_to_f32(d) * np.float32(-8.0))
    out[:, 0:512] = d.view(np.uint8).reshape(t, 512)
    out[:, 512:1024] = m.view(np.uint8).reshape(t, 512)
    return out.reshape(tr, kt, Q4_TILE_BYTES)


def q8_tiles(rng: np.random.Generator, n: int, k: int, s_scale: float = 0.01) -> np.ndarray:
    """uint8[n/32, k/256, 8704] of q8 tiles, codes uniform in [-127, 127]."""
    tr, kt = tiled_shape(n, k)
    t = tr * kt
    out = np.empty((t, Q8_TILE_BYTES), dtype=np.uint8)
    out[:, 512:] = rng.integers(-127, 128, size=(t, 8192), dtype=np.int8).view(np.uint8)
    s = f32_to_bf16_bits(np.abs(rng.standard_normal((t, 256))).astype(np.float32) * np.float32(s_scale))
    out[:, 0:512] = s.view(np.uint8).reshape(t, 512)
    return out.reshape(tr, kt, Q8_TILE_BYTES)


def pack_q4_tile(codes_rk: np.ndarray, d_rk: np.ndarray, m_rk: np.ndarray) -> np.ndarray:
    """Pack one q4 tile from its natural view.

    codes_rk: uint8[32 rows, 256 K] in 0..15; d_rk, m_rk: uint16 bf16 bits [32 rows, 8 groups].
    Returns uint8[5120] laid out as tools/q4nx.py:7-15 describes. Used by tests to build
    tiles with known codes (one row-block / one group / one nibble at a time).
    """
    codes_rk = np.asarray(codes_rk, dtype=np.uint8)
    assert codes_rk.shape == (TILE_ROWS, TILE_K) and codes_rk.max(initial=0) < 16
    tile = np.zeros(Q4_TILE_BYTES, dtype=np.uint8)
    d = np.zeros(256, np.uint16)
    m = np.zeros(256, np.uint16)
    for row in range(TILE_ROWS):
        rb, r = divmod(row, 16)
        for kb in range(8):
            g = kb * 32 + rb * 16 + r
            d[g] = d_rk[row, kb]
            m[g] = m_rk[row, kb]
    tile[0:512] = d.view(np.uint8)
    tile[512:1024] = m.view(np.uint8)
    nib = np.zeros(4096, np.uint8)
    for row in range(TILE_ROWS):
        rb, r = divmod(row, 16)
        for k in range(TILE_K):
            i = rb * 4096 + k * 16 + r
            c = int(codes_rk[row, k])
            if i & 1:
                nib[i >> 1] |= c << 4
            else:
                nib[i >> 1] |= c
    tile[1024:] = nib
    return tile


def quantize_q8(w: np.ndarray) -> np.ndarray:
    """q8 tiles of a float matrix [N, K]: per row and 32-K group s = bf16(max|w| / 127) and
    code = clip(round(w / s), -127, 127), so that code * s -- the q8 dequantisation of
    tools/q4nx.py:140-143 -- is within s/2 of w. FastFlowLM wrote the reference's files; this
    writes the same layout from any weights (a small transformers model's lm_head in the
    tests). Returns uint8[N/32, K/256, 8704]."""
    w = np.asarray(w, np.float32)
    n, k = w.shape
    tr, kt = tiled_shape(n, k)
    grp = w.reshape(n, k // 32, 32)
    s_bits = f32_to_bf16_bits(np.abs(grp).max(-1) / np.float32(127.0))      # [n, k/32]
    s = bf16_bits_to_f32(s_bits)
    safe = np.where(s > 0, s, np.float32(1.0))[..., None]
    codes = np.clip(np.rint(grp / safe), -127, 127).astype(np.int8).reshape(n, k)
    # weight index i = rb*4096 + kk*16 + r of tile (tr, kt): order [tr, kt, rb, kk, r]
    cod = codes.reshape(tr, 2, 16, kt, 256).transpose(0, 3, 1, 4, 2).reshape(tr, kt, 8192)
    # metadata index g = kb*32 + rb*16 + r: order [tr, kt, kb, rb, r]
    meta = s_bits.reshape(tr, 2, 16, kt, 8).transpose(0, 3, 4, 1, 2).reshape(tr, kt, 256)
    out = np.empty((tr, kt, Q8_TILE_BYTES), np.uint8)
    out[..., :512] = np.ascontiguousarray(meta).view(np.uint8)
    out[..., 512:] = np.ascontiguousarray(cod).view(np.uint8)
    return out
