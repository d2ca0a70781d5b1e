"""The q4nx weight container: format constants, tile addressing and the file reader.

This is the host side of the format that tools/q4nx.py documents (tools/q4nx.py:1-34):
a `.q4nx` file is a safetensors file whose quantised tensors are pre-tiled as
`[N/32][K/256][tile bytes]`. One tile covers 32 output rows x 256 K in two
row-blocks of 16:

    q4  5120 B  [bf16 d x256][bf16 m x256][4096 B packed nibbles]   w = code*d + m
    q8  8704 B  [bf16 s x256][8192 B int8]                          w = code*s

    metadata index g = kb*32 + rb*16 + r      (kb = k // 32)
    weight index   i = rb*4096 + k*16 + r     (q4: byte i >> 1, low nibble when i is even)

Nothing here dequantises on the CPU: the product path hands raw tile bytes to the
HIP kernels (`llmnputest_amd.ops`), which read this layout directly in device memory.
"""

from __future__ import annotations

import json
import struct
from pathlib import Path
from typing import BinaryIO

import numpy as np

# tools/q4nx.py:46-56
GROUP = 32            # weights per quantisation group (one K block)
TILE_ROWS = 32        # output rows per tile
TILE_K = 256          # K per tile
ROW_BLOCK = 16        # rows per row-block; a tile holds two
N_META = TILE_ROWS * (TILE_K // GROUP)   # 256 scale entries per plane
N_WEIGHTS = TILE_ROWS * TILE_K           # 8192 weights per tile
Q4_TILE_BYTES = 2 * 2 * N_META + N_WEIGHTS // 2   # 5120
Q8_TILE_BYTES = 2 * N_META + N_WEIGHTS            # 8704
LOW_NIBBLE_IS_EVEN = True   # tools/q4nx.py:56 (measured by the reference against bf16 weights)

Q4 = "q4"
Q8 = "q8"
TILE_BYTES = {Q4: Q4_TILE_BYTES, Q8: Q8_TILE_BYTES}


class Q4NXFormatError(ValueError):
    """A byte count, shape or tile size that does not fit the q4nx tiling."""


def kind_of_tile_bytes(tile_bytes: int) -> str:
    """'q4' or 'q8' for a tile size; anything else is an error (tools/q4nx.py:190-195)."""
    for k, v in TILE_BYTES.items():
        if tile_bytes == v:
            return k
    raise Q4NXFormatError(f"{tile_bytes} B/tile is neither q4 nor q8")


def tiled_shape(n: int, k: int) -> tuple[int, int]:
    """(tile_rows, k_tiles) for a logical [N, K] projection; N % 32 and K % 256 must be 0."""
    if n <= 0 or k <= 0 or n % TILE_ROWS or k % TILE_K:
        raise Q4NXFormatError(f"[{n}, {k}] is not a whole number of {TILE_ROWS}x{TILE_K} tiles")
    return n // TILE_ROWS, k // TILE_K


def padded_shape(n: int, k: int) -> tuple[int, int]:
    """(tile_rows, k_tiles) that store an [N, K] tensor whose N or K need not be a tile
    multiple: the file pads to whole tiles (N=16 is stored as 32 rows) and a reader trims
    the padding back off (tools/q4nx.py:180-197)."""
    if n <= 0 or k <= 0:
        raise Q4NXFormatError(f"[{n}, {k}] is not a tensor shape")
    return -(-n // TILE_ROWS), -(-k // TILE_K)


def tensor_bytes(kind: str, n: int, k: int) -> int:
    tr, kt = tiled_shape(n, k)
    return tr * kt * TILE_BYTES[kind]


def check_tile_bytes(raw_len: int, kind: str, n: int, k: int) -> None:
    """Raise if `raw_len` bytes are not exactly the q4nx tiles of an [N, K] tensor."""
    want = tensor_bytes(kind, n, k)
    if raw_len != want:
        raise Q4NXFormatError(f"{raw_len} bytes, expected {want} B of {kind} tiles for [{n}, {k}]")


def projection_shape(name: str, cfg: dict) -> tuple[int, int]:
    """(N, K) for a tensor name, from the model config, never from the stored shape.

    gate_proj and down_proj are both stored as [2560, 5120] for granite (256 x 10 tiles
    against 80 x 32), so the stored shape alone cannot tell them apart
    (designs/granite_gemv/granite_gemv.py:11-16, 90-102).
    """
    h, i = cfg["hidden_size"], cfg["intermediate_size"]
    hd = cfg.get("head_dim") or h // cfg["num_attention_heads"]
    q = cfg["num_attention_heads"] * hd
    kv = cfg["num_key_value_heads"] * hd
    if name == "lm_head.weight":
        return cfg["vocab_size"], h
    leaf = name.rsplit(".", 2)[-2] if name.endswith(".weight") else name
    table = {
        "q_proj": (q, h), "k_proj": (kv, h), "v_proj": (kv, h), "o_proj": (h, q),
        "gate_proj": (i, h), "up_proj": (i, h), "down_proj": (h, i),
    }
    if leaf not in table:
        raise KeyError(f"no projection shape for {name!r}")
    return table[leaf]


def check_stored_shape(stored, n: int, k: int) -> None:
    """The config-derived factoring must reproduce the stored [tiles, tile_bytes] shape
    (designs/granite_gemv/granite_gemv.py:282-288), padding to whole tiles included. A
    mismatch is an error here, not a skip."""
    tr, kt = padded_shape(n, k)
    if len(stored) == 3:   # [n_t, k_t, bytes]
        ok = stored[0] == tr and stored[1] == kt and stored[2] in (Q4_TILE_BYTES, Q8_TILE_BYTES)
    elif len(stored) == 2:  # [n_t * k_t, bytes]
        ok = stored[0] == tr * kt and stored[1] in (Q4_TILE_BYTES, Q8_TILE_BYTES)
    else:
        ok = False
    if not ok:
        raise Q4NXFormatError(f"config says N={n} K={k} -> {tr}x{kt} tiles, file stores {list(stored)}")


def read_header(f: BinaryIO) -> dict:
    """Parse the safetensors header only (tools/q4nx.py:59-62)."""
    raw = f.read(8)
    if len(raw) != 8:
        raise Q4NXFormatError("file too short for a safetensors header")
    (n,) = struct.unpack("<Q", raw)
    return json.loads(f.read(n))


class Q4NX:
    """A `.q4nx` file: header, names and raw tile bytes (tools/q4nx.py:152-197).

    `raw()` returns the stored bytes untouched; dequantisation happens on the GPU
    (`llmnputest_amd.ops.dequant`). `tiles()` returns a uint8 view shaped
    `[tile_rows * k_tiles, tile_bytes]` without copying the file into Python objects.
    """

    _DT = {"BF16": np.uint16, "F32": np.float32, "F16": np.float16, "I8": np.int8}

    def __init__(self, path):
        self.path = Path(path)
        with self.path.open("rb") as f:
            self.header = read_header(f)
            self._data_start = f.tell()
        self.header.pop("__metadata__", None)

    def __contains__(self, name: str) -> bool:
        return name in self.header

    def names(self) -> list[str]:
        return sorted(self.header)

    def raw(self, name: str) -> bytes:
        first, last = self.header[name]["data_offsets"]
        with self.path.open("rb") as f:
            f.seek(self._data_start + first)
            return f.read(last - first)

    def tiles(self, name: str) -> tuple[str, np.ndarray]:
        """(kind, uint8[n_tiles, tile_bytes]) of a quantised tensor."""
        e = self.header[name]
        if e["dtype"] != "I8":
            raise Q4NXFormatError(f"{name} is stored as {e['dtype']}, not as q4nx tiles")
        shape = e["shape"]
        tile_bytes = shape[-1]
        kind = kind_of_tile_bytes(tile_bytes)
        b = np.frombuffer(self.raw(name), dtype=np.uint8)
        return kind, b.reshape(-1, tile_bytes)

    def tensor(self, name: str, shape: tuple[int, int] | None = None, device="cuda",
               dtype=None):
        """The reference's `Q4NX.tensor` (tools/q4nx.py:176-197) on the GPU: a tiled tensor is
        dequantised and un-tiled by the HIP kernels (bf16 by default, float32 if asked) and
        `shape` = the logical (N, K) trims the tile padding; a plain tensor comes back as
        stored (bf16 as torch.bfloat16). Returns a torch tensor on `device`."""
        import torch
        from . import ops
        e = self.header[name]
        if e["dtype"] != "I8":
            v = self.plain(name)
            t = torch.from_numpy(np.array(v, copy=True))
            if e["dtype"] == "BF16":
                t = t.view(torch.bfloat16)
            return t.to(device)
        kind, tiles = self.tiles(name)
        st = e["shape"]
        n_t, k_t = (st[0], st[1]) if len(st) == 3 else (None, None)
        if shape is not None:
            tr, kt = padded_shape(*shape)
            if n_t is None:
                n_t, k_t = tr, kt
            if (n_t, k_t) != (tr, kt) or n_t * k_t != tiles.shape[0]:
                raise Q4NXFormatError(f"{name}: shape {tuple(shape)} needs {tr}x{kt} tiles, "
                                      f"the file stores {list(st)}")
        elif n_t is None:
            raise Q4NXFormatError(f"{name} is stored as {list(st)}: give its logical shape")
        dev_tiles = torch.from_numpy(np.array(tiles, copy=True)).to(device)
        w = ops.dequant(dev_tiles, kind, n_t, k_t, untile=True,
                        out_dtype=torch.bfloat16 if dtype is None else dtype)
        return w if shape is None else w[: shape[0], : shape[1]]

    def plain(self, name: str) -> np.ndarray:
        """A tensor stored as-is (embeddings, norms): bf16 comes back as raw uint16 bits."""
        e = self.header[name]
        if e["dtype"] == "I8":
            raise Q4NXFormatError(f"{name} is a tiled tensor; use tiles()")
        v = np.frombuffer(self.raw(name), dtype=self._DT[e["dtype"]])
        return v.reshape(e["shape"])


def write_q4nx(path, tensors: dict) -> None:
    """Write a minimal `.q4nx` (safetensors) file.

    `tensors` maps a name to either ("q4"|"q8", uint8[n_t, k_t, tile_bytes]) for tiled
    tensors, or to a numpy array (uint16 is written as BF16). Used to build synthetic
    model files with the same container the reference reads.
    """
    header: dict = {}
    blobs = []
    off = 0
    for name, v in tensors.items():
        if isinstance(v, tuple):
            kind, arr = v
            arr = np.ascontiguousarray(arr, dtype=np.uint8)
            if arr.shape[-1] != TILE_BYTES[kind]:
                raise Q4NXFormatError(f"{name}: last dim {arr.shape[-1]} is not a {kind} tile")
            dtype = "I8"
        else:
            arr = np.ascontiguousarray(v)
            dtype = {np.dtype(np.uint16): "BF16", np.dtype(np.float32): "F32",
                     np.dtype(np.float16): "F16", np.dtype(np.int8): "I8"}[arr.dtype]
        b = arr.tobytes()
        header[name] = {"dtype": dtype, "shape": list(arr.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    hj = json.dumps(header).encode()
    hj += b" " * ((8 - len(hj) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for b in blobs:
            f.write(b)
