"""Drop-in for the reference's host dispatch (reference/npu.py:41-163), on the GPU.

`NpuDesign` keeps the reference's surface -- buffers 0/1/2 are weights (raw q4nx tile
bytes), x (bf16) and y (fp32); `upload(i, ndarray)`, `run()`, `download(i, dtype, count)`,
`close()`, `meta`, and the `calls`/`seconds` counters -- but a "design" is a GEMV of the
HIP library instead of an xclbin: the weights stay resident in HBM, `run()` launches the
q4 or q8 GEMV and waits for it. `NpuLmHead` and `attach_lm_head` swap a torch lm_head for
the GPU one with the same counters (npu.py:117-163); prefill runs on the GPU too.
"""

from __future__ import annotations

import json
import time
from pathlib import Path

import numpy as np
import torch

from . import _lib, ops
from .q4nx import TILE_BYTES, TILE_K, TILE_ROWS, kind_of_tile_bytes

ARTIFACTS = Path(__file__).resolve().parent.parent / "artifacts"

# Designs the reference exports (tools/export_design.py:52-94): lm_head is Qwen3.5-0.8B's
# q8 projection y[248320] = W[248320, 1024] @ x (designs/lm_head/lm_head.py:35-38).
BUILTIN = {
    "lm_head": {"name": "lm_head", "kind": "q8", "n_rows": 248320, "k": 1024},
}


def _meta_for(name: str, meta: dict | None) -> dict:
    if meta is None:
        f = ARTIFACTS / name / "design.json"
        if f.exists():
            meta = json.loads(f.read_text())
        elif name in BUILTIN:
            meta = dict(BUILTIN[name])
        else:
            raise SystemExit(f"no design {name!r}: pass meta={{kind, n_rows, k}} or write "
                             f"{f}")
    meta = dict(meta)
    n, k = int(meta["n_rows"]), int(meta["k"])
    if n % TILE_ROWS or k % TILE_K:
        raise ValueError(f"design {name}: N={n}, K={k} are not whole 32x256 tiles")
    kind = meta.get("kind")
    if kind is None:   # the reference's design.json has no kind: infer it from the W size
        w_bytes = meta["buffers"][0]
        kind = kind_of_tile_bytes(w_bytes // ((n // TILE_ROWS) * (k // TILE_K)))
    meta["kind"] = kind
    meta["tile_rows"] = n // TILE_ROWS
    meta["buffers"] = [(n // TILE_ROWS) * (k // TILE_K) * TILE_BYTES[kind], k * 2, n * 4]
    return meta


class NpuDesign:
    """One GEMV design resident on the GPU (reference/npu.py:41-114)."""

    def __init__(self, name: str, device=None, meta: dict | None = None):
        self.meta = _meta_for(name, meta)
        self.name = name
        self.device = torch.device(device or "cuda")
        _lib.lib()                          # no silent fallback: the HIP library must load
        self.bos = [torch.zeros(self.meta["buffers"][0], dtype=torch.uint8, device=self.device),
                    torch.zeros(self.meta["k"], dtype=torch.bfloat16, device=self.device),
                    torch.zeros(self.meta["n_rows"], dtype=torch.float32, device=self.device)]
        self.calls = 0
        self.seconds = 0.0

    def upload(self, i: int, data) -> None:
        """Copy host data into buffer i: 0 = weight tile bytes (u8), 1 = x (bf16: uint16
        bits, or float values rounded to bf16), 2 = y (fp32)."""
        bo = self.bos[i]
        if isinstance(data, torch.Tensor):
            src = data.detach().reshape(-1)
        else:
            arr = np.ascontiguousarray(data).reshape(-1)
            if i == 1 and arr.dtype == np.uint16:
                src = torch.from_numpy(arr.view(np.int16).copy()).view(torch.bfloat16)
            else:
                src = torch.from_numpy(arr.copy())
        if i == 0:
            src = src.view(torch.uint8) if src.dtype != torch.uint8 else src
        elif i == 1 and src.dtype != torch.bfloat16:
            src = src.to(torch.float32).to(torch.bfloat16)
        elif i == 2:
            src = src.to(torch.float32)
        if src.numel() != bo.numel():
            raise ValueError(f"buffer {i} holds {bo.numel()} elements, got {src.numel()}")
        bo.copy_(src.to(self.device))

    def run(self) -> None:
        """y = W x on the GPU, synchronously (reference/npu.py:93-97)."""
        m = self.meta
        try:
            ops.gemv(self.bos[0], m["kind"], self.bos[1], m["tile_rows"], m["k"] // TILE_K,
                     out=self.bos[2].view(1, -1))
            torch.cuda.current_stream(self.device).synchronize()
        except _lib.Q4NXError as e:
            raise RuntimeError(f"GPU returned {e}") from e

    def download(self, i: int, dtype, count: int) -> np.ndarray:
        """Copy `count` elements of buffer i back to the host (reference/npu.py:111-114)."""
        t = self.bos[i].reshape(-1)
        raw = t.view(torch.uint8).cpu().numpy().view(np.uint8)
        return np.frombuffer(raw.tobytes()[: count * np.dtype(dtype).itemsize], dtype=dtype)

    def close(self) -> None:
        for attr in ("bos",):
            if hasattr(self, attr):
                delattr(self, attr)


class NpuLmHead(torch.nn.Module):
    """The tied lm_head on the GPU (reference/npu.py:117-150).

    The reference runs one row (decode) on the NPU and hands anything longer (prefill) to the
    torch fallback (npu.py:136-139). Here every row count runs on the GPU: one row on the q8
    contraction the design names, several rows (prefill) on the batched matrix-core
    contraction over the same resident tile bytes. `npu_calls` counts GPU calls,
    `prefill_calls` those with more than one row; `cpu_calls` counts fallback calls, which
    happen only for an input with no rows. The fallback module is kept, as in the reference."""

    def __init__(self, fallback: torch.nn.Module, meta: dict | None = None, device=None):
        super().__init__()
        self.design = NpuDesign("lm_head", device=device, meta=meta)
        self.fallback = fallback
        self.n_rows = self.design.meta["n_rows"]
        self.k = self.design.meta["k"]
        self.npu_calls = 0
        self.prefill_calls = 0
        self.cpu_calls = 0

    def load_weights(self, raw: bytes) -> None:
        self.design.upload(0, np.frombuffer(raw, dtype=np.uint8))

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        rows = h.shape[:-1].numel()
        if rows == 0:
            self.cpu_calls += 1
            return self.fallback(h)
        t = time.perf_counter()
        d = self.design
        x = h.detach().to(torch.float32).reshape(rows, -1).to(torch.bfloat16).to(d.device)
        y = ops.gemm(d.bos[0], d.meta["kind"], x, d.meta["tile_rows"], self.k // TILE_K)
        out = y.reshape(*h.shape[:-1], -1).to(h.device).to(h.dtype)
        if out.is_cuda:
            torch.cuda.current_stream(out.device).synchronize()
        d.seconds += time.perf_counter() - t
        d.calls += 1
        self.npu_calls += 1
        self.prefill_calls += rows > 1
        return out


def attach_lm_head(model, f, meta: dict | None = None) -> NpuLmHead:
    """Swap the model's lm_head for the GPU one and upload its raw tile bytes
    (reference/npu.py:153-163). `f` is a `q4nx.Q4NX` file."""
    e = f.header["lm_head.weight"]
    raw = f.raw("lm_head.weight")
    if meta is None:
        n_t, k_t, tb = e["shape"]
        meta = {"name": "lm_head", "kind": kind_of_tile_bytes(tb), "n_rows": n_t * TILE_ROWS,
                "k": k_t * TILE_K}
    mod = NpuLmHead(model.lm_head, meta=meta)
    mod.load_weights(raw)
    model.lm_head = mod
    return mod
