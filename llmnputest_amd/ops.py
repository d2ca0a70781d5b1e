"""Torch-facing wrappers over the C ABI. PyTorch supplies device memory and the stream;
all arithmetic runs in libq4nx_hip.so.

Tensor conventions: tile bytes are torch.uint8 (raw q4nx bytes), bf16 values are
torch.bfloat16 (bit-identical to the uint16 patterns of the C ABI), positions/lengths are
torch.int32. Every tensor must live on the current CUDA (HIP) device. Sums of squares and
argmax keys are kept per 16-row block ([B, N/16]).

Launch policy: every op that chooses between kernel families takes `policy=` (a `Policy`,
the C ABI's q4nx_policy). When it is omitted, the policy of the innermost `policy_scope`
of the calling context applies, else the library's defaults. The scope is a context
variable (per thread / task), so callers that pass their own policy never see another's.
"""

from __future__ import annotations

import contextlib
import contextvars

import numpy as np
import torch

from . import _lib
from ._lib import Policy
from .q4nx import Q4_TILE_BYTES, Q8_TILE_BYTES, Q4NXFormatError

KIND = {"q4": 4, "q8": 8, "bf16": 16}
WS_COUNTER_BYTES = 65536   # Q4NX_WS_COUNTER_BYTES
TILE_BYTES = {"q4": Q4_TILE_BYTES, "q8": Q8_TILE_BYTES}


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_POLICY: contextvars.ContextVar = contextvars.ContextVar("q4nx_policy", default=None)


@contextlib.contextmanager
def policy_scope(policy: Policy | None):
    """Ops called inside the block without an explicit `policy=` use this one."""
    tok = _POLICY.set(policy)
    try:
        yield policy
    finally:
        _POLICY.reset(tok)


def current_policy() -> Policy:
    """The policy an op called here without `policy=` would use."""
    p = _POLICY.get()
    return p if p is not None else Policy()


def _pol(policy: Policy | None):
    p = policy if policy is not None else _POLICY.get()
    return None if p is None else _lib.C.byref(p)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dev(t: torch.Tensor, name: str, dtype=None) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor, got {t.device}")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


class Workspace:
    """Zero-filled device scratch shared by the split-K launches on one stream.

    Kernels that use it leave its counters at zero, so it is zeroed only on (re)allocation.
    """

    def __init__(self, nbytes: int = 0, device=None):
        self.device = torch.device(device or "cuda")
        self.buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=self.device)

    def get(self, nbytes: int) -> tuple[int, int]:
        if nbytes > self.buf.numel():
            self.buf = torch.zeros(nbytes, dtype=torch.uint8, device=self.device)
        return self.buf.data_ptr(), self.buf.numel()


_default_ws: dict = {}


def default_workspace() -> Workspace:
    d = torch.cuda.current_device()
    if d not in _default_ws:
        _default_ws[d] = Workspace(1 << 20, device=f"cuda:{d}")
    return _default_ws[d]


def _tiles(w: torch.Tensor, kind: str, n_tile_rows: int, k_tiles: int, name="w") -> None:
    _dev(w, name, torch.uint8)
    want = n_tile_rows * k_tiles * TILE_BYTES[kind]
    if w.numel() != want:
        raise Q4NXFormatError(f"{name}: {w.numel()} bytes, expected {want} for "
                              f"{n_tile_rows}x{k_tiles} {kind} tiles")


# ---------------------------------------------------------------- dequantisation

def dequant(tiles: torch.Tensor, kind: str, n_tile_rows: int, k_tiles: int,
            out_dtype=torch.bfloat16, untile: bool = False) -> torch.Tensor:
    """Dequantise q4nx tiles on the GPU. out_dtype bfloat16 = `dequant_q4/q8`
    (tools/q4nx.py:97-111); float32 = `_q4_tiles/_q8_tiles` (:127-143). untile=True returns
    the [N, K] matrix (`_untile`, :146-149), else [n_tiles, 8192] in weight-index order."""
    _tiles(tiles, kind, n_tile_rows, k_tiles, "tiles")
    shape = (n_tile_rows * 32, k_tiles * 256) if untile else (n_tile_rows * k_tiles, 8192)
    out = torch.empty(shape, dtype=out_dtype, device=tiles.device)
    f32 = 1 if out_dtype == torch.float32 else 0
    if not f32 and out_dtype != torch.bfloat16:
        raise TypeError("out_dtype must be bfloat16 or float32")
    _lib.call(f"q4nx_dequant_{kind}", _ptr(tiles), _ptr(out), n_tile_rows, k_tiles, f32,
              int(untile), _stream())
    return out


# ---------------------------------------------------------------- GEMV

def gemv_trimmed(tiles: torch.Tensor, kind: str, x: torch.Tensor, n: int, k: int,
                 ws: "Workspace | None" = None, policy: "Policy | None" = None) -> torch.Tensor:
    """y = W @ x for a tensor stored padded to whole tiles (N or K not a tile multiple, as
    tools/q4nx.py:180-184 describes): x bf16 [K] or [B, K] is zero-extended to the stored K
    (the padding columns then add nothing) and the padding rows of y are dropped. Returns
    fp32 [n] or [B, n]."""
    n_t, k_t = -(-n // 32), -(-k // 256)
    _dev(x, "x", torch.bfloat16)
    if x.shape[-1] != k:
        raise Q4NXFormatError(f"x has K={x.shape[-1]}, the tensor has K={k}")
    if k != k_t * 256:
        xp = torch.zeros((*x.shape[:-1], k_t * 256), dtype=torch.bfloat16, device=x.device)
        xp[..., :k] = x
        x = xp
    y = gemv(tiles, kind, x.contiguous(), n_t, k_t, ws=ws, policy=policy)
    return y[..., :n]


def gemv(tiles: torch.Tensor, kind: str, x: torch.Tensor, n_tile_rows: int, k_tiles: int,
         residual: torch.Tensor | None = None, out: torch.Tensor | None = None,
         ws: Workspace | None = None, policy: Policy | None = None) -> torch.Tensor:
    """y = residual + W @ x, fp32. x: bf16 [K] or [B, K]; B <= 8 on the VALU kernels, any B on
    the matrix-core ones (the policy's mfma_rows choose). Returns [N] or [B, N]."""
    _tiles(tiles, kind, n_tile_rows, k_tiles)
    _dev(x, "x", torch.bfloat16)
    squeeze = x.dim() == 1
    x2 = x.reshape(1, -1) if squeeze else x
    b, k = x2.shape
    if k != k_tiles * 256:
        raise Q4NXFormatError(f"x has K={k}, tiles have K={k_tiles * 256}")
    n = n_tile_rows * 32
    if out is None:
        out = torch.empty((b, n), dtype=torch.float32, device=x.device)
    _dev(out, "out", torch.float32)
    if residual is not None:
        _dev(residual, "residual", torch.float32)
        if residual.numel() != b * n:
            raise ValueError("residual must have the shape of the output")
    ws = ws or default_workspace()
    pol = _pol(policy)
    wp, wn = ws.get(_lib.lib().q4nx_gemv_ws_bytes(KIND[kind], n_tile_rows, k_tiles, b, pol))
    _lib.call(f"q4nx_gemv_{kind}", _ptr(tiles), _ptr(x2), _ptr(out), n_tile_rows, k_tiles, b,
              k, n, _ptr(residual), wp, wn, pol, _stream())
    return out.reshape(n) if squeeze else out


def gemm(tiles: torch.Tensor, kind: str, x: torch.Tensor, n_tile_rows: int, k_tiles: int,
         residual: torch.Tensor | None = None, out: torch.Tensor | None = None,
         ws: Workspace | None = None, policy: Policy | None = None) -> torch.Tensor:
    """Y = residual + X @ W^T on the matrix cores, fp32, for any number of rows.
    x: bf16 [M, K] (row stride a multiple of 8) or [K]. Returns [M, N] (or [N])."""
    _tiles(tiles, kind, n_tile_rows, k_tiles)
    if not (x.is_cuda and x.dtype == torch.bfloat16):
        raise ValueError("x must be a bf16 tensor on the GPU")
    squeeze = x.dim() == 1
    x2 = x.reshape(1, -1) if squeeze else x
    if x2.dim() != 2 or x2.stride(1) != 1:
        raise ValueError("x must be [M, K] with unit stride along K")
    m, k = x2.shape
    if k != k_tiles * 256:
        raise Q4NXFormatError(f"x has K={k}, tiles have K={k_tiles * 256}")
    n = n_tile_rows * 32
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=x.device)
    _dev(out, "out", torch.float32)
    if out.numel() != m * n:
        raise ValueError("out must hold [M, N] fp32")
    if residual is not None:
        _dev(residual, "residual", torch.float32)
        if residual.numel() != m * n:
            raise ValueError("residual must have the shape of the output")
    ws = ws or default_workspace()
    pol = _pol(policy)
    wp, wn = ws.get(_lib.lib().q4nx_gemm_ws_bytes(KIND[kind], n_tile_rows, k_tiles, m, pol))
    _lib.call("q4nx_gemm", KIND[kind], _ptr(tiles), n_tile_rows, k_tiles, _ptr(x2), x2.stride(0),
              m, _ptr(out), n, _ptr(residual), wp, wn, pol, _stream())
    return out.reshape(n) if squeeze else out


def _ssq(t, name, b, n):
    if t is not None:
        _dev(t, name, torch.float32)
        if t.numel() < b * n:
            raise ValueError(f"{name} needs batch * {n} entries")


def gemv_ex(tiles: torch.Tensor, kind: str, x: torch.Tensor, n_tile_rows: int, k_tiles: int,
            norm_w: torch.Tensor | None = None, eps: float = 1e-5,
            residual: torch.Tensor | None = None, out: torch.Tensor | None = None,
            argmax_keys: torch.Tensor | None = None, want_y: bool = True,
            ssq_in: torch.Tensor | None = None, ssq_out: torch.Tensor | None = None,
            ws: Workspace | None = None, policy: Policy | None = None):
    """General GEMV: y = residual + W f(x), f = RMSNorm(x; norm_w) when norm_w is given
    (x fp32 [B, K]) else identity (x bf16). argmax_keys: int64 [B, N/16] receives one
    order-preserving (max, first row) key per 16-row block -- reduced by `decode_advance`.
    ssq_out: fp32 [B, N/16] sums of y^2 per 16-row block; ssq_in: the same for x
    ([B, K/16], written by x's producer) so the norm needs no cross-wave reduction."""
    _tiles(tiles, kind, n_tile_rows, k_tiles)
    _dev(x, "x", torch.float32 if norm_w is not None else torch.bfloat16)
    x2 = x.reshape(1, -1) if x.dim() == 1 else x
    b = x2.shape[0]
    n = n_tile_rows * 32
    if norm_w is not None:
        _dev(norm_w, "norm_w", torch.bfloat16)
    if out is None and want_y:
        out = torch.empty((b, n), dtype=torch.float32, device=x.device)
    if argmax_keys is not None:
        _dev(argmax_keys, "argmax_keys", torch.int64)
        if argmax_keys.numel() < b * n_tile_rows * 2:
            raise ValueError("argmax_keys needs batch * N/16 entries")
    _ssq(ssq_in, "ssq_in", b, k_tiles * 16)
    _ssq(ssq_out, "ssq_out", b, n_tile_rows * 2)
    ws = ws or default_workspace()
    pol = _pol(policy)
    wp, wn = ws.get(_lib.lib().q4nx_gemv_ws_bytes(KIND[kind], n_tile_rows, k_tiles, b, pol))
    _lib.call("q4nx_gemv_ex", KIND[kind], _ptr(tiles), n_tile_rows, k_tiles, _ptr(x2),
              x2.shape[1], _ptr(norm_w), float(eps), _ptr(ssq_in), b, _ptr(out), n,
              _ptr(residual), _ptr(ssq_out), _ptr(argmax_keys), wp, wn, pol, _stream())
    return out


def decode_advance(keys: torch.Tensor, n_slots: int, tokens: torch.Tensor, pos: torch.Tensor,
                   lens: torch.Tensor, step: torch.Tensor, history: torch.Tensor | None = None) -> None:
    """tokens = argmax over keys [B, n_slots], pos += 1, lens = pos + 1, history[step] =
    tokens while step < len(history), step += 1 -- one launch, no host round trip."""
    b = tokens.numel()
    hl = 0 if history is None else history.shape[0]
    _lib.call("q4nx_decode_advance", _ptr(keys), int(n_slots), _ptr(tokens), _ptr(pos),
              _ptr(lens), _ptr(history), _ptr(step), hl, b, _stream())


def decode_advance_embed(keys: torch.Tensor, n_slots: int, tokens: torch.Tensor,
                         pos: torch.Tensor, lens: torch.Tensor, step: torch.Tensor,
                         history: torch.Tensor | None, table: torch.Tensor, kind: str, vocab: int,
                         hidden: int, h: torch.Tensor, ssq_out: torch.Tensor | None = None) -> None:
    """`decode_advance`, then `embed` of the new tokens into h (and ssq_out), in one launch."""
    if kind == "bf16":
        _dev(table, "table", torch.bfloat16)
        if table.numel() != vocab * hidden:
            raise ValueError(f"table has {table.numel()} values, expected {vocab}x{hidden}")
    else:
        _tiles(table, kind, vocab // 32, hidden // 256, "table")
    b = tokens.numel()
    _dev(h, "h", torch.float32)
    if h.numel() < b * hidden:
        raise ValueError(f"h holds {h.numel()} values, expected {b}x{hidden}")
    _ssq(ssq_out, "ssq_out", b, hidden // 16)
    hl = 0 if history is None else history.shape[0]
    _lib.call("q4nx_decode_advance_embed", _ptr(keys), int(n_slots), _ptr(tokens), _ptr(pos),
              _ptr(lens), _ptr(history), _ptr(step), hl, b, KIND[kind], _ptr(table), vocab,
              hidden, _ptr(h), _ptr(ssq_out), _stream())


def gemv_q4_null(tiles: torch.Tensor, x: torch.Tensor, n_tile_rows: int, k_tiles: int,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """The weight-stream floor of the batch-1 q4 GEMV: the row-block kernel's grid and loads
    with no arithmetic (the reference's --null design, designs/granite_gemv/granite_gemv.py:
    105-121). `out` receives XOR folds of the loaded bits, not y."""
    _tiles(tiles, "q4", n_tile_rows, k_tiles)
    _dev(x, "x", torch.bfloat16)
    if x.numel() != k_tiles * 256:
        raise Q4NXFormatError(f"x has {x.numel()} values, tiles have K={k_tiles * 256}")
    if out is None:
        out = torch.empty(n_tile_rows * 32, dtype=torch.float32, device=x.device)
    _dev(out, "out", torch.float32)
    if out.numel() < n_tile_rows * 32:
        raise ValueError("out must hold N values")
    _lib.call("q4nx_gemv_q4_null", _ptr(tiles), _ptr(x), _ptr(out), n_tile_rows, k_tiles,
              _stream())
    return out


def stream_read(buf: torch.Tensor, sink: torch.Tensor) -> None:
    """A plain streaming read of every byte of `buf` (contiguous, 16-byte aligned, a multiple
    of 16 bytes); sink: int32 [64] on the same device, written only on a fixed fold value."""
    _dev(buf, "buf")
    _dev(sink, "sink", torch.int32)
    if sink.numel() < 64:
        raise ValueError("sink must hold 64 words")
    nbytes = buf.numel() * buf.element_size()
    _lib.call("q4nx_stream_read", _ptr(buf), nbytes, _ptr(sink), _stream())


def round_bf16(x: torch.Tensor) -> torch.Tensor:
    """bf16 rounding of an fp32 device tensor on the GPU (round to nearest even)."""
    _dev(x, "x", torch.float32)
    y = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    _lib.call("q4nx_round_bf16", _ptr(x), _ptr(y), x.numel(), _stream())
    return y


# ---------------------------------------------------------------- elementwise

def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-5,
            want_f32: bool = False, out: torch.Tensor | None = None):
    """bf16 RMSNorm of x (bf16 or fp32, [C] or [B, C]); returns y or (y, y_f32)."""
    _dev(x, "x")
    _dev(w, "w", torch.bfloat16)
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("x must be bfloat16 or float32")
    cols = x.shape[-1]
    b = x.numel() // cols
    y = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device) if out is None else out
    _dev(y, "out", torch.bfloat16)
    yf = torch.empty(x.shape, dtype=torch.float32, device=x.device) if want_f32 else None
    _lib.call("q4nx_rmsnorm", _ptr(x), int(x.dtype == torch.float32), _ptr(w), _ptr(y),
              _ptr(yf), cols, b, float(eps), _stream())
    return (y, yf) if want_f32 else y


def rope_table(max_pos: int, head_dim: int = 64, theta: float = 10000.0,
               device="cuda") -> torch.Tensor:
    """fp32 [max_pos, 2, head_dim/2] cos/sin table, float64 angles rounded once (host)."""
    tab = np.empty((max_pos, 2, head_dim // 2), np.float32)
    _lib.call("q4nx_rope_table_host", tab.ctypes.data, max_pos, head_dim, float(theta))
    return torch.from_numpy(tab).to(device)


def rope(x: torch.Tensor, positions: torch.Tensor, table: torch.Tensor, want_f32: bool = False,
         out: torch.Tensor | None = None):
    """Half-split RoPE on bf16 x [B, H, D] with per-sequence positions [B]."""
    _dev(x, "x", torch.bfloat16)
    _dev(positions, "positions", torch.int32)
    _dev(table, "table", torch.float32)
    b, h, d = x.shape
    if positions.numel() != b:
        raise ValueError("one position per sequence")
    y = torch.empty_like(x) if out is None else out
    _dev(y, "out", torch.bfloat16)
    yf = torch.empty(x.shape, dtype=torch.float32, device=x.device) if want_f32 else None
    _lib.call("q4nx_rope", _ptr(x), _ptr(y), _ptr(yf), h, d, b, _ptr(positions), _ptr(table),
              table.shape[0], _stream())
    return (y, yf) if want_f32 else y


def swiglu(g: torch.Tensor, u: torch.Tensor, want_f32: bool = False):
    """bf16(silu(g) * u); fp32 g/u are narrowed to bf16 first."""
    _dev(g, "g")
    _dev(u, "u")
    if g.shape != u.shape or g.dtype != u.dtype:
        raise ValueError("g and u must match")
    n = g.shape[-1]
    b = g.numel() // n
    y = torch.empty(g.shape, dtype=torch.bfloat16, device=g.device)
    yf = torch.empty(g.shape, dtype=torch.float32, device=g.device) if want_f32 else None
    _lib.call("q4nx_swiglu", _ptr(g), _ptr(u), int(g.dtype == torch.float32), _ptr(y), _ptr(yf),
              n, b, _stream())
    return (y, yf) if want_f32 else y


# ---------------------------------------------------------------- fused groups

def qkv_rope(wq, wk, wv, n_q_heads: int, n_kv_heads: int, k_tiles: int, x: torch.Tensor,
             positions: torch.Tensor, table: torch.Tensor, k_cache: torch.Tensor,
             v_cache: torch.Tensor, q_out: torch.Tensor | None = None,
             norm_w: torch.Tensor | None = None, eps: float = 1e-5, raw_out=None, xn_out=None,
             ws: Workspace | None = None, ssq_in: torch.Tensor | None = None,
             policy: Policy | None = None) -> torch.Tensor:
    """[q,k,v,RoPE] in one launch. x: bf16 [B, K], or fp32 residual [B, K] with norm_w
    (and its per-16 sums of squares ssq_in [B, K/16], which the one-row kernels need).
    Caches: bf16 [B, Hkv, Lmax, 64]. Returns q_out bf16 [B, Hq*64]."""
    for t, n, kk in ((wq, "wq", n_q_heads), (wk, "wk", n_kv_heads), (wv, "wv", n_kv_heads)):
        _tiles(t, "q4", kk * 2, k_tiles, n)
    _dev(x, "x", torch.float32 if norm_w is not None else torch.bfloat16)
    b = x.shape[0]
    _dev(positions, "positions", torch.int32)
    _dev(k_cache, "k_cache", torch.bfloat16)
    _dev(v_cache, "v_cache", torch.bfloat16)
    if k_cache.shape != v_cache.shape or k_cache.shape[0] < b or k_cache.shape[1] != n_kv_heads \
            or k_cache.shape[3] != 64:
        raise ValueError("caches must be [B, Hkv, Lmax, 64]")
    if q_out is None:
        q_out = torch.empty((b, n_q_heads * 64), dtype=torch.bfloat16, device=x.device)
    if norm_w is not None:
        _dev(norm_w, "norm_w", torch.bfloat16)
    ws = ws or default_workspace()
    pol = _pol(policy)
    wp, wn = ws.get(_lib.lib().q4nx_qkv_rope_ws_bytes(n_q_heads, n_kv_heads, k_tiles, b, pol))
    _ssq(ssq_in, "ssq_in", b, k_tiles * 16)
    lmax = k_cache.shape[2]
    _lib.call("q4nx_qkv_rope", _ptr(wq), _ptr(wk), _ptr(wv), n_q_heads, n_kv_heads, k_tiles,
              _ptr(x), x.shape[1], _ptr(norm_w), float(eps), _ptr(ssq_in), b, _ptr(positions),
              _ptr(table),
              table.shape[0] if table.shape[0] < lmax else lmax, _ptr(q_out), _ptr(k_cache),
              _ptr(v_cache), k_cache.stride(0), k_cache.stride(1), _ptr(raw_out), _ptr(xn_out),
              wp, wn, pol, _stream())
    return q_out


def gate_up_swiglu(wg, wu, n_tile_rows: int, k_tiles: int, x: torch.Tensor,
                   h_out: torch.Tensor | None = None, norm_w: torch.Tensor | None = None,
                   eps: float = 1e-5, raw_out=None, xn_out=None,
                   ws: Workspace | None = None,
                   ssq_in: torch.Tensor | None = None,
                   policy: Policy | None = None) -> torch.Tensor:
    """[gate, up, SwiGLU] in one launch; returns bf16 h [B, N]."""
    _tiles(wg, "q4", n_tile_rows, k_tiles, "wg")
    _tiles(wu, "q4", n_tile_rows, k_tiles, "wu")
    _dev(x, "x", torch.float32 if norm_w is not None else torch.bfloat16)
    b = x.shape[0]
    n = n_tile_rows * 32
    if h_out is None:
        h_out = torch.empty((b, n), dtype=torch.bfloat16, device=x.device)
    ws = ws or default_workspace()
    pol = _pol(policy)
    wp, wn = ws.get(_lib.lib().q4nx_gate_up_ws_bytes(n_tile_rows, k_tiles, b, pol))
    _ssq(ssq_in, "ssq_in", b, k_tiles * 16)
    _lib.call("q4nx_gate_up_swiglu", _ptr(wg), _ptr(wu), n_tile_rows, k_tiles, _ptr(x),
              x.shape[1], _ptr(norm_w), float(eps), _ptr(ssq_in), b, _ptr(h_out), h_out.stride(0),
              _ptr(raw_out), _ptr(xn_out), wp, wn, pol, _stream())
    return h_out


# ---------------------------------------------------------------- attention

def gqa_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
               lens: torch.Tensor, scale: float = 0.125, max_len: int | None = None,
               n_split: int = 0, out: torch.Tensor | None = None, want_f32: bool = False,
               ws: Workspace | None = None, policy: Policy | None = None):
    """GQA flash-decode. q: bf16 [B, Hq, 64]; caches bf16 [B, Hkv, Lmax, 64]; lens int32 [B].
    Returns bf16 [B, Hq, 64] (and the fp32 copy when want_f32). policy.attn_mfma picks the
    matrix-core (default) or the VALU kernel."""
    _dev(q, "q", torch.bfloat16)
    _dev(lens, "lens", torch.int32)
    for t, n in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        if not t.is_cuda or t.dtype != torch.bfloat16 or t.stride(3) != 1 or t.stride(2) != 64:
            raise ValueError(f"{n} must be a bf16 device tensor [B, Hkv, Lmax, 64] with "
                             f"contiguous rows")
    b, hq, d = q.shape
    hkv, lmax = k_cache.shape[1], k_cache.shape[2]
    max_len = lmax if max_len is None else min(max_len, lmax)
    if out is None:
        out = torch.empty((b, hq, d), dtype=torch.bfloat16, device=q.device)
    of = torch.empty((b, hq, d), dtype=torch.float32, device=q.device) if want_f32 else None
    ws = ws or default_workspace()
    pol = _pol(policy)
    need = _lib.lib().q4nx_gqa_decode_ws_bytes(b, hq, hkv, max_len, pol)
    if n_split:
        need = max(need, WS_COUNTER_BYTES + b * hkv * n_split * (hq // hkv) * 68 * 4)
    wp, wn = ws.get(need)
    _lib.call("q4nx_gqa_decode", _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), _ptr(of), b,
              hq, hkv, d, _ptr(lens), max_len, k_cache.stride(0), k_cache.stride(1),
              float(scale), int(n_split), wp, wn, pol, _stream())
    return (out, of) if want_f32 else out


def gqa_decode_splits(batch: int, n_q_heads: int, n_kv_heads: int, max_len: int,
                      policy: Policy | None = None) -> int:
    """The split count `gqa_decode` chooses for n_split=0 under the policy."""
    return int(_lib.lib().q4nx_gqa_decode_splits(batch, n_q_heads, n_kv_heads, max_len,
                                                 _pol(policy)))


def gqa_decode_records_splits(batch: int, n_q_heads: int, n_kv_heads: int,
                              max_len: int, policy: Policy | None = None) -> int:
    """The split count for records that `gemv_attn_q4` merges (the attention policy's, capped
    at 12: fewer, longer splits make the pair faster)."""
    return int(_lib.lib().q4nx_gqa_decode_records_splits(batch, n_q_heads, n_kv_heads, max_len,
                                                         _pol(policy)))


def gqa_decode_records(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       lens: torch.Tensor, n_split: int, scale: float = 0.125,
                       max_len: int | None = None, ws: Workspace | None = None,
                       policy: Policy | None = None) -> torch.Tensor:
    """The publishing half of `gqa_decode`: every split writes its (acc[64], m, l) record and
    nothing is merged. Returns the records, an fp32 view of the workspace shaped
    [B, Hkv, n_split, Hq/Hkv, 68] (valid until the workspace is next used)."""
    _dev(q, "q", torch.bfloat16)
    _dev(lens, "lens", torch.int32)
    for t, n in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        if not t.is_cuda or t.dtype != torch.bfloat16 or t.stride(3) != 1 or t.stride(2) != 64:
            raise ValueError(f"{n} must be a bf16 device tensor [B, Hkv, Lmax, 64] with "
                             f"contiguous rows")
    if n_split < 1:
        raise ValueError("n_split must be >= 1 (see gqa_decode_splits)")
    b, hq, d = q.shape
    hkv, lmax = k_cache.shape[1], k_cache.shape[2]
    max_len = lmax if max_len is None else min(max_len, lmax)
    g = hq // hkv
    pb = b * hkv * n_split * g * 68 * 4
    ws = ws or default_workspace()
    wp, wn = ws.get(WS_COUNTER_BYTES + pb)
    _lib.call("q4nx_gqa_decode_records", _ptr(q), _ptr(k_cache), _ptr(v_cache), b, hq, hkv, d,
              _ptr(lens), max_len, k_cache.stride(0), k_cache.stride(1), float(scale),
              int(n_split), wp, wn, _pol(policy), _stream())
    return ws.buf[WS_COUNTER_BYTES:WS_COUNTER_BYTES + pb].view(torch.float32).view(
        b, hkv, n_split, g, 68)


def gemv_attn_q4(tiles: torch.Tensor, n_tile_rows: int, records: torch.Tensor,
                 residual: torch.Tensor | None = None, out: torch.Tensor | None = None,
                 ssq_out: torch.Tensor | None = None) -> torch.Tensor:
    """Batch-1 o-projection from attention split records: y = residual + W bf16(merge(records)),
    equal bit for bit to `gqa_decode` followed by `gemv_ex`. records: fp32
    [1, Hkv, n_split, Hq/Hkv, 68] from `gqa_decode_records`; W: q4 tiles, K = 64 Hq."""
    _dev(records, "records", torch.float32)
    if records.dim() != 5 or records.shape[0] != 1 or records.shape[4] != 68:
        raise ValueError("records must be [1, Hkv, n_split, Hq/Hkv, 68] (gqa_decode_records)")
    _, hkv, ns, g, _ = records.shape
    hq = hkv * g
    _tiles(tiles, "q4", n_tile_rows, hq // 4)
    n = n_tile_rows * 32
    if out is None:
        out = torch.empty((1, n), dtype=torch.float32, device=records.device)
    _ssq(ssq_out, "ssq_out", 1, n_tile_rows * 2)
    _lib.call("q4nx_gemv_attn_q4", _ptr(tiles), n_tile_rows, _ptr(records), ns, hq, hkv,
              _ptr(out), _ptr(residual), _ptr(ssq_out), _stream())
    return out


# ---------------------------------------------------------------- decode helpers

def embed(table: torch.Tensor, kind: str, tokens: torch.Tensor, vocab: int, hidden: int,
          out: torch.Tensor | None = None,
          ssq_out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 rows `tokens` of a [vocab, hidden] table: kind "bf16" (a stored embedding
    matrix) or "q4" / "q8" tiles (a tied lm_head, dequantised exactly). ssq_out: fp32
    [B, hidden/16] sums of squares for a following RMSNorm."""
    if kind == "bf16":
        _dev(table, "table", torch.bfloat16)
        if table.numel() != vocab * hidden:
            raise ValueError(f"table has {table.numel()} values, expected {vocab}x{hidden}")
    else:
        _tiles(table, kind, vocab // 32, hidden // 256, "table")
    _dev(tokens, "tokens", torch.int32)
    b = tokens.numel()
    if out is None:
        out = torch.empty((b, hidden), dtype=torch.float32, device=table.device)
    _ssq(ssq_out, "ssq_out", b, hidden // 16)
    _lib.call("q4nx_embed", KIND[kind], _ptr(table), _ptr(tokens), _ptr(out), _ptr(ssq_out),
              vocab, hidden, b, _stream())
    return out


def embed_q8(tiles: torch.Tensor, tokens: torch.Tensor, vocab: int, hidden: int,
             out: torch.Tensor | None = None,
             ssq_out: torch.Tensor | None = None) -> torch.Tensor:
    """`embed` of a q8-tiled table."""
    return embed(tiles, "q8", tokens, vocab, hidden, out=out, ssq_out=ssq_out)


def argmax(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    _dev(logits, "logits", torch.float32)
    l2 = logits.reshape(-1, logits.shape[-1])
    b, n = l2.shape
    if out is None:
        out = torch.empty(b, dtype=torch.int32, device=logits.device)
    _lib.call("q4nx_argmax", _ptr(l2), n, b, n, _ptr(out), None, _stream())
    return out
