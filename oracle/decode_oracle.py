"""Oracle for the decode ops around the GEMV: RMSNorm, RoPE, SwiGLU, GQA decode
attention, the fused groups, and the granite-shaped decode step built from them.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The reference writes each op's check as a float64 numpy formula; these functions restate
those formulas (file:line given per function). Where an op's output is bf16, the oracle
returns the float64 value *before* rounding and the caller compares either the kernel's
fp32 pre-rounding output at 1e-5 or its bf16 output by ulp-mismatch count.

Conventions the reference leaves open and the build fixes:
  * RoPE cos/sin come from a float64 table rounded once to float32 and indexed by
    position (the reference passes cos/sin in from the host,
    designs/granite_gemv/granite_elementwise.h:45-47);
  * q and k are narrowed to bf16 before the rotation, v is only narrowed
    (designs/granite_gemv/granite_qkv_rope.h:37-69);
  * gate/up are narrowed to bf16 before SwiGLU and the product is narrowed again
    (designs/granite_gemv/granite_mlp_full.py:231-237);
  * GQA maps q head h to kv head h // (Hq // Hkv);
  * decode step (no token loop exists in the reference): fp32 residual stream,
    pre-norm Llama/Granite order, final RMSNorm, tied q8 lm_head whose dequantised
    row t is also the embedding of token t.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import q4nx_oracle as qo


def f64(a):
    return np.asarray(a, dtype=np.float64)


# ------------------------------------------------------------------ RMSNorm

def rmsnorm(x, w_bf16, eps: float = 1e-5) -> np.ndarray:
    """y = x * (1/sqrt(mean(x^2) + eps)) * w in float64
    (designs/granite_gemv/granite_rmsnorm.py:112-113, granite_rmsnorm.h:45-80).
    x: float values [..., C] (bf16-decoded or fp32 residual); w: bf16 bits [C]."""
    xf = f64(x)
    wf = f64(qo.bf16_to_f32(w_bf16))
    inv = 1.0 / np.sqrt((xf * xf).mean(axis=-1, keepdims=True) + eps)
    return xf * inv * wf


# ------------------------------------------------------------------ RoPE

def rope_inv_freq(head_dim: int, theta: float) -> np.ndarray:
    """1/theta^(2i/hd), float64 (designs/granite_gemv/granite_elementwise.py:135-136)."""
    half = head_dim // 2
    return 1.0 / (theta ** (np.arange(0, half, dtype=np.float64) * 2.0 / head_dim))


def rope_table(max_pos: int, head_dim: int, theta: float) -> np.ndarray:
    """float32 [max_pos, 2, half]: cos then sin of pos*inv_freq, computed in float64 and
    rounded once (positions up to 2^15 keep the angle exact in float64)."""
    inv = rope_inv_freq(head_dim, theta)
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * inv[None, :]
    return np.stack([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)


def rope(x, pos, table: np.ndarray) -> np.ndarray:
    """Half-split `rotate_half` RoPE in float64 with the float32 table values
    (designs/granite_gemv/granite_elementwise.h:40-75; reference check
    granite_elementwise.py:146-151).
    x: [..., n_heads, hd] values; pos: int or int array broadcast over the leading dims."""
    xf = f64(x)
    half = xf.shape[-1] // 2
    cs = f64(table[np.asarray(pos)])          # [..., 2, half]
    c = cs[..., 0, :][..., None, :]
    s = cs[..., 1, :][..., None, :]
    lo, hi = xf[..., :half], xf[..., half:]
    return np.concatenate([lo * c - hi * s, hi * c + lo * s], axis=-1)


def rope_interleaved(x, pos, table: np.ndarray) -> np.ndarray:
    """The GPT-NeoX interleaved-pair convention, which must NOT match
    (designs/granite_gemv/granite_elementwise.py:153-162)."""
    xf = f64(x)
    cs = f64(table[np.asarray(pos)])
    c = cs[..., 0, :][..., None, :]
    s = cs[..., 1, :][..., None, :]
    e, o = xf[..., 0::2], xf[..., 1::2]
    out = np.empty_like(xf)
    out[..., 0::2] = e * c - o * s
    out[..., 1::2] = e * s + o * c
    return out


# ------------------------------------------------------------------ SwiGLU

def swiglu(g, u) -> np.ndarray:
    """h = g / (1 + exp(-g)) * u in float64 (designs/granite_gemv/granite_elementwise.py:172-174)."""
    gf, uf = f64(g), f64(u)
    return (gf / (1.0 + np.exp(-gf))) * uf


# ------------------------------------------------------------------ attention

def gqa_attention(q, k, v, lens=None, scale: float = 0.125) -> np.ndarray:
    """GQA decode attention in float64 (designs/granite_gemv/granite_attention.py:163-167).

    q: [B, Hq, D]; k, v: [B, Hkv, L, D]; lens: valid positions per sequence (default L).
    Returns [B, Hq, D]."""
    qf, kf, vf = f64(q), f64(k), f64(v)
    b_n, hq, d = qf.shape
    hkv = kf.shape[1]
    grp = hq // hkv
    out = np.empty((b_n, hq, d))
    for b in range(b_n):
        n = kf.shape[2] if lens is None else int(lens[b])
        for h in range(hq):
            j = h // grp
            s = (kf[b, j, :n] @ qf[b, h]) * scale
            p = np.exp(s - s.max())
            out[b, h] = (p / p.sum()) @ vf[b, j, :n]
    return out


# ------------------------------------------------------------------ fused groups

def qkv_rope_from_raw(q_raw, k_raw, v_raw, pos, table, hd: int = 64):
    """RoPE epilogue on fp32 GEMV outputs: narrow to bf16, rotate q and k, narrow v.
    q_raw: [B, Hq*hd]; k_raw, v_raw: [B, Hkv*hd]; pos: [B]. Returns fp64 (q, k, v)."""
    b_n = q_raw.shape[0]
    qb = f64(qo.bf16_round_f32(q_raw)).reshape(b_n, -1, hd)
    kb = f64(qo.bf16_round_f32(k_raw)).reshape(b_n, -1, hd)
    pos = np.asarray(pos).reshape(b_n)
    qr = np.stack([rope(qb[b], pos[b], table) for b in range(b_n)])
    kr = np.stack([rope(kb[b], pos[b], table) for b in range(b_n)])
    vr = f64(qo.bf16_round_f32(v_raw)).reshape(b_n, -1, hd)
    return qr, kr, vr


def swiglu_from_raw(g_raw, u_raw) -> np.ndarray:
    """[gate, up, SwiGLU] epilogue on fp32 GEMV outputs (granite_mlp.py:172-181):
    g, u narrowed to bf16, then silu(g)*u in float64 (narrowed by the caller)."""
    return swiglu(qo.bf16_round_f32(g_raw), qo.bf16_round_f32(u_raw))


# ------------------------------------------------------------------ decode step

@dataclass
class DecodeConfig:
    hidden: int = 2560
    inter: int = 8192
    n_layers: int = 40
    n_q: int = 40
    n_kv: int = 8
    head_dim: int = 64
    vocab: int = 100352
    eps: float = 1e-5
    theta: float = 10000.0
    scale: float = 0.125


@dataclass
class DecodeWeights:
    """Raw tile bytes per layer (uint8 [n_t*k_t, tile_bytes]) and bf16 norm weights."""
    cfg: DecodeConfig
    wq: list = field(default_factory=list)
    wk: list = field(default_factory=list)
    wv: list = field(default_factory=list)
    wo: list = field(default_factory=list)
    wg: list = field(default_factory=list)
    wu: list = field(default_factory=list)
    wd: list = field(default_factory=list)
    norm_in: list = field(default_factory=list)
    norm_post: list = field(default_factory=list)
    norm_final: np.ndarray | None = None
    lm_head: np.ndarray | None = None       # q8 tiles [vocab/32 * hidden/256, 8704]


def embed_rows(lm_head_raw: np.ndarray, tokens, vocab: int, hidden: int) -> np.ndarray:
    """Tied embedding: row t of the dequantised q8 lm_head, float32 [len(tokens), hidden]."""
    k_t = hidden // 256
    tiles = np.asarray(lm_head_raw, np.uint8).reshape(vocab // 32, k_t, qo.Q8_TILE_BYTES)
    out = []
    for t in np.asarray(tokens).ravel():
        w = qo.dequant_matrix(tiles[t // 32].reshape(k_t, -1), "q8", 1, k_t)
        out.append(w[t % 32])
    return np.stack(out).astype(np.float32)


class DecodeOracle:
    """Numpy decode step in the conventions of the module docstring. Pure float64 /
    float32 reference with bf16 narrowing at the same points as the GPU path; slow,
    meant for reduced layer counts in tests."""

    def __init__(self, w: DecodeWeights, k_cache: list, v_cache: list, max_pos: int,
                 gemv=None):
        self.w = w
        self.cfg = w.cfg
        self.k_cache = k_cache      # per layer: bf16 bits [B, Hkv, Lmax, hd]
        self.v_cache = v_cache
        self.table = rope_table(max_pos, self.cfg.head_dim, self.cfg.theta)
        # float64 GEMV from tile bytes: the numpy restatement, or the equal C one
        self.gemv = gemv or (lambda raw, kind, x, n_t, k_t: qo.gemv(raw, kind, x, n_t, k_t, acc=np.float64))

    def step(self, tokens, pos) -> np.ndarray:
        """One decode step for B sequences at positions pos[b]; returns fp32 logits [B, V]
        and appends this step's k, v to the caches."""
        c = self.cfg
        w = self.w
        tokens = np.asarray(tokens).ravel()
        pos = np.asarray(pos).ravel()
        b_n = tokens.size
        kt_h = c.hidden // 256
        kt_i = c.inter // 256
        kt_q = c.n_q * c.head_dim // 256
        h = embed_rows(w.lm_head, tokens, c.vocab, c.hidden).astype(np.float32)
        for layer in range(c.n_layers):
            xn = qo.bf16_round(rmsnorm(h, w.norm_in[layer], c.eps).astype(np.float32))
            q_raw = self.gemv(w.wq[layer], "q4", xn, c.n_q * c.head_dim // 32, kt_h)
            k_raw = self.gemv(w.wk[layer], "q4", xn, c.n_kv * c.head_dim // 32, kt_h)
            v_raw = self.gemv(w.wv[layer], "q4", xn, c.n_kv * c.head_dim // 32, kt_h)
            qr, kr, vr = qkv_rope_from_raw(q_raw.reshape(b_n, -1), k_raw.reshape(b_n, -1),
                                           v_raw.reshape(b_n, -1), pos, self.table, c.head_dim)
            qb = qo.bf16_round(qr.astype(np.float32))
            kb = qo.bf16_round(kr.astype(np.float32))
            vb = qo.bf16_round(vr.astype(np.float32))
            kc, vc = self.k_cache[layer], self.v_cache[layer]
            for b in range(b_n):
                kc[b, :, pos[b]] = kb[b]
                vc[b, :, pos[b]] = vb[b]
            lens = pos + 1
            att = gqa_attention(qo.bf16_to_f32(qb), qo.bf16_to_f32(kc), qo.bf16_to_f32(vc),
                                lens, c.scale)
            ab = qo.bf16_round(att.astype(np.float32).reshape(b_n, -1))
            o = self.gemv(w.wo[layer], "q4", ab, c.hidden // 32, kt_q)
            h = (h + o.reshape(b_n, -1)).astype(np.float32)   # fp32 residual add
            xn2 = qo.bf16_round(rmsnorm(h, w.norm_post[layer], c.eps).astype(np.float32))
            g_raw = self.gemv(w.wg[layer], "q4", xn2, c.inter // 32, kt_h)
            u_raw = self.gemv(w.wu[layer], "q4", xn2, c.inter // 32, kt_h)
            m = qo.bf16_round(swiglu_from_raw(g_raw, u_raw).astype(np.float32)).reshape(b_n, -1)
            dn = self.gemv(w.wd[layer], "q4", m, c.hidden // 32, kt_i)
            h = (h + dn.reshape(b_n, -1)).astype(np.float32)
        hf = qo.bf16_round(rmsnorm(h, w.norm_final, c.eps).astype(np.float32))
        return self.gemv(w.lm_head, "q8", hf, c.vocab // 32, kt_h).reshape(b_n, -1)
