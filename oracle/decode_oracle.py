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
    pre-norm Llama/Granite order, final RMSNorm, a q8 or q4 lm_head; the embedding of
    token t is row t of a stored embedding matrix when the model has one, else row t of
    the dequantised (tied) lm_head.

`DecodeOracle.step(..., forced=...)` runs the step teacher-forced at its bf16 narrowing
points: where the caller supplies another implementation's bf16 bits for a point (the GPU's
normalised inputs, q/k before and after the rotation, the appended v, the attention output,
gate/up and the SwiGLU product), the oracle checks that each is the bf16 rounding of a value
within the fp32 bar (FORCE_TOL of the row's largest magnitude) of its own value there, counts
the values whose bits differ from its own rounding (flips), and continues from those bits.
Two correct implementations then differ only by floating-point arithmetic error between
narrowing points, with no flip carried into the next layer.

`DecodeOracle(narrow=False)` runs the same step with every bf16 narrowing point removed
(float64 throughout); that mode is what the composition is pinned with: it must equal a
float64 transformers Llama decoder built from the same dequantised weights
(tests/test_decode_oracle_cpu.py).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import q4nx_oracle as qo


def f64(a):
    return np.asarray(a, dtype=np.float64)


# A forced narrowing point accepts the bf16 rounding of any value within this fraction of the
# row's largest magnitude of the oracle's value: the fp32 bar every op of the step meets
# (GEMV, RMSNorm, RoPE, SwiGLU, attention). Near zero that spans several bf16 ulps.
FORCE_TOL = 1e-5


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
    """Raw tile bytes per layer (uint8 [n_t*k_t, tile_bytes]) and bf16 norm weights.
    lm_head: q8 or q4 tiles [vocab/32 * hidden/256, tile bytes] (lm_head_kind);
    embed: optional float32 or bf16-bits [vocab, hidden] embedding (None: tied lm_head)."""
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
    lm_head: np.ndarray | None = None
    lm_head_kind: str = "q8"
    embed: np.ndarray | None = None


def embed_rows(lm_head_raw: np.ndarray, tokens, vocab: int, hidden: int,
               kind: str = "q8") -> np.ndarray:
    """Tied embedding: row t of the dequantised lm_head (q8 or q4 tiles), float32
    [len(tokens), hidden]."""
    k_t = hidden // 256
    tb = qo.Q8_TILE_BYTES if kind == "q8" else qo.Q4_TILE_BYTES
    tiles = np.asarray(lm_head_raw, np.uint8).reshape(vocab // 32, k_t, tb)
    out = []
    for t in np.asarray(tokens).ravel():
        w = qo.dequant_matrix(tiles[t // 32].reshape(k_t, -1), kind, 1, k_t)
        out.append(w[t % 32])
    return np.stack(out).astype(np.float32)


def embedding(w: "DecodeWeights", tokens) -> np.ndarray:
    """Embedding rows of `tokens`: the stored matrix (bf16 bits or float) when present,
    else the tied lm_head's dequantised rows."""
    c = w.cfg
    if w.embed is None:
        return embed_rows(w.lm_head, tokens, c.vocab, c.hidden, w.lm_head_kind)
    e = np.asarray(w.embed)
    rows = e[np.asarray(tokens).ravel()]
    return qo.bf16_to_f32(rows) if e.dtype == np.uint16 else rows.astype(np.float32)


class DecodeOracle:
    """Numpy decode step in the conventions of the module docstring. Float64 / float32
    reference with bf16 narrowing at the same points as the GPU path (narrow=True), or
    with no narrowing at all (narrow=False: float64 everywhere, used to pin the
    composition against an independent decoder); slow, meant for reduced layer counts."""

    def __init__(self, w: DecodeWeights, k_cache: list, v_cache: list, max_pos: int,
                 gemv=None, narrow: bool = True, mats: dict | None = None):
        self.w = w
        self.cfg = w.cfg
        self.narrow = narrow
        if narrow:
            self.k_cache = k_cache      # per layer: bf16 bits [B, Hkv, Lmax, hd]
            self.v_cache = v_cache
        else:                           # per layer: float64 values [B, Hkv, Lmax, hd]
            val = lambda c: f64(qo.bf16_to_f32(c)) if np.asarray(c).dtype == np.uint16 else f64(c)
            self.k_cache = [val(c) for c in k_cache]
            self.v_cache = [val(c) for c in v_cache]
        self.table = rope_table(max_pos, self.cfg.head_dim, self.cfg.theta)
        # float64 GEMV from tile bytes: the numpy restatement, or the equal C one
        self.gemv = gemv or (lambda raw, kind, x, n_t, k_t: qo.gemv(raw, kind, x, n_t, k_t, acc=np.float64))
        self._mats = {} if mats is None else mats   # float64 matrices (narrow=False), shareable
        self._forced = None     # {(point, layer): bf16 bits} during a forced step
        self.flips: dict = {}   # one-ulp flips met at forced points, by point
        self.recorded: dict | None = None   # set to {} to keep each point's own bf16 bits

    # ---- the narrowing points and the GEMV on values
    def _nb(self, a, name: str, layer: int) -> np.ndarray:
        """Narrowing point `name` of `layer`: the value rounded to bf16, or, when the step is
        forced at this point, the given bf16 bits after checking that each is what
        round-to-nearest-even gives for some value within FORCE_TOL * max|row| of the
        oracle's own (the fp32 bar of the op that produced it; a row is one sequence's
        values at the point). Values whose bits differ from the oracle's own rounding are
        counted in self.flips."""
        v = self._bf(a)
        af = np.asarray(a, np.float64)
        if self.recorded is not None:   # the bits this step narrows to, for a later forcing
            self.recorded[(name, layer)] = qo.bf16_round(af.astype(np.float32))
        f = None if self._forced is None else self._forced.get((name, layer))
        if f is None:
            return v
        rows = af.reshape(af.shape[0], -1)
        got = np.asarray(f, np.uint16).reshape(-1)
        if rows.size != got.size:
            raise ValueError(f"forced {name}[{layer}]: {got.size} values, the step has {rows.size}")
        tol = (FORCE_TOL * np.abs(rows).max(axis=1, keepdims=True)) * np.ones_like(rows)
        ordered = lambda b: np.where(b & 0x8000, -(b & 0x7FFF).astype(np.int64),
                                     (b & 0x7FFF).astype(np.int64))
        lo = ordered(qo.bf16_round((rows - tol).astype(np.float32)).reshape(-1))
        hi = ordered(qo.bf16_round((rows + tol).astype(np.float32)).reshape(-1))
        g = ordered(got)
        bad = (g < lo) | (g > hi)
        if bad.any():
            i = int(np.flatnonzero(bad)[0])
            raise AssertionError(f"forced {name}[{layer}] at {i}: {got[i]:#06x} is not the bf16 "
                                 f"rounding of a value within {FORCE_TOL:g} * max|row| of "
                                 f"{rows.reshape(-1)[i]!r}")
        own = qo.bf16_round(rows.astype(np.float32)).reshape(-1)
        self.flips[name] = self.flips.get(name, 0) + int((own != got).sum())
        return f64(qo.bf16_to_f32(got)).reshape(np.shape(a))

    def _bf(self, a) -> np.ndarray:
        """A bf16 narrowing point: the value rounded to bf16 (narrow) or kept (float64)."""
        a = np.asarray(a)
        if self.narrow:
            return f64(qo.bf16_round_f32(a.astype(np.float32)))
        return f64(a)

    def _res(self, a) -> np.ndarray:
        """The residual stream's storage type: float32 (narrow) or float64."""
        return np.asarray(a, np.float32) if self.narrow else f64(a)

    def _mv(self, raw, kind: str, xv, n_t: int, k_t: int) -> np.ndarray:
        """y = W x for x given as values (bf16-exact values when narrowing)."""
        if self.narrow:
            return f64(self.gemv(raw, kind, qo.bf16_round(np.asarray(xv, np.float32)), n_t, k_t))
        key = (id(raw), kind)
        m = self._mats.get(key)
        if m is None:
            m = self._mats[key] = f64(qo.dequant_matrix(raw, kind, n_t, k_t))
        return f64(xv) @ m.T

    def step(self, tokens, pos, forced: dict | None = None) -> np.ndarray:
        """One decode step for B sequences at positions pos[b]; returns the float64 logits
        [B, V] and appends this step's k, v to the caches. `forced` maps (point, layer) to
        bf16 bits for a teacher-forced step (see the module docstring); points: "xn", "q_pre",
        "k_pre", "q", "k", "v", "attn", "xn2", "g", "u", "m" (shapes as the step's values,
        [B, ...] in the step's order)."""
        if forced is not None and not self.narrow:
            raise ValueError("a forced step needs the narrowing oracle")
        self._forced = forced
        try:
            return self._step(tokens, pos)
        finally:
            self._forced = None

    def _step(self, tokens, pos) -> np.ndarray:
        c = self.cfg
        w = self.w
        tokens = np.asarray(tokens).ravel()
        pos = np.asarray(pos).ravel()
        b_n = tokens.size
        hd = c.head_dim
        kt_h = c.hidden // 256
        kt_i = c.inter // 256
        kt_q = c.n_q * hd // 256
        h = self._res(embedding(w, tokens))
        for layer in range(c.n_layers):
            xn = self._nb(rmsnorm(h, w.norm_in[layer], c.eps).astype(np.float32)
                          if self.narrow else rmsnorm(h, w.norm_in[layer], c.eps), "xn", layer)
            q_raw = self._mv(w.wq[layer], "q4", xn, c.n_q * hd // 32, kt_h).reshape(b_n, -1, hd)
            k_raw = self._mv(w.wk[layer], "q4", xn, c.n_kv * hd // 32, kt_h).reshape(b_n, -1, hd)
            v_raw = self._mv(w.wv[layer], "q4", xn, c.n_kv * hd // 32, kt_h).reshape(b_n, -1, hd)
            # q and k narrowed before the rotation, the rotated values narrowed again
            # (designs/granite_gemv/granite_qkv_rope.h:37-69); v only narrowed
            q_pre, k_pre = self._nb(q_raw, "q_pre", layer), self._nb(k_raw, "k_pre", layer)
            qr = np.stack([rope(q_pre[b], pos[b], self.table) for b in range(b_n)])
            kr = np.stack([rope(k_pre[b], pos[b], self.table) for b in range(b_n)])
            qv, kv = self._nb(qr, "q", layer), self._nb(kr, "k", layer)
            vv = self._nb(v_raw, "v", layer)
            kc, vc = self.k_cache[layer], self.v_cache[layer]
            for b in range(b_n):
                if self.narrow:
                    kc[b, :, pos[b]] = qo.bf16_round(kv[b].astype(np.float32))
                    vc[b, :, pos[b]] = qo.bf16_round(vv[b].astype(np.float32))
                else:
                    kc[b, :, pos[b]] = kv[b]
                    vc[b, :, pos[b]] = vv[b]
            lens = pos + 1
            kval = qo.bf16_to_f32(kc) if self.narrow else kc
            vval = qo.bf16_to_f32(vc) if self.narrow else vc
            att = gqa_attention(qv, kval, vval, lens, c.scale)
            ab = self._nb(att.astype(np.float32) if self.narrow else att, "attn",
                          layer).reshape(b_n, -1)
            o = self._mv(w.wo[layer], "q4", ab, c.hidden // 32, kt_q)
            h = self._res(h + o.reshape(b_n, -1))          # residual add (fp32 when narrowing)
            xn2 = self._nb(rmsnorm(h, w.norm_post[layer], c.eps).astype(np.float32)
                           if self.narrow else rmsnorm(h, w.norm_post[layer], c.eps), "xn2", layer)
            g_raw = self._mv(w.wg[layer], "q4", xn2, c.inter // 32, kt_h)
            u_raw = self._mv(w.wu[layer], "q4", xn2, c.inter // 32, kt_h)
            sw = swiglu(self._nb(g_raw, "g", layer), self._nb(u_raw, "u", layer))
            m = self._nb(sw.astype(np.float32) if self.narrow else sw, "m", layer).reshape(b_n, -1)
            dn = self._mv(w.wd[layer], "q4", m, c.hidden // 32, kt_i)
            h = self._res(h + dn.reshape(b_n, -1))
        hf = self._bf(rmsnorm(h, w.norm_final, c.eps).astype(np.float32)
                      if self.narrow else rmsnorm(h, w.norm_final, c.eps))
        return self._mv(w.lm_head, w.lm_head_kind, hf, c.vocab // 32, kt_h).reshape(b_n, -1)
