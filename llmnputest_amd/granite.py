"""A granite-3B-shaped decode step on one MI355X, built from the q4nx HIP ops.

The reference validates every op of granite-4.2-3B on the NPU but strings none of them
into a forward pass (README.md:295-311); this module is that token loop. Per layer the
step issues five launches, grouped the way designs/granite_gemv/granite_layer.py:54-59
groups the projections by shared input:

    [RMSNorm, q, k, v, RoPE, KV append]   q4nx_qkv_rope (norm fused as the prologue)
    [GQA flash-decode attention]          q4nx_gqa_decode
    [o, residual add]                     q4nx_gemv_ex (residual epilogue, in place)
    [RMSNorm, gate, up, SwiGLU]           q4nx_gate_up_swiglu (norm fused)
    [down, residual add]                  q4nx_gemv_ex

At one sequence the attention launch only publishes its split records
(q4nx_gqa_decode_records) and the o-projection merges them in its prologue
(q4nx_gemv_attn_q4), which gives the same bits sooner. Then one lm_head launch (q8 or q4;
final RMSNorm fused as its prologue, one order-preserving (max, row) key per 16-row block in
its epilogue) and one bookkeeping launch that reduces the keys to the next token and
advances positions. A whole step is captured once in a HIP graph, and so are
GRAPH_STEPS steps back to back in a second graph (each graph launch leaves the GPU idle for
about 6-7 us, so generate() replays the longer graph and the one-step graph only for the
remainder, or for every step when it records logits); the greedy loop never leaves the
device. Every launch carries the decoder's own launch policy.

Conventions (the reference fixes none of them): fp32 residual stream, pre-norm
Llama/Granite order, final RMSNorm; the embedding of token t is row t of the stored
model.embed_tokens.weight when the weights have one, else row t of the dequantised (tied)
lm_head; KV cache bf16 [B][Hkv][L][64] per layer.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import numpy as np
import torch

from . import ops
from .ops import Policy
from .q4nx import Q4_TILE_BYTES, Q8_TILE_BYTES, Q4NX, TILE_BYTES, check_stored_shape, projection_shape

# greedy steps per replay of the multi-step decode graph
GRAPH_STEPS = 16


@dataclass(frozen=True)
class GraniteConfig:
    """granite-4.2-3B shapes (README.md:160-161; designs/granite_gemv/granite_gemv.py:6-9)."""
    hidden: int = 2560
    inter: int = 8192
    n_layers: int = 40
    n_q: int = 40
    n_kv: int = 8
    head_dim: int = 64
    vocab: int = 100352
    eps: float = 1e-5
    theta: float = 10000.0
    scale: float = 0.125        # head_dim ** -0.5 (designs/granite_gemv/granite_attention.h:28-34)

    @property
    def q_dim(self) -> int:
        return self.n_q * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv * self.head_dim

    def layer_bytes(self) -> int:
        """q4 tile bytes of one layer's seven projections."""
        h, i, q, kv = self.hidden, self.inter, self.q_dim, self.kv_dim
        elems = q * h + 2 * kv * h + h * q + 3 * h * i
        return elems // 2 + elems // 32 * 4     # 4 bits per weight + bf16 d, m per 32

    def lm_head_bytes(self, kind: str = "q8") -> int:
        return (self.vocab // 32) * (self.hidden // 256) * TILE_BYTES[kind]


@dataclass
class GraniteWeights:
    """Device tensors: raw q4nx tiles (uint8) per projection, bf16 norm weights, the
    lm_head's tiles (q8 or q4) and, when the model stores one, a bf16 embedding matrix."""
    cfg: GraniteConfig
    layers: list = field(default_factory=list)   # dicts: q k v o gate up down norm_in norm_post
    norm_final: torch.Tensor | None = None
    lm_head: torch.Tensor | None = None           # tiles of [vocab, hidden]
    lm_head_kind: str = "q8"
    embed: torch.Tensor | None = None             # bf16 [vocab, hidden]; None: tied lm_head

    def lm_head_bytes(self) -> int:
        return self.cfg.lm_head_bytes(self.lm_head_kind)

    # ------------------------------------------------------------ synthetic
    @staticmethod
    def synthetic(cfg: GraniteConfig, seed: int = 0, device="cuda", lm_head_kind: str = "q8",
                  stored_embed: bool = False) -> "GraniteWeights":
        """Random-init weights of the granite architecture in q4nx tiles, generated on the
        device from a seeded generator (Q4_1 with d = bf16(|N|*0.02), m = -8d; a q8 lm_head
        with s = bf16(|N|*0.01) or a q4 one; norm weights bf16(1 + 0.1 N); optionally a bf16
        N(0,1) embedding matrix)."""
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        w = GraniteWeights(cfg, lm_head_kind=lm_head_kind)
        h, i = cfg.hidden, cfg.inter
        for _ in range(cfg.n_layers):
            w.layers.append({
                "q": random_q4_tiles(cfg.q_dim, h, g, device),
                "k": random_q4_tiles(cfg.kv_dim, h, g, device),
                "v": random_q4_tiles(cfg.kv_dim, h, g, device),
                "o": random_q4_tiles(h, cfg.q_dim, g, device),
                "gate": random_q4_tiles(i, h, g, device),
                "up": random_q4_tiles(i, h, g, device),
                "down": random_q4_tiles(h, i, g, device),
                "norm_in": random_norm(h, g, device),
                "norm_post": random_norm(h, g, device),
            })
        w.norm_final = random_norm(h, g, device)
        w.lm_head = (random_q8_tiles(cfg.vocab, h, g, device) if lm_head_kind == "q8"
                     else random_q4_tiles(cfg.vocab, h, g, device))
        if stored_embed:
            w.embed = torch.randn((cfg.vocab, h), device=device, generator=g).to(torch.bfloat16)
        return w

    # ------------------------------------------------------------ real files
    @staticmethod
    def from_q4nx(path, cfg: GraniteConfig, device="cuda") -> "GraniteWeights":
        """Load a granite `.q4nx` file: raw tiles straight to the device, (N, K) from the
        config and checked against the stored shape (granite_gemv.py:90-102, 282-288).
        The projections are q4; the lm_head is q4 in granite's file
        (designs/granite_gemv/granite_gemv.h:4-7) and q8 in others, either is taken; the
        embedding is model.embed_tokens.weight when the file stores it (bf16, as
        tools/q4nx.py:182-184 reads plain tensors), else the tied lm_head's rows."""
        f = Q4NX(path)
        hf_cfg = {"hidden_size": cfg.hidden, "intermediate_size": cfg.inter,
                  "num_attention_heads": cfg.n_q, "num_key_value_heads": cfg.n_kv,
                  "head_dim": cfg.head_dim, "vocab_size": cfg.vocab}

        def tiles(name, want_kind=None):
            n, k = projection_shape(name, hf_cfg)
            check_stored_shape(f.header[name]["shape"], n, k)
            kind, b = f.tiles(name)
            if want_kind is not None and kind != want_kind:
                raise ValueError(f"{name}: stored as {kind}, this decoder expects {want_kind}")
            return kind, torch.from_numpy(np.array(b, copy=True).reshape(-1)).to(device)

        def norm(name):
            return torch.from_numpy(f.plain(name).astype(np.uint16).view(np.int16).copy()).to(device).view(torch.bfloat16)

        w = GraniteWeights(cfg)
        for li in range(cfg.n_layers):
            p = f"model.layers.{li}."
            w.layers.append({
                "q": tiles(p + "self_attn.q_proj.weight", "q4")[1],
                "k": tiles(p + "self_attn.k_proj.weight", "q4")[1],
                "v": tiles(p + "self_attn.v_proj.weight", "q4")[1],
                "o": tiles(p + "self_attn.o_proj.weight", "q4")[1],
                "gate": tiles(p + "mlp.gate_proj.weight", "q4")[1],
                "up": tiles(p + "mlp.up_proj.weight", "q4")[1],
                "down": tiles(p + "mlp.down_proj.weight", "q4")[1],
                "norm_in": norm(p + "input_layernorm.weight"),
                "norm_post": norm(p + "post_attention_layernorm.weight"),
            })
        w.norm_final = norm("model.norm.weight")
        w.lm_head_kind, w.lm_head = tiles("lm_head.weight")
        name = "model.embed_tokens.weight"
        if name in f:
            e = f.plain(name)
            if f.header[name]["dtype"] != "BF16" or tuple(e.shape) != (cfg.vocab, cfg.hidden):
                raise ValueError(f"{name}: expected BF16 [{cfg.vocab}, {cfg.hidden}], file has "
                                 f"{f.header[name]['dtype']} {list(e.shape)}")
            w.embed = torch.from_numpy(e.astype(np.uint16).view(np.int16).copy()).to(device).view(
                torch.bfloat16)
        return w


def random_q4_tiles(n: int, k: int, gen: torch.Generator, device) -> torch.Tensor:
    """q4 tiles [n/32 * k/256 * 5120] uint8: uniform nibbles, d = bf16(|N|*0.02), m = bf16(-8d)."""
    t = (n // 32) * (k // 256)
    w = torch.randint(0, 256, (t, Q4_TILE_BYTES), dtype=torch.uint8, device=device, generator=gen)
    d = (torch.randn((t, 256), device=device, generator=gen).abs() * 0.02).to(torch.bfloat16)
    m = (d.float() * -8.0).to(torch.bfloat16)
    w[:, 0:512] = d.view(torch.uint8).reshape(t, 512)
    w[:, 512:1024] = m.view(torch.uint8).reshape(t, 512)
    return w.reshape(-1)


def random_q8_tiles(n: int, k: int, gen: torch.Generator, device) -> torch.Tensor:
    """q8 tiles: int8 codes uniform in [-127, 127], s = bf16(|N|*0.01)."""
    t = (n // 32) * (k // 256)
    w = torch.empty((t, Q8_TILE_BYTES), dtype=torch.uint8, device=device)
    w[:, 512:] = torch.randint(-127, 128, (t, 8192), dtype=torch.int8, device=device,
                               generator=gen).view(torch.uint8)
    s = (torch.randn((t, 256), device=device, generator=gen).abs() * 0.01).to(torch.bfloat16)
    w[:, 0:512] = s.view(torch.uint8).reshape(t, 512)
    return w.reshape(-1)


def random_norm(n: int, gen: torch.Generator, device) -> torch.Tensor:
    return (1.0 + 0.1 * torch.randn(n, device=device, generator=gen)).to(torch.bfloat16)


class GraniteDecoder:
    """Decode state for up to `max_batch` sequences of up to `max_len` positions.

    `step()` runs one token for every sequence at its own position; `generate()` runs the
    greedy loop on the device from HIP graphs of GRAPH_STEPS steps and of one step."""

    def __init__(self, weights: GraniteWeights, max_batch: int = 1, max_len: int = 4096,
                 device="cuda", fused_attn_o: bool = True, attn_splits: int = 0,
                 policy: Policy | None = None):
        c = weights.cfg
        self.cfg, self.w = c, weights
        # the launch policy of every kernel this decoder issues (its own copy: other
        # decoders and callers in the process keep theirs)
        self.policy = Policy() if policy is None else policy.replace()
        # batch 1: attention only publishes its split records and the o-projection merges
        # them in its prologue (q4nx_gemv_attn_q4), saving attention's cross-workgroup merge
        self.fused_attn_o = fused_attn_o
        self.attn_splits = attn_splits   # 0: the library's choice for the path taken
        self.dev = torch.device(device)
        self.max_batch = max_batch
        self.max_len = (max_len + 63) // 64 * 64
        b, dev = max_batch, self.dev
        kv_shape = (b, c.n_kv, self.max_len, c.head_dim)
        self.k_cache = [torch.zeros(kv_shape, dtype=torch.bfloat16, device=dev) for _ in range(c.n_layers)]
        self.v_cache = [torch.zeros(kv_shape, dtype=torch.bfloat16, device=dev) for _ in range(c.n_layers)]
        self.rope = ops.rope_table(self.max_len, c.head_dim, c.theta, device=dev)
        self.h = torch.zeros((b, c.hidden), dtype=torch.float32, device=dev)
        # sums of h^2 per 16 entries, written by each producer of h for the next RMSNorm
        self.ssq = torch.zeros((b, c.hidden // 16), dtype=torch.float32, device=dev)
        self.q = torch.zeros((b, c.q_dim), dtype=torch.bfloat16, device=dev)
        self.attn = torch.zeros((b, c.n_q, c.head_dim), dtype=torch.bfloat16, device=dev)
        self.mlp = torch.zeros((b, c.inter), dtype=torch.bfloat16, device=dev)
        self.logits = torch.zeros((b, c.vocab), dtype=torch.float32, device=dev)
        self.tokens = torch.zeros(b, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(b, dtype=torch.int32, device=dev)
        self.lens = torch.ones(b, dtype=torch.int32, device=dev)
        self.keys = torch.zeros((b, c.vocab // 16), dtype=torch.int64, device=dev)  # argmax keys
        self.history = torch.zeros((self.max_len, b), dtype=torch.int32, device=dev)
        self.step_ctr = torch.zeros(1, dtype=torch.int32, device=dev)
        self.ws = ops.Workspace(ops.WS_COUNTER_BYTES + (64 << 20), device=dev)
        self.graph: torch.cuda.CUDAGraph | None = None         # one greedy step
        self.graph_steps: torch.cuda.CUDAGraph | None = None   # GRAPH_STEPS greedy steps
        self.graph_batch = 0
        self.calls = 0
        self.seconds = 0.0

    def fuses_attn_o(self, b: int, n_split: int) -> bool:
        """Whether a step of b sequences runs attention's merge inside the o-projection
        (q4nx_gemv_attn_q4: one sequence, at most 18 splits, the attention row of at most 40
        heads held by one workgroup)."""
        c = self.cfg
        return (self.fused_attn_o and b == 1 and 1 <= n_split <= 18
                and c.n_q % 4 == 0 and c.n_q <= 40)

    # ------------------------------------------------------------ one step, eager
    def _embed_table(self):
        """The embedding rows: a stored bf16 matrix, or the tied lm_head's tiles."""
        w = self.w
        return (w.embed, "bf16") if w.embed is not None else (w.lm_head, w.lm_head_kind)

    def _embed(self, b: int) -> None:
        table, kind = self._embed_table()
        ops.embed(table, kind, self.tokens[:b], self.cfg.vocab, self.cfg.hidden, out=self.h[:b],
                  ssq_out=self.ssq[:b])

    def _launch_step(self, b: int, embed: bool = True, trace: list | None = None) -> None:
        """Every kernel of one decode step for the first b sequences (no allocation); without
        `embed` the step starts from h as the previous step's advance left it. With `trace`
        (eager steps only) the same launches also write their bf16 narrowing points, which are
        appended per layer as host arrays (see `step`)."""
        c, w = self.cfg, self.w
        kt_h, kt_q, kt_i = c.hidden // 256, c.q_dim // 256, c.inter // 256
        h, q, attn, mlp = self.h[:b], self.q[:b], self.attn[:b], self.mlp[:b]
        ssq = self.ssq[:b]
        pol = self.policy
        n_split = self.attn_splits or ops.gqa_decode_records_splits(b, c.n_q, c.n_kv,
                                                                    self.max_len, policy=pol)
        fuse_o = self.fuses_attn_o(b, n_split)
        if embed:
            self._embed(b)
        tr = None
        if trace is not None:
            tr = {"raw": torch.empty((b, (c.n_q + 2 * c.n_kv) * c.head_dim), dtype=torch.float32,
                                     device=self.dev),
                  "xn": torch.empty((b, c.hidden), dtype=torch.bfloat16, device=self.dev),
                  "gu": torch.empty((b, 2 * c.inter), dtype=torch.float32, device=self.dev),
                  "xn2": torch.empty((b, c.hidden), dtype=torch.bfloat16, device=self.dev),
                  "attn": torch.empty((b, c.n_q, c.head_dim), dtype=torch.bfloat16,
                                      device=self.dev)}
            pos_host = self.pos[:b].cpu().numpy()
        for li, L in enumerate(w.layers):
            kc, vc = self.k_cache[li], self.v_cache[li]
            ops.qkv_rope(L["q"], L["k"], L["v"], c.n_q, c.n_kv, kt_h, h, self.pos[:b], self.rope,
                         kc, vc, q_out=q, norm_w=L["norm_in"], eps=c.eps, ws=self.ws,
                         ssq_in=ssq, policy=pol, raw_out=tr and tr["raw"], xn_out=tr and tr["xn"])
            if fuse_o:
                rec = ops.gqa_decode_records(q.view(b, c.n_q, c.head_dim), kc, vc, self.lens[:b],
                                             n_split, c.scale, max_len=self.max_len, ws=self.ws,
                                             policy=pol)
                ops.gemv_attn_q4(L["o"], c.hidden // 32, rec, residual=h, out=h, ssq_out=ssq)
                if tr is not None:   # what the o-projection's merge read: the same bits
                    ops.gqa_decode(q.view(b, c.n_q, c.head_dim), kc, vc, self.lens[:b], c.scale,
                                   max_len=self.max_len, n_split=n_split, out=tr["attn"],
                                   ws=self.ws, policy=pol)
            else:
                ops.gqa_decode(q.view(b, c.n_q, c.head_dim), kc, vc, self.lens[:b], c.scale,
                               max_len=self.max_len, n_split=self.attn_splits, out=attn,
                               ws=self.ws, policy=pol)
                ops.gemv_ex(L["o"], "q4", attn.view(b, c.q_dim), c.hidden // 32, kt_q,
                            residual=h, out=h, ssq_out=ssq, ws=self.ws, policy=pol)
                if tr is not None:
                    tr["attn"].copy_(attn)
            ops.gate_up_swiglu(L["gate"], L["up"], c.inter // 32, kt_h, h, h_out=mlp,
                               norm_w=L["norm_post"], eps=c.eps, ws=self.ws, ssq_in=ssq,
                               policy=pol, raw_out=tr and tr["gu"], xn_out=tr and tr["xn2"])
            if tr is not None:
                trace.append(self._trace_layer(tr, li, b, pos_host, mlp))
            ops.gemv_ex(L["down"], "q4", mlp, c.hidden // 32, kt_i, residual=h, out=h,
                        ssq_out=ssq, ws=self.ws, policy=pol)
        # final RMSNorm fused into the lm_head prologue, greedy argmax into its epilogue
        ops.gemv_ex(w.lm_head, w.lm_head_kind, h, c.vocab // 32, kt_h, norm_w=w.norm_final,
                    eps=c.eps, out=self.logits[:b], argmax_keys=self.keys[:b], ssq_in=ssq,
                    ws=self.ws, policy=pol)

    def _trace_layer(self, tr: dict, li: int, b: int, pos_host, mlp) -> dict:
        """Host copies of one layer's bf16 narrowing points (uint16 bits): the normalised
        inputs, q and k narrowed before the rotation (from the fp32 GEMV outputs), q after
        it, the k and v rows appended at each sequence's position, the attention output,
        gate and up narrowed, and the SwiGLU product."""
        c = self.cfg
        bits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        rnd = lambda t: bits(ops.round_bf16(t.contiguous()))
        qd, kd = c.n_q * c.head_dim, c.n_kv * c.head_dim
        raw = tr["raw"]
        kc, vc = bits(self.k_cache[li][:b]), bits(self.v_cache[li][:b])
        return {
            "xn": bits(tr["xn"]), "xn2": bits(tr["xn2"]),
            "q_pre": rnd(raw[:, :qd]).reshape(b, c.n_q, c.head_dim),
            "k_pre": rnd(raw[:, qd:qd + kd]).reshape(b, c.n_kv, c.head_dim),
            "q": bits(self.q[:b]).reshape(b, c.n_q, c.head_dim),
            "k": np.stack([kc[i, :, pos_host[i]] for i in range(b)]),
            "v": np.stack([vc[i, :, pos_host[i]] for i in range(b)]),
            "attn": bits(tr["attn"]),
            "g": rnd(tr["gu"][:, :c.inter]), "u": rnd(tr["gu"][:, c.inter:]),
            "m": bits(mlp),
        }

    def step(self, tokens, positions, trace: list | None = None) -> torch.Tensor:
        """One decode step, eager: tokens/positions for B sequences -> fp32 logits [B, V].
        With `trace` (a list), one dict per layer of the step's bf16 narrowing points is
        appended to it (uint16 bits, keys as DecodeOracle's forced points: "xn", "q_pre",
        "k_pre", "q", "k", "v", "attn", "xn2", "g", "u", "m"); the step's launches and results
        are those of an untraced step."""
        tokens = torch.as_tensor(tokens, dtype=torch.int32).reshape(-1)
        positions = torch.as_tensor(positions, dtype=torch.int32).reshape(-1)
        b = tokens.numel()
        if b > self.max_batch or positions.numel() != b:
            raise ValueError("batch exceeds max_batch or positions do not match tokens")
        if int(positions.max()) >= self.max_len or int(positions.min()) < 0:
            raise ValueError(f"positions must be in [0, {self.max_len})")
        self.tokens[:b].copy_(tokens)
        self.pos[:b].copy_(positions)
        self.lens[:b].copy_(positions + 1)
        self._launch_step(b, trace=trace)
        return self.logits[:b]

    # ------------------------------------------------------------ graph + greedy loop
    def _advance(self, b: int) -> None:
        """The next token from the argmax keys, positions and history advanced, and the
        token's embedding row into h for the next step: one launch."""
        table, kind = self._embed_table()
        ops.decode_advance_embed(self.keys[:b], self.cfg.vocab // 16, self.tokens[:b],
                                 self.pos[:b], self.lens[:b], self.step_ctr,
                                 self.history[:, :b] if b == self.max_batch else None,
                                 table, kind, self.cfg.vocab, self.cfg.hidden, self.h[:b],
                                 self.ssq[:b])

    def capture(self, b: int) -> None:
        """Capture one greedy step for b sequences: the step's kernels from h, then one launch
        that turns the argmax key into the next token, advances positions and history, and
        embeds the token into h for the next replay (the first replay's h comes from
        generate()). A second graph holds GRAPH_STEPS such steps back to back: the same
        launches in the same order, so replaying it once equals GRAPH_STEPS replays of the
        first."""
        snap = (self.tokens.clone(), self.pos.clone(), self.lens.clone(), self.step_ctr.clone())
        self._launch_step(b)                       # warm: sizes every workspace
        self._advance(b)
        torch.cuda.synchronize()
        graphs = []
        for steps in (1, GRAPH_STEPS):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(steps):
                    self._launch_step(b, embed=False)
                    self._advance(b)
            graphs.append(g)
        self.graph, self.graph_steps = graphs
        self.graph_batch = b
        for t, s0 in zip((self.tokens, self.pos, self.lens, self.step_ctr), snap):
            t.copy_(s0)

    def generate(self, first_tokens, start_pos, n_new: int, record_logits: bool = False):
        """Greedy decode of n_new tokens for B sequences from `first_tokens` at `start_pos`.
        Returns (tokens [B, n_new] int32 on the host, per-step logits list or None)."""
        first = torch.as_tensor(first_tokens, dtype=torch.int32).reshape(-1)
        start = torch.as_tensor(start_pos, dtype=torch.int32).reshape(-1)
        b = first.numel()
        if int(start.max()) + n_new > self.max_len:
            raise ValueError("max_len too small for this many new tokens")
        if int(start.min()) < 0 or start.numel() != b:
            raise ValueError("start positions must be >= 0, one per sequence")
        if b != self.max_batch:
            raise ValueError("generate() runs all max_batch sequences; size the decoder to them")
        if self.graph is None or self.graph_batch != b:
            self.pos[:b].copy_(start)
            self.lens[:b].copy_(start + 1)
            self.tokens[:b].copy_(first)
            self.capture(b)
        self.tokens[:b].copy_(first)
        self.pos[:b].copy_(start)
        self.lens[:b].copy_(start + 1)
        self.step_ctr.zero_()
        self._embed(b)                             # each replay embeds the token after it
        logs = [] if record_logits else None
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        if record_logits:
            for _ in range(n_new):
                self.graph.replay()
                logs.append(self.logits[:b].clone())
        else:
            for _ in range(n_new // GRAPH_STEPS):
                self.graph_steps.replay()
            for _ in range(n_new % GRAPH_STEPS):
                self.graph.replay()
        torch.cuda.synchronize()
        self.seconds += time.perf_counter() - t0
        self.calls += n_new
        return self.history[:n_new, :b].t().contiguous().cpu().numpy(), logs

    def seed_cache(self, ctx: int, seed: int = 0) -> None:
        """Fill positions [0, ctx) of every layer's K/V cache with bf16 N(0,1) (a synthetic
        context; no prefill runs through the model)."""
        g = torch.Generator(device=self.dev)
        g.manual_seed(seed)
        for kc, vc in zip(self.k_cache, self.v_cache):
            for t in (kc, vc):
                t.zero_()
                t[:, :, :ctx] = torch.randn(t[:, :, :ctx].shape, device=self.dev, generator=g).to(torch.bfloat16)
