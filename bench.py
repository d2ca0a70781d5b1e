#!/usr/bin/env python3
"""Benchmark of the q4nx decode hot path on one MI355X.

Headline (one JSON line): q4 W4A16 GEMV throughput at granite-3B projection shapes,
batch 1 -- gate/up 2560->8192 and down 8192->2560 -- in GB/s of algorithmic bytes
(packed weights + activation in + fp32 output), with the HBM roofline fraction of the GEMV
kernel and the reference's own CPU GEMV timed on this host beside it. When the decode
engine is available the same line also carries granite-3B-shaped decode tokens/s.

A step is one pass over ROT distinct layers' gate, up and down weights (ROT * 39.3 MB,
well above the 256 MB Infinity Cache, so the bytes come from HBM), captured once in a HIP
graph and replayed: 3 * ROT GEMV launches per step, inputs resident in HBM.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from llmnputest_amd import ops  # noqa: E402
from llmnputest_amd.granite import GraniteConfig, GraniteDecoder, GraniteWeights  # noqa: E402

HBM_PEAK_GBS = 8000.0
HIDDEN, INTER = 2560, 8192
Q4_TILE = 5120


def q4_bytes(n: int, k: int) -> int:
    return (n // 32) * (k // 256) * Q4_TILE


def algo_bytes(n: int, k: int) -> int:
    """Packed weights + bf16 activation in + fp32 output."""
    return q4_bytes(n, k) + 2 * k + 4 * n


def random_q4_tiles(n: int, k: int, gen: torch.Generator, dev) -> torch.Tensor:
    """Device-generated q4 tiles: uniform nibbles, d = bf16(|N|*0.02), m = bf16(-8d)."""
    t = (n // 32) * (k // 256)
    w = torch.randint(0, 256, (t, Q4_TILE), dtype=torch.uint8, device=dev, generator=gen)
    d = (torch.randn((t, 256), device=dev, generator=gen).abs() * 0.02).to(torch.bfloat16)
    m = (d.float() * -8.0).to(torch.bfloat16)
    w[:, 0:512] = d.view(torch.uint8).reshape(t, 512)
    w[:, 512:1024] = m.view(torch.uint8).reshape(t, 512)
    return w.reshape(-1)


def gemv_bench(steps: int, warmup: int, rot: int, dev) -> dict:
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    layers = [(random_q4_tiles(INTER, HIDDEN, gen, dev), random_q4_tiles(INTER, HIDDEN, gen, dev),
               random_q4_tiles(HIDDEN, INTER, gen, dev)) for _ in range(rot)]
    x = torch.randn(HIDDEN, device=dev, generator=gen).to(torch.bfloat16)
    h = torch.randn(INTER, device=dev, generator=gen).to(torch.bfloat16)
    y_gu = torch.empty(INTER, dtype=torch.float32, device=dev)
    y_d = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    ws = ops.Workspace(8 << 20, device=dev)

    sink = torch.zeros(64, dtype=torch.int32, device=dev)
    tiny = torch.zeros(16, dtype=torch.uint8, device=dev)

    def run(which: str, mode: str = "gemv"):
        """One step: gate and up (2560->8192) and/or down (8192->2560) of every rotated layer,
        as the GEMV, as the null kernel (same grid and loads, no arithmetic), or as a plain
        read of the same weight bytes; "empty" launches a 16-byte read in place of each."""
        for g, u, d in layers:
            for w_, x_, y_, n_, k_, part in ((g, x, y_gu, INTER, HIDDEN, "gate_up"),
                                             (u, x, y_gu, INTER, HIDDEN, "gate_up"),
                                             (d, h, y_d, HIDDEN, INTER, "down")):
                if which not in ("all", part):
                    continue
                if mode == "gemv":
                    ops.gemv(w_, "q4", x_, n_ // 32, k_ // 256, out=y_, ws=ws)
                elif mode == "null":
                    ops.gemv_q4_null(w_, x_, n_ // 32, k_ // 256, out=y_)
                elif mode == "read":
                    ops.stream_read(w_, sink)
                else:
                    ops.stream_read(tiny, sink)

    def timed(which: str, n_steps: int, mode: str = "gemv") -> float:
        run(which, mode)                        # eager warm-up (no allocation later)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            run(which, mode)
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n_steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3 / n_steps   # seconds per step

    b_gu, b_d = algo_bytes(INTER, HIDDEN), algo_bytes(HIDDEN, INTER)
    t_all = timed("all", steps)
    t_gu = timed("gate_up", steps)
    t_d = timed("down", steps)
    # the floors of the same launches: the null kernel per shape, a plain read of the same
    # 13,107,200-byte tensors, and a near-empty launch (one 16-byte read)
    f_gu = timed("gate_up", steps, "null") / (2 * rot)
    f_d = timed("down", steps, "null") / rot
    f_all = timed("all", steps, "null") / (3 * rot)
    r_all = timed("all", steps, "read") / (3 * rot)
    e_all = timed("all", steps, "empty") / (3 * rot)
    step_bytes = rot * (2 * b_gu + b_d)
    return {
        "t_step": t_all,
        "launches_per_step": 3 * rot,
        "step_bytes": step_bytes,
        "gbs": step_bytes / t_all / 1e9,
        "us_per_launch": t_all / (3 * rot) * 1e6,
        "gate_up_gbs": 2 * rot * b_gu / t_gu / 1e9,
        "gate_up_us": t_gu / (2 * rot) * 1e6,
        "down_gbs": rot * b_d / t_d / 1e9,
        "down_us": t_d / rot * 1e6,
        "bytes_gate_up": b_gu,
        "bytes_down": b_d,
        "null_gate_up_us": f_gu * 1e6,
        "null_down_us": f_d * 1e6,
        "null_us_per_launch": f_all * 1e6,
        "read_us_per_launch": r_all * 1e6,
        "empty_us_per_launch": e_all * 1e6,
    }


def copy_calibration(mib: int, reps: int, dev) -> int:
    """A plain device copy of `mib` MiB, `reps` times: the known-size kernel that scales the
    FETCH_SIZE / WRITE_SIZE counters (read mib MiB and write mib MiB per launch)."""
    n = mib << 20
    src = torch.ones(n // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_read": n, "bytes_written": n, "reps": reps}),
          flush=True)
    return 0


TRAFFIC_FILE = ROOT / "profiles" / "traffic_q4_gemv_granite_b1.json"


def measured_traffic() -> int | None:
    """HBM bytes per GEMV launch from the committed counter runs (FETCH_SIZE + WRITE_SIZE,
    scaled by the copy calibration), averaged over the bench's 2 gate/up : 1 down mix."""
    try:
        t = json.loads(TRAFFIC_FILE.read_text())
        return int(t["bytes_per_launch_mix"])
    except (OSError, KeyError, ValueError):
        return None


def _graph_time(fn, reps: int, warm: int = 2) -> float:
    """Seconds per call of fn (a sequence of launches) captured in one HIP graph."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warm):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / reps


def random_q8_tiles(n: int, k: int, gen: torch.Generator, dev) -> torch.Tensor:
    """Device-generated q8 tiles: int8 codes in [-127, 127], s = bf16(|N|*0.01)."""
    t = (n // 32) * (k // 256)
    w = torch.randint(-127, 128, (t, 8704), dtype=torch.int8, device=dev, generator=gen)
    s = (torch.randn((t, 256), device=dev, generator=gen).abs() * 0.01).to(torch.bfloat16)
    w = w.view(torch.uint8)
    w[:, 0:512] = s.view(torch.uint8).reshape(t, 512)
    return w.reshape(-1)


SECONDARY_GROUPS = ("lm_head", "mlp", "prefill", "rope", "attention", "copy")


def secondary_bench(dev, groups=SECONDARY_GROUPS) -> dict:
    """The other shapes of the hot path, each timed over a graph of launches with inputs
    resident in HBM (weights rotated past the 256 MB Infinity Cache where they would fit):
    the q8 lm_head GEMV (and its 512-row prefill block), the [gate,up,SwiGLU] + down MLP at
    batch 1 and 8, the prefill contraction over 2048 rows, RoPE, GQA decode attention over
    the context lengths and batches of the parity tests, and a plain copy. `groups` picks a
    subset (profiling runs)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(99)
    out = {}
    if "lm_head" in groups:
        # q8 lm_head 248320 x 1024, two copies (540 MB)
        n, k = 248320, 1024
        ws = [random_q8_tiles(n, k, gen, dev) for _ in range(2)]
        x = torch.randn(k, device=dev, generator=gen).to(torch.bfloat16)
        y = torch.empty(n, dtype=torch.float32, device=dev)
        t = _graph_time(lambda: [ops.gemv(ws[i % 2], "q8", x, n // 32, k // 256, out=y)
                                 for i in range(8)], 10) / 8   # alternating: each read cold
        b = ws[0].numel() + 2 * k + 4 * n
        out["lm_head_q8_248320x1024"] = {"us": round(t * 1e6, 2), "GB/s": round(b / t / 1e9, 1)}
        # the same lm_head over a 512-row prefill block (the rows the reference hands to torch)
        xp = torch.randn(512, k, device=dev, generator=gen).to(torch.bfloat16)
        yp = torch.empty(512, n, dtype=torch.float32, device=dev)
        wsg = ops.Workspace(1 << 20, device=dev)
        t = _graph_time(lambda: ops.gemm(ws[0], "q8", xp, n // 32, k // 256, out=yp, ws=wsg), 5)
        fl = 2.0 * 512 * n * k
        out["lm_head_q8_248320x1024_prefill_m512"] = {"us": round(t * 1e6, 1),
                                                      "TFLOP/s": round(fl / t / 1e12, 1)}
        del ws, xp, yp
    if "mlp" in groups or "prefill" in groups:
        # MLP: [gate, up, SwiGLU] then down, 8 layers rotated (315 MB), batch 1 and 8
        layers = [(random_q4_tiles(INTER, HIDDEN, gen, dev),
                   random_q4_tiles(INTER, HIDDEN, gen, dev),
                   random_q4_tiles(HIDDEN, INTER, gen, dev)) for _ in range(8)]
        wsp = ops.Workspace(8 << 20, device=dev)
    if "mlp" in groups:
        # batch 8 runs on the matrix cores by default; "_valu" pins the VALU GEMV
        for bb, path in ((1, ""), (8, ""), (8, "_valu")):
            xb = torch.randn(bb, HIDDEN, device=dev, generator=gen).to(torch.bfloat16)
            hb = torch.empty(bb, INTER, dtype=torch.bfloat16, device=dev)
            yb = torch.empty(bb, HIDDEN, dtype=torch.float32, device=dev)
            pol = ops.Policy(mfma_rows_q4=0) if path else ops.Policy()

            def mlp():
                for g_, u_, d_ in layers:
                    ops.gate_up_swiglu(g_, u_, INTER // 32, HIDDEN // 256, xb, h_out=hb, ws=wsp,
                                       policy=pol)
                    ops.gemv(d_, "q4", hb, HIDDEN // 32, INTER // 256, out=yb, ws=wsp, policy=pol)
            t = _graph_time(mlp, 10) / len(layers)
            byt = 3 * q4_bytes(INTER, HIDDEN) + bb * (2 * HIDDEN + 2 * INTER * 2 + 4 * HIDDEN)
            out[f"mlp_gate_up_swiglu_down_b{bb}{path}"] = {"us": round(t * 1e6, 2),
                                                           "GB/s": round(byt / t / 1e9, 1)}
    if "prefill" in groups:
        # the batched contraction over 2048 rows (gate 2560->8192, down 8192->2560)
        for name, (n_, k_) in (("gate_2560x8192", (INTER, HIDDEN)),
                               ("down_8192x2560", (HIDDEN, INTER))):
            m_ = 2048
            xp = torch.randn(m_, k_, device=dev, generator=gen).to(torch.bfloat16)
            yp = torch.empty(m_, n_, dtype=torch.float32, device=dev)
            wl = [L[0] if n_ == INTER else L[2] for L in layers[:4]]
            t = _graph_time(lambda: [ops.gemm(w_, "q4", xp, n_ // 32, k_ // 256, out=yp, ws=wsp)
                                     for w_ in wl], 5) / len(wl)
            fl = 2.0 * m_ * n_ * k_
            out[f"prefill_q4_{name}_m{m_}"] = {"us": round(t * 1e6, 1),
                                               "TFLOP/s": round(fl / t / 1e12, 1),
                                               "frac_of_bf16_mfma_peak": round(fl / t / 2.5e15, 4)}
    if "mlp" in groups or "prefill" in groups:
        del layers
    if "rope" in groups:
        # RoPE on q [B,40,64] and k [B,8,64]
        tab = ops.rope_table(4096, 64, 10000.0, device=dev)
        for bb in (1, 8):
            q = torch.randn(bb, 40, 64, device=dev, generator=gen).to(torch.bfloat16)
            kk = torch.randn(bb, 8, 64, device=dev, generator=gen).to(torch.bfloat16)
            pos = torch.randint(0, 4096, (bb,), dtype=torch.int32, device=dev, generator=gen)
            qo_, ko_ = torch.empty_like(q), torch.empty_like(kk)
            t = _graph_time(lambda: [(ops.rope(q, pos, tab, out=qo_),
                                      ops.rope(kk, pos, tab, out=ko_)) for _ in range(16)],
                            20) / 16
            out[f"rope_q40_k8_b{bb}"] = {"us": round(t * 1e6, 2)}
    if "attention" in groups:
        # GQA decode attention, 40 q / 8 kv heads, d 64
        wsa = ops.Workspace(64 << 20, device=dev)
        for bb in (1, 8):
            for L in (512, 4096, 32768):
                # enough cache copies to pass the 256 MB Infinity Cache (each launch reads its
                # K/V cold, as a decode step does), at least 8 launches per graph
                kv_bytes = bb * 8 * L * 64 * 2 * 2
                copies = max(2, min(600, -(-(600 << 20) // kv_bytes)))
                caches = [(torch.randn(bb, 8, L, 64, device=dev, generator=gen).to(torch.bfloat16),
                           torch.randn(bb, 8, L, 64, device=dev, generator=gen).to(torch.bfloat16))
                          for _ in range(copies)]
                q = torch.randn(bb, 40, 64, device=dev, generator=gen).to(torch.bfloat16)
                lens = torch.full((bb,), L, dtype=torch.int32, device=dev)
                o = torch.empty_like(q)
                nl = max(8, copies)
                t = _graph_time(lambda: [ops.gqa_decode(q, *caches[i % copies], lens, 0.125,
                                                        out=o, ws=wsa)
                                         for i in range(nl)], 10) / nl
                out[f"gqa_decode_b{bb}_L{L}"] = {"us": round(t * 1e6, 2),
                                                 "GB/s": round(kv_bytes / t / 1e9, 1)}
                del caches
    if "copy" in groups:
        # plain device copy of 1 GiB (reads 1 GiB, writes 1 GiB): the achievable streaming rate
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        t = _graph_time(lambda: dst.copy_(src), 5)
        out["copy_1GiB"] = {"us": round(t * 1e6, 1), "GB/s": round(2 * (1 << 30) / t / 1e9, 1)}
        del src, dst
        # the same copy at the size of one 2560->8192 q4 weight tensor (13,107,200 B read and
        # written), 48 buffers rotated past the Infinity Cache: what a single launch of this
        # size reaches, the per-launch reference for the GEMV
        nb = q4_bytes(INTER, HIDDEN)
        srcs = [torch.ones(nb // 4, dtype=torch.float32, device=dev) for _ in range(48)]
        dsts = [torch.empty_like(x) for x in srcs]
        t = _graph_time(lambda: [d.copy_(x) for d, x in zip(dsts, srcs)], 10) / len(srcs)
        out["copy_13MB"] = {"us": round(t * 1e6, 2), "GB/s": round(2 * nb / t / 1e9, 1)}
        del srcs, dsts
    return out


def decode_bytes_per_token(cfg: GraniteConfig, ctx: int, n_new: int, batch: int = 1) -> float:
    """Algorithmic HBM bytes of one decode step, averaged over the generated positions:
    every weight tile once, and per sequence the K/V cache up to the current position (read)
    plus one appended row, the embedding row and the logits; norm weights once."""
    mean_len = ctx + (n_new + 1) / 2.0
    kv = cfg.n_layers * cfg.n_kv * cfg.head_dim * 2 * 2 * (mean_len + 1)
    norms = (2 * cfg.n_layers + 1) * cfg.hidden * 2
    return (cfg.n_layers * cfg.layer_bytes() + cfg.lm_head_bytes() + norms
            + batch * (kv + cfg.hidden * 4 + cfg.vocab * 4))


def decode_bench(ctx: int, n_new: int, dev, cpu_tokens: int, batch: int = 1,
                 w: GraniteWeights | None = None) -> dict:
    """Greedy decode of n_new tokens for `batch` sequences at context ctx, timed with events
    around the device token loop. Bytes per step: the weights once plus every sequence's
    K/V cache."""
    cfg = GraniteConfig()
    if w is None:
        w = GraniteWeights.synthetic(cfg, seed=5, device=dev)
    dec = GraniteDecoder(w, max_batch=batch, max_len=ctx + n_new, device=dev)
    dec.seed_cache(ctx, seed=6)
    first = np.random.default_rng(7).integers(0, cfg.vocab, batch).tolist()
    dec.generate(first, [ctx] * batch, 4)               # capture + warm
    dec.seed_cache(ctx, seed=6)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    toks, _ = dec.generate(first, [ctx] * batch, n_new)
    e1.record()
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) / 1e3
    step_bytes = decode_bytes_per_token(cfg, ctx, n_new, batch)
    out = {"tok_s": batch * n_new / sec, "ms_per_token": sec / n_new * 1e3,
           "bytes_per_token": int(step_bytes), "gbs": step_bytes * n_new / sec / 1e9, "ctx": ctx,
           "new_tokens": n_new, "batch": batch, "weights": w}
    if cpu_tokens > 0 and batch == 1:
        out["cpu"] = decode_cpu_baseline(w, dec, first[0], ctx, toks[0], cpu_tokens)
    del dec
    return out


def decode_cpu_baseline(w, dec, first, ctx, gpu_tokens, n_tok: int) -> dict | None:
    """The CPU oracle's decode step (C float64 GEMVs from the same tiles + numpy for the
    rest) on this host, timed over a few teacher-forced tokens of the same workload."""
    try:
        from oracle import cpu_oracle
        from oracle import decode_oracle as do
    except Exception as e:  # pragma: no cover
        print(f"cpu decode baseline unavailable: {e}", file=sys.stderr)
        return None
    c = w.cfg
    bits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    hw = do.DecodeWeights(do.DecodeConfig(n_layers=c.n_layers))
    for L in w.layers:
        for key, dst in (("q", hw.wq), ("k", hw.wk), ("v", hw.wv), ("o", hw.wo),
                         ("gate", hw.wg), ("up", hw.wu), ("down", hw.wd)):
            dst.append(L[key].cpu().numpy().reshape(-1, 5120))
        hw.norm_in.append(bits(L["norm_in"]))
        hw.norm_post.append(bits(L["norm_post"]))
    hw.norm_final = bits(w.norm_final)
    hw.lm_head = w.lm_head.cpu().numpy().reshape(-1, 8704)
    dec.seed_cache(ctx, seed=6)
    oracle = do.DecodeOracle(hw, [bits(t) for t in dec.k_cache], [bits(t) for t in dec.v_cache],
                             dec.max_len, gemv=cpu_oracle.gemv)
    toks = [first] + [int(t) for t in gpu_tokens]
    s = time.perf_counter()
    for i in range(n_tok):
        oracle.step([toks[i]], [ctx + i])
    sec = (time.perf_counter() - s) / n_tok
    return {"value": round(1.0 / sec, 4), "unit": "tok/s", "cores": cpu_oracle.host_threads(),
            "kind": "port", "sample": f"{n_tok} decode steps of the same 40-layer workload, "
                                      f"float64 C GEMVs + numpy"}


def blas_threads() -> tuple[str, int | None]:
    """The BLAS numpy calls into and its thread count (threadpoolctl), if it can be read."""
    try:
        from threadpoolctl import threadpool_info
        for i in threadpool_info():
            if i.get("user_api") == "blas":
                return str(i.get("internal_api")), int(i.get("num_threads"))
    except Exception:   # pragma: no cover
        pass
    return "unknown", None


COLD_COPIES = 3   # q8 head copies rotated by the CPU legs: 3 x 270 MB, past a host's caches


def _cpu_time(fn, iters: int) -> float:
    """Seconds per call of fn after one untimed call."""
    fn()
    s = time.perf_counter()
    for _ in range(iters):
        fn()
    return (time.perf_counter() - s) / iters


def _q8_cold(w, x, n_t, k_t, threads, copies) -> float:
    """Seconds per q8 CPU GEMV, rotating `copies` distinct copies of the tiles so that no
    pass finds its bytes in a cache the previous pass filled."""
    from oracle import cpu_oracle
    ws = [w] + [w.copy() for _ in range(copies - 1)]
    cpu_oracle.q8_baseline_gemv(ws[-1], x, n_t, k_t, threads)
    s = time.perf_counter()
    for i in range(3 * copies):
        cpu_oracle.q8_baseline_gemv(ws[i % copies], x, n_t, k_t, threads)
    return (time.perf_counter() - s) / (3 * copies)


def decode_cpu_composed(ctx: int, threads: int, iters: int = 50) -> dict | None:
    """A like-for-like CPU decode step of the granite-3B workload, composed from the CPU
    paths timed on this host: every q4 projection shape (q and o 2560x2560, k and v
    512x2560, gate and up 8192x2560, down 2560x8192) on the reference's own CPU GEMV
    (designs/granite_gemv/cpu_baseline.cpp, built into oracle/_ref/, its own timing loop),
    GQA attention over a context-`ctx` bf16 cache per layer (oracle/cpu_attn.c, rotating 40
    distinct layer caches), and the q8 lm_head 100352x2560 (oracle/cpu_q8_baseline.c,
    copies rotated cold). Per token: 40 x (2 q/o + 2 k/v + 2 gate/up + down + attention) +
    head; the elementwise ops (RMSNorm, RoPE, SwiGLU: about 40 KB per layer) are left out,
    in the CPU's favour."""
    try:
        from oracle import cpu_oracle
        from llmnputest_amd import synth
    except Exception as e:  # pragma: no cover
        print(f"cpu decode baseline unavailable: {e}", file=sys.stderr)
        return None
    if not cpu_oracle.REF_BASELINE.exists():
        return None
    rng = np.random.default_rng(17)
    legs = {}
    for name, (n, k) in (("q_o_2560x2560", (HIDDEN, HIDDEN)), ("k_v_512x2560", (512, HIDDEN)),
                         ("gate_up_8192x2560", (INTER, HIDDEN)), ("down_2560x8192", (HIDDEN, INTER))):
        raw = synth.q4_tiles(rng, n, k).reshape(-1)
        r = cpu_oracle.run_ref_baseline(raw, n // 32, k // 256, threads, iters)
        legs[name] = r["gemv_ms"]
    gemv_ms = 2 * legs["q_o_2560x2560"] + 2 * legs["k_v_512x2560"] + \
        2 * legs["gate_up_8192x2560"] + legs["down_2560x8192"]
    cfg = GraniteConfig()
    caches = [(synth.random_bf16(rng, (cfg.n_kv, ctx, 64)), synth.random_bf16(rng, (cfg.n_kv, ctx, 64)))
              for _ in range(cfg.n_layers)]
    q = rng.standard_normal((cfg.n_q, 64)).astype(np.float32)
    cpu_oracle.gqa_decode(q, *caches[-1], ctx, 0.125, threads)
    s = time.perf_counter()
    for kc, vc in caches:
        cpu_oracle.gqa_decode(q, kc, vc, ctx, 0.125, threads)
    attn_ms = (time.perf_counter() - s) / len(caches) * 1e3
    del caches
    wh = synth.q8_tiles(rng, cfg.vocab, cfg.hidden).reshape(-1)
    xh = synth.random_bf16(rng, cfg.hidden)
    head_ms = _q8_cold(wh, xh, cfg.vocab // 32, cfg.hidden // 256, threads, COLD_COPIES) * 1e3
    tok_ms = cfg.n_layers * (gemv_ms + attn_ms) + head_ms
    return {"value": round(1e3 / tok_ms, 2), "unit": "tok/s", "cores": threads, "kind": "port",
            "ms_per_token": round(tok_ms, 3),
            "legs_ms": {**{k: round(v, 4) for k, v in legs.items()},
                        "attention_L%d" % ctx: round(attn_ms, 4),
                        "lm_head_q8_100352x2560_cold": round(head_ms, 3)},
            "sample": f"per token: 40 x (2 q/o + 2 k/v + 2 gate/up + down on the reference's "
                      f"cpu_baseline.cpp, {iters} iterations each, + GQA attention at context "
                      f"{ctx}, oracle/cpu_attn.c over 40 distinct caches) + q8 lm_head "
                      f"100352x2560 (oracle/cpu_q8_baseline.c, {COLD_COPIES} rotated copies); "
                      f"{threads} threads"}


def cpu_baseline(sample_iters: int) -> dict | None:
    """The reference's own CPU GEMV (designs/granite_gemv/cpu_baseline.cpp, built from its
    source into oracle/_ref/) on the same shapes, all host cores; else the C port."""
    try:
        from oracle import cpu_oracle
        from llmnputest_amd import synth
    except Exception as e:  # pragma: no cover
        print(f"cpu baseline unavailable: {e}", file=sys.stderr)
        return None
    threads = cpu_oracle.host_threads()
    rng = np.random.default_rng(7)
    gate = synth.q4_tiles(rng, INTER, HIDDEN).reshape(-1)
    down = synth.q4_tiles(rng, HIDDEN, INTER).reshape(-1)
    b_gu, b_d = algo_bytes(INTER, HIDDEN), algo_bytes(HIDDEN, INTER)
    t0 = time.time()
    if cpu_oracle.REF_BASELINE.exists():
        rg = cpu_oracle.run_ref_baseline(gate, INTER // 32, HIDDEN // 256, threads, sample_iters)
        rd = cpu_oracle.run_ref_baseline(down, HIDDEN // 32, INTER // 256, threads, sample_iters)
        t_layer = (2 * rg["gemv_ms"] + rd["gemv_ms"]) / 1e3
        stream = rg["stream_gbs"]
        kind = "reference"
        sample = (f"cpu_baseline.cpp (reference source, AVX2) on gate 8192x2560 and down "
                  f"2560x8192 q4 tiles, {sample_iters} iterations each; per layer = 2*gate + down")
    else:
        x = synth.random_bf16(rng, HIDDEN)
        xd = synth.random_bf16(rng, INTER)
        s = time.perf_counter()
        for _ in range(sample_iters):
            cpu_oracle.gemv(gate, "q4", x, INTER // 32, HIDDEN // 256, threads)
        tg = (time.perf_counter() - s) / sample_iters
        s = time.perf_counter()
        for _ in range(sample_iters):
            cpu_oracle.gemv(down, "q4", xd, HIDDEN // 32, INTER // 256, threads)
        td = (time.perf_counter() - s) / sample_iters
        t_layer = 2 * tg + td
        stream = None
        kind = "port"
        sample = f"oracle/cpu_oracle.c fp64 GEMV, {sample_iters} iterations per shape"
    out = {"value": round((2 * b_gu + b_d) / t_layer / 1e9, 2), "unit": "GB/s",
           "cores": threads, "kind": kind, "sample": sample}
    if stream is not None:   # the reference binary's STREAM read of the same gate tiles
        out["stream_read_GBs"] = stream
    # the q8 lm_head 248320 x 1024 shape: the reference has no CPU q8 GEMV, so its q4
    # baseline's method (AVX2 + FMA, one thread per core claiming tile-rows from an atomic
    # counter, the scales factored out of the inner sums) applied to the q8 tile
    # (oracle/cpu_q8_baseline.c); and beside it the numpy oracle (un-tile, dequantise to fp32,
    # BLAS matmul) on the same bytes, one call, with its BLAS thread count
    n8, k8 = 248320, 1024
    w8 = synth.q8_tiles(rng, n8, k8).reshape(-1)
    x8 = synth.random_bf16(rng, k8)
    b8 = w8.size + 2 * k8 + 4 * n8
    t8w = _cpu_time(lambda: cpu_oracle.q8_baseline_gemv(w8, x8, n8 // 32, k8 // 256, threads), 20)
    t8 = _q8_cold(w8, x8, n8 // 32, k8 // 256, threads, COLD_COPIES)
    out["lm_head_q8"] = {"value": round(b8 / t8 / 1e9, 2), "unit": "GB/s", "cores": threads,
                         "kind": "port",
                         "sample": f"oracle/cpu_q8_baseline.c (AVX2 + FMA, {threads} threads on "
                                   f"an atomic tile-row counter) on 248320x1024 q8 tiles, "
                                   f"{COLD_COPIES} copies (813 MB) rotated so each pass reads "
                                   f"its 270 MB cold, {3 * COLD_COPIES} passes",
                         "warm_same_buffer_GBs": round(b8 / t8w / 1e9, 2)}
    from oracle import q4nx_oracle as qo
    s = time.perf_counter()
    qo.gemv(w8, "q8", x8, n8 // 32, k8 // 256)
    tn = time.perf_counter() - s
    blas = blas_threads()
    out["lm_head_q8"]["numpy_oracle"] = {
        "value": round(b8 / tn / 1e9, 3), "unit": "GB/s", "blas": blas[0],
        "blas_threads": blas[1],
        "sample": "oracle/q4nx_oracle.gemv (un-tile, dequantise to fp32 in 256-tile-row chunks, "
                  "numpy matmul) on the same 248320x1024 q8 tiles, 1 call"}
    out["wall_s"] = round(time.time() - t0, 1)
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--rot", type=int, default=16, help="distinct layers rotated per step")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-iters", type=int, default=400)
    ap.add_argument("--ctx", type=int, default=2048, help="decode context length")
    ap.add_argument("--new-tokens", type=int, default=128)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--cpu-decode-tokens", type=int, default=2)
    ap.add_argument("--decode-batch", type=int, default=8,
                    help="also time decode with this many sequences per step (1: skip)")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the other shapes (lm_head, MLP, RoPE, attention, copy)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain copy of MIB MiB (counter calibration) and exit")
    ap.add_argument("--only", default=None, metavar="GROUPS",
                    help="profiling: only these comma-separated groups (" +
                         ",".join(SECONDARY_GROUPS + ("gemv", "decode", "decode_batched")) +
                         "; gemv: the headline GEMV steps and their floors; "
                         "decode: the batch-1 decode at --ctx / --new-tokens; "
                         "decode_batched: the same with --decode-batch sequences); prints "
                         "their JSON and exits")
    a = ap.parse_args()

    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the decode hot path runs on a single MI355X and has "
              "no multi-GPU path (every tile-row is independent, so q/k/v/gate/up would split "
              "by tile-row and o/down by K with one 10 KB all-reduce per layer).",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if a.calibrate_copy:
        return copy_calibration(a.calibrate_copy, 10, dev)
    if a.only:
        groups = tuple(g for g in a.only.split(",") if g)
        dec_groups = ("gemv", "decode", "decode_batched")
        bad = [g for g in groups if g not in SECONDARY_GROUPS + dec_groups]
        if bad:
            print(f"unknown groups {bad}; choose from {SECONDARY_GROUPS + dec_groups}",
                  file=sys.stderr)
            return 2
        out = {}
        if "gemv" in groups:
            out["gemv"] = {k: (round(v, 4) if isinstance(v, float) else v)
                           for k, v in gemv_bench(a.steps, a.warmup, a.rot, dev).items()}
        if "decode" in groups:
            d = decode_bench(a.ctx, a.new_tokens, dev, 0)
            d.pop("weights")
            out["decode"] = d
        if "decode_batched" in groups:
            d = decode_bench(a.ctx, a.new_tokens, dev, 0, batch=a.decode_batch)
            d.pop("weights")
            out["decode_batched"] = d
        sec = tuple(g for g in groups if g not in dec_groups)
        if sec:
            out["other_shapes"] = secondary_bench(dev, sec)
        print(json.dumps(out), flush=True)
        return 0

    r = gemv_bench(a.steps, a.warmup, a.rot, dev)
    cpu = None if a.no_cpu else cpu_baseline(a.cpu_iters)
    dec = dec8 = None
    if not a.no_decode:
        dec = decode_bench(a.ctx, a.new_tokens, dev, 0 if a.no_cpu else a.cpu_decode_tokens)
        if a.decode_batch > 1:   # the same weights, several sequences per step
            dec8 = decode_bench(a.ctx, a.new_tokens, dev, 0, batch=a.decode_batch,
                                w=dec["weights"])
        dec.pop("weights")
    sec = None if a.no_secondary else secondary_bench(dev)
    dec_cpu = None
    if dec is not None and not a.no_cpu:
        from oracle import cpu_oracle
        dec_cpu = decode_cpu_composed(a.ctx, cpu_oracle.host_threads())
        if dec_cpu is None:
            dec_cpu = dec.get("cpu")
    gbs = r["gbs"]
    line = {
        "metric": "q4 GEMV HBM GB/s (% of peak) + decode tok/s, granite-3B shape, batch 1",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(r["t_step"] * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded device RNG, q4nx tiles)",
        "config": {
            "workload": "q4 W4A16 GEMV batch 1, granite-3B projections gate/up 2560->8192 and "
                        "down 8192->2560",
            "layers_rotated": a.rot,
            "bytes_per_step": r["step_bytes"],
            "launches_per_step": r["launches_per_step"],
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
        },
        "per_shape": {
            "gate_up_2560x8192": {"GB/s": round(r["gate_up_gbs"], 1), "us": round(r["gate_up_us"], 3),
                                  "floor_us": round(r["null_gate_up_us"], 3),
                                  "frac_of_floor": round(r["null_gate_up_us"] / r["gate_up_us"], 4)},
            "down_8192x2560": {"GB/s": round(r["down_gbs"], 1), "us": round(r["down_us"], 3),
                               "floor_us": round(r["null_down_us"], 3),
                               "frac_of_floor": round(r["null_down_us"] / r["down_us"], 4)},
            "us_per_launch": round(r["us_per_launch"], 3),
        },
        # the same 48 launches per step as floors: the null kernel (the GEMV's grid and loads,
        # no arithmetic; the reference's --null design), a plain read of the same weight
        # tensors, and a 16-byte read (what a launch costs with no bytes to move)
        "floors": {
            "null_us_per_launch": round(r["null_us_per_launch"], 3),
            "null_GB/s": round(r["step_bytes"] / (3 * a.rot) / r["null_us_per_launch"] / 1e3, 1),
            "gemv_frac_of_null": round(r["null_us_per_launch"] / r["us_per_launch"], 4),
            "read_13MB_us_per_launch": round(r["read_us_per_launch"], 3),
            "read_GB/s": round(q4_bytes(INTER, HIDDEN) / r["read_us_per_launch"] / 1e3, 1),
            "empty_us_per_launch": round(r["empty_us_per_launch"], 3),
        },
        "cpu_baseline": cpu,
    }
    if dec is not None:
        line["decode"] = {
            "workload": f"granite-3B-shaped decode, 40 layers q4nx q4 + q8 lm_head 2560->100352, "
                        f"batch 1, context {dec['ctx']}, {dec['new_tokens']} greedy tokens",
            "tok_s": round(dec["tok_s"], 1),
            "ms_per_token": round(dec["ms_per_token"], 4),
            "bytes_per_token": dec["bytes_per_token"],
            "GB/s": round(dec["gbs"], 1),
            "roofline_frac": round(dec["gbs"] / HBM_PEAK_GBS, 4),
            "cpu_baseline": dec_cpu,
        }
        if dec_cpu is not None and dec.get("cpu") is not None:
            # the float64 oracle's own rate on the same workload, kept apart: it checks
            # results and is not a CPU decoder
            dec_cpu["float64_oracle"] = dec["cpu"]
    if dec8 is not None:
        line["decode_batched"] = {
            "workload": f"the same decode with {dec8['batch']} sequences per step (weights read "
                        f"once per step, each sequence its own K/V cache)",
            "tok_s": round(dec8["tok_s"], 1),
            "ms_per_step": round(dec8["ms_per_token"], 4),
            "bytes_per_step": dec8["bytes_per_token"],
            "GB/s": round(dec8["gbs"], 1),
        }
    if sec is not None:
        line["other_shapes"] = sec
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
