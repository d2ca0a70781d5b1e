"""Token loop in the shape of the reference's chat.py (chat.py:25-95), on the GPU decoder.

The reference chats with Qwen3.5-0.8B through transformers' `generate` with its lm_head
swapped for the NPU one; model files, tokenizer and network are not available here, so
this loop drives the granite-3B-shaped decoder (llmnputest_amd.granite) directly from
prompt token ids: a synthetic context fills the KV cache, then MAX_NEW greedy tokens are
decoded on the device and the reference's report line is printed.

    python -m llmnputest_amd.chat [--layers 40] [--ctx 2048] [--new 128] [--batch 1]
    python -m llmnputest_amd.chat --q4nx model.q4nx ...     # a real granite q4nx file
"""

from __future__ import annotations

import argparse
import sys
import time

import numpy as np
import torch

MAX_NEW = 128   # chat.py:22


def main(argv: list[str]) -> int:
    from .granite import GraniteConfig, GraniteDecoder, GraniteWeights

    ap = argparse.ArgumentParser(prog="llmnputest_amd.chat")
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--ctx", type=int, default=2048, help="synthetic context length")
    ap.add_argument("--new", type=int, default=MAX_NEW)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--q4nx", default=None, help="load weights from a granite .q4nx file")
    ap.add_argument("prompt_ids", nargs="*", type=int)
    a = ap.parse_args(argv[1:])

    t0 = time.time()
    cfg = GraniteConfig(n_layers=a.layers)
    w = (GraniteWeights.from_q4nx(a.q4nx, cfg) if a.q4nx
         else GraniteWeights.synthetic(cfg, seed=a.seed))
    dec = GraniteDecoder(w, max_batch=a.batch, max_len=a.ctx + a.new)
    dec.seed_cache(a.ctx, seed=a.seed + 1)
    rng = np.random.default_rng(a.seed)
    prompt = a.prompt_ids or rng.integers(0, cfg.vocab, a.batch).tolist()
    first = (prompt + prompt * a.batch)[:a.batch]
    print(f"gpu      granite-3B shape, {cfg.n_layers} layers, lm_head q8 {cfg.vocab} x "
          f"{cfg.hidden}, batch {a.batch}, context {a.ctx}")
    dec.generate(first, [a.ctx] * a.batch, 2)          # capture the step graph
    print(f"ready    {time.time() - t0:.1f}s\n")

    torch.cuda.synchronize()
    t = time.time()
    toks, _ = dec.generate(first, [a.ctx] * a.batch, a.new)
    dt = time.time() - t
    for b in range(a.batch):
        print(" ".join(str(int(x)) for x in toks[b]))
    n = toks.shape[1] * a.batch
    print(f"\n[{n} tokens, {dt:.3f}s, {n / dt:.2f} tok/s; "
          f"{dt / toks.shape[1] * 1e3:.3f} ms per step on the gpu]\n")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
