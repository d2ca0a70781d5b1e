"""Token loop in the shape of the reference's chat.py (chat.py:25-95), on the GPU decoder.

The reference chats with Qwen3.5-0.8B through transformers' `generate` with its lm_head
swapped for the NPU one; model files, tokenizer and network are not available here, so
this loop drives the granite-3B-shaped decoder (llmnputest_amd.granite) directly from
prompt token ids: a synthetic context fills the KV cache, then MAX_NEW greedy tokens are
decoded on the device and the reference's report line is printed.

    python -m llmnputest_amd.chat [--layers 40] [--ctx 2048] [--new 128] [--batch 1]
    python -m llmnputest_amd.chat --q4nx model.q4nx ...     # a real granite q4nx file
    python -m llmnputest_amd.chat --hf-tiny                 # chat.py's own flow (below)

`--hf-tiny` runs chat.py's flow itself (chat.py:36-42, 80-94): a transformers causal LM whose
lm_head is swapped for the GPU one with `attach_lm_head` and a .q4nx file, greedy `generate`
with the rest of the model in torch on the CPU, and the report line with the head's share
of the wall time. Without model files the model is a random `Qwen3_5ForCausalLM` with
the reference model's head (hidden 1024, vocab 248320, tied embeddings) and a few layers,
and its lm_head is written as q8 tiles by `synth.quantize_q8`.
"""

from __future__ import annotations

import argparse
import sys
import time

import numpy as np
import torch

MAX_NEW = 128   # chat.py:22


def tiny_qwen35(seed: int, n_layers: int = 4):
    """A random-weight `Qwen3_5ForCausalLM` with the reference model's head: hidden 1024,
    vocab 248320, embeddings tied to the lm_head (reference/from_q4nx.py:140-171 builds the
    same class from the q4nx file; no model files are available offline). Layers follow
    Qwen3.5's pattern of three gated delta-net layers to one full-attention layer, ending on a
    full-attention layer."""
    import transformers

    types = ["linear_attention"] * n_layers
    for i in range(n_layers - 1, -1, -4):
        types[i] = "full_attention"
    cfg = transformers.Qwen3_5TextConfig(
        vocab_size=248320, hidden_size=1024, intermediate_size=3584, num_hidden_layers=n_layers,
        num_attention_heads=8, num_key_value_heads=2, head_dim=256, linear_num_key_heads=16,
        linear_num_value_heads=16, linear_key_head_dim=128, linear_value_head_dim=128,
        layer_types=types, tie_word_embeddings=True, max_position_embeddings=1024)
    cfg._attn_implementation = "eager"
    torch.manual_seed(seed)
    return transformers.Qwen3_5ForCausalLM(cfg).eval()


def hf_tiny(new_tokens: int, seed: int) -> int:
    import tempfile

    from . import npu, q4nx, synth

    t0 = time.time()
    model = tiny_qwen35(seed)
    cfg = model.config
    with tempfile.TemporaryDirectory() as d:
        path = f"{d}/model.q4nx"
        q4nx.write_q4nx(path, {"lm_head.weight": (
            "q8", synth.quantize_q8(model.lm_head.weight.detach().float().numpy()))})
        head = npu.attach_lm_head(model, q4nx.Q4NX(path))
    print(f"gpu      lm_head on the gpu, {head.n_rows} x {head.k}, q8 tiles "
          f"(random Qwen3.5, {cfg.num_hidden_layers} layers, in torch on the cpu)")
    print(f"ready    {time.time() - t0:.1f}s\n")
    ids = torch.from_numpy(np.random.default_rng(seed).integers(0, cfg.vocab_size, (1, 16)))
    head.design.seconds = head.design.calls = head.npu_calls = 0
    t = time.time()
    with torch.no_grad():
        out = model.generate(ids, max_new_tokens=new_tokens, do_sample=False, pad_token_id=0)
    dt = time.time() - t
    new = out[0, ids.shape[-1]:]
    print(" ".join(str(int(x)) for x in new))
    per = head.design.seconds / max(head.design.calls, 1) * 1e3
    print(f"\n[{len(new)} tokens, {dt:.1f}s, {len(new) / dt:.2f} tok/s; lm_head on gpu "
          f"{head.npu_calls}x at {per:.1f} ms, {100 * head.design.seconds / dt:.0f}% of wall]\n")
    return 0


def main(argv: list[str]) -> int:
    from .granite import GraniteConfig, GraniteDecoder, GraniteWeights

    ap = argparse.ArgumentParser(prog="llmnputest_amd.chat")
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--ctx", type=int, default=2048, help="synthetic context length")
    ap.add_argument("--new", type=int, default=MAX_NEW)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--q4nx", default=None, help="load weights from a granite .q4nx file")
    ap.add_argument("--hf-tiny", action="store_true",
                    help="transformers generate with the GPU lm_head (chat.py's flow)")
    ap.add_argument("prompt_ids", nargs="*", type=int)
    a = ap.parse_args(argv[1:])
    if a.hf_tiny:
        return hf_tiny(a.new, a.seed)

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
