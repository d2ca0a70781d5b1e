"""The granite-shaped decode step on the GPU against the oracle, per step.

Full widths (hidden 2560, intermediate 8192, 40q/8kv heads, d=64, vocab 100352, q8
lm_head); reduced layer counts and contexts keep the float64 CPU oracle to seconds. The
GPU runs its own greedy loop from a HIP graph; the oracle replays the same tokens
(teacher-forced on the GPU's choices) and every step's logits are compared. bf16
narrowing inside the step makes rare 1-ulp flips unavoidable between two correct
implementations, so the per-step gate is cosine >= 0.9999 with max|Δ|/max|ref| < 5e-3, and
the GPU's greedy token must be the oracle's argmax unless the oracle's top two logits lie
within that tolerance.
"""

import numpy as np
import pytest
import torch

from llmnputest_amd import ops
from llmnputest_amd.granite import GraniteConfig, GraniteDecoder, GraniteWeights
from oracle import cpu_oracle
from oracle import decode_oracle as do
from oracle import q4nx_oracle as qo

pytestmark = pytest.mark.gpu

COS = 0.9999
REL = 5e-3


def host_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host_copy(w: GraniteWeights) -> do.DecodeWeights:
    c = w.cfg
    hw = do.DecodeWeights(do.DecodeConfig(hidden=c.hidden, inter=c.inter, n_layers=c.n_layers,
                                          n_q=c.n_q, n_kv=c.n_kv, head_dim=c.head_dim,
                                          vocab=c.vocab, eps=c.eps, theta=c.theta, scale=c.scale))
    for L in w.layers:
        for key, dst in (("q", hw.wq), ("k", hw.wk), ("v", hw.wv), ("o", hw.wo), ("gate", hw.wg),
                         ("up", hw.wu), ("down", hw.wd)):
            dst.append(L[key].cpu().numpy().reshape(-1, 5120))
        hw.norm_in.append(host_bits(L["norm_in"]))
        hw.norm_post.append(host_bits(L["norm_post"]))
    hw.norm_final = host_bits(w.norm_final)
    hw.lm_head = w.lm_head.cpu().numpy().reshape(-1, 8704)
    return hw


def check_step(got, ref, token):
    rel, cos = qo.metrics(got, ref)
    assert cos >= COS and rel < REL, (rel, cos)
    top = np.sort(ref)[-2:]
    if top[1] - top[0] > REL * np.abs(ref).max():
        assert token == int(np.argmax(ref)), (token, int(np.argmax(ref)))
    return rel, cos


@pytest.mark.parametrize("n_layers,batch,ctx,n_new,fused", [(2, 1, 256, 6, False),
                                                            (1, 3, 100, 3, False),
                                                            (2, 1, 200, 3, True),
                                                            (2, 1, 2100, 2, False)])
def test_decode_steps_vs_oracle(dev, kpath, n_layers, batch, ctx, n_new, fused):
    cfg = GraniteConfig(n_layers=n_layers)
    w = GraniteWeights.synthetic(cfg, seed=11, device=dev)
    dec = GraniteDecoder(w, max_batch=batch, max_len=ctx + n_new, device=dev, fused_tail=fused)
    dec.seed_cache(ctx, seed=12)
    kc = [host_bits(t) for t in dec.k_cache]
    vc = [host_bits(t) for t in dec.v_cache]
    rng = np.random.default_rng(13)
    first = rng.integers(0, cfg.vocab, batch).astype(np.int32)
    start = np.full(batch, ctx, np.int32) - np.arange(batch, dtype=np.int32) * 7   # ragged
    toks, logits = dec.generate(first, start, n_new, record_logits=True)
    oracle = do.DecodeOracle(host_copy(w), kc, vc, dec.max_len, gemv=cpu_oracle.gemv)
    prev = first
    for i in range(n_new):
        ref = oracle.step(prev, start + i)
        got = logits[i].cpu().numpy()
        for b in range(batch):
            check_step(got[b], ref[b], int(toks[b, i]))
        prev = toks[:, i]


def test_full_granite_step_vs_oracle(dev):
    """The full granite-3B-shaped decode (40 layers, q8 lm_head 2560->100352, batch 1, context
    2048, the default kernels and fusions) against the CPU oracle for two greedy tokens."""
    cfg = GraniteConfig()
    assert cfg.n_layers == 40
    w = GraniteWeights.synthetic(cfg, seed=91, device=dev)
    ctx, n_new = 2048, 2
    dec = GraniteDecoder(w, max_batch=1, max_len=ctx + n_new, device=dev)
    dec.seed_cache(ctx, seed=92)
    kc = [host_bits(t) for t in dec.k_cache]
    vc = [host_bits(t) for t in dec.v_cache]
    first = np.array([4242], np.int32)
    start = np.array([ctx], np.int32)
    toks, logits = dec.generate(first, start, n_new, record_logits=True)
    oracle = do.DecodeOracle(host_copy(w), kc, vc, dec.max_len, gemv=cpu_oracle.gemv)
    prev = first
    for i in range(n_new):
        ref = oracle.step(prev, start + i)
        check_step(logits[i].cpu().numpy()[0], ref[0], int(toks[0, i]))
        prev = toks[:, i]


@pytest.mark.parametrize("ctx", [300, 2100])
def test_fused_attn_o_equals_unfused(dev, apath, ctx):
    """Batch 1 with attention's merge in the o-projection prologue decodes the same tokens with
    bit-identical logits as attention merging on its own at the same split count."""
    cfg = GraniteConfig(n_layers=2)
    w = GraniteWeights.synthetic(cfg, seed=41, device=dev)
    n_split = ops.gqa_decode_records_splits(1, cfg.n_q, cfg.n_kv, ctx + 64)
    assert 1 <= n_split <= ops.gqa_decode_splits(1, cfg.n_q, cfg.n_kv, ctx + 64)
    out = []
    for fused in (True, False):   # the same split count on both paths
        dec = GraniteDecoder(w, max_batch=1, max_len=ctx + 64, device=dev, fused_attn_o=fused,
                             attn_splits=n_split)
        assert dec.fuses_attn_o(1, n_split) == fused
        dec.seed_cache(ctx, seed=42)
        out.append(dec.generate([77], [ctx], 3, record_logits=True))
    (t_f, l_f), (t_u, l_u) = out
    assert np.array_equal(t_f, t_u)
    for a, b in zip(l_f, l_u):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))


@pytest.mark.parametrize("fused", [False, True])
def test_graph_equals_eager(dev, kpath, fused):
    """A graph replay computes bit-identical logits to the eager step."""
    cfg = GraniteConfig(n_layers=2)
    w = GraniteWeights.synthetic(cfg, seed=21, device=dev)
    dec = GraniteDecoder(w, max_batch=1, max_len=320, device=dev, fused_tail=fused)
    dec.seed_cache(300, seed=22)
    snap_k = [t.clone() for t in dec.k_cache]
    snap_v = [t.clone() for t in dec.v_cache]
    toks, logits = dec.generate([123], [300], 2, record_logits=True)
    for t, s in zip(dec.k_cache + dec.v_cache, snap_k + snap_v):
        t.copy_(s)
    e0 = dec.step([123], [300]).clone()
    e1 = dec.step([int(toks[0, 0])], [301]).clone()
    assert torch.equal(e0, logits[0]) and torch.equal(e1, logits[1])
