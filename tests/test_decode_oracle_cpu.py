"""Closed forms and special cases that pin the decode-op oracle (RMSNorm, RoPE, SwiGLU,
attention) independently of its own formulas, and a tiny decode step through it."""

import numpy as np
import pytest
from scipy.special import expit, softmax

from llmnputest_amd import synth
from oracle import cpu_oracle
from oracle import decode_oracle as do
from oracle import q4nx_oracle as qo


def test_rmsnorm_unit_rms_and_weight():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 2560)) * 7
    ones = synth.f32_to_bf16_bits(np.ones(2560, np.float32))
    y = do.rmsnorm(x, ones, 0.0)
    assert np.allclose(np.sqrt((y * y).mean(-1)), 1.0, atol=1e-12)
    w = synth.f32_to_bf16_bits(np.full(2560, 2.0, np.float32))
    assert np.allclose(do.rmsnorm(x, w, 0.0), 2 * y, atol=1e-12)


def test_rope_closed_forms():
    rng = np.random.default_rng(1)
    tab = do.rope_table(4096, 64, 10000.0)
    x = rng.standard_normal((40, 64))
    assert np.array_equal(do.rope(x, 0, tab), x)                      # position 0: identity
    y = do.rope(x, 1234, tab)
    pair = lambda a: a[:, :32] ** 2 + a[:, 32:] ** 2
    assert np.allclose(pair(y), pair(x), rtol=1e-6)                   # rotations keep norms
    # dimension i rotates by pos * theta^(-2i/64): i = 0 turns by exactly `pos` radians
    ang = np.arctan2(y[:, 32], y[:, 0]) - np.arctan2(x[:, 32], x[:, 0])
    assert np.allclose(np.cos(ang), np.cos(1234.0), atol=1e-6)
    assert np.abs(do.rope_interleaved(x, 1234, tab) - y).max() > 0.1


def test_swiglu_vs_scipy():
    rng = np.random.default_rng(2)
    g, u = rng.standard_normal(8192) * 4, rng.standard_normal(8192)
    assert np.allclose(do.swiglu(g, u), g * expit(g) * u, rtol=1e-12, atol=1e-15)
    assert do.swiglu(np.array([0.0]), np.array([5.0]))[0] == 0.0


def test_attention_special_cases():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((2, 40, 64))
    k = rng.standard_normal((2, 8, 50, 64))
    v = rng.standard_normal((2, 8, 50, 64))
    one = do.gqa_attention(q, k, v, lens=[1, 1])
    assert np.allclose(one, np.repeat(v[:, :, 0], 5, axis=1))         # L = 1: out = V[0]
    kc = np.repeat(k[:, :, :1], 50, axis=2)
    uni = do.gqa_attention(q, kc, v)
    assert np.allclose(uni, np.repeat(v.mean(axis=2), 5, axis=1))      # constant K: mean V
    ref = do.gqa_attention(q, k, v, lens=[50, 17], scale=0.125)
    for b, n in ((0, 50), (1, 17)):
        for h in (0, 7, 39):
            p = softmax(k[b, h // 5, :n] @ q[b, h] * 0.125)
            assert np.allclose(ref[b, h], p @ v[b, h // 5, :n], atol=1e-12)


def test_tiny_decode_step_numpy_equals_c_gemv():
    cfg = do.DecodeConfig(hidden=256, inter=512, n_layers=2, n_q=4, n_kv=2, head_dim=64,
                          vocab=96)
    rng = np.random.default_rng(4)
    w = do.DecodeWeights(cfg)
    h, i, q, kv = cfg.hidden, cfg.inter, cfg.n_q * 64, cfg.n_kv * 64
    for _ in range(cfg.n_layers):
        w.wq.append(synth.q4_tiles(rng, q, h).reshape(-1, 5120))
        w.wk.append(synth.q4_tiles(rng, kv, h).reshape(-1, 5120))
        w.wv.append(synth.q4_tiles(rng, kv, h).reshape(-1, 5120))
        w.wo.append(synth.q4_tiles(rng, h, q).reshape(-1, 5120))
        w.wg.append(synth.q4_tiles(rng, i, h).reshape(-1, 5120))
        w.wu.append(synth.q4_tiles(rng, i, h).reshape(-1, 5120))
        w.wd.append(synth.q4_tiles(rng, h, i).reshape(-1, 5120))
        w.norm_in.append(synth.f32_to_bf16_bits(1 + 0.1 * rng.standard_normal(h).astype(np.float32)))
        w.norm_post.append(synth.f32_to_bf16_bits(1 + 0.1 * rng.standard_normal(h).astype(np.float32)))
    w.norm_final = synth.f32_to_bf16_bits(np.ones(h, np.float32))
    w.lm_head = synth.q8_tiles(rng, cfg.vocab, h).reshape(-1, 8704)
    caches = lambda: [synth.random_bf16(np.random.default_rng(9), (1, cfg.n_kv, 40, 64)) for _ in range(2)]
    a = do.DecodeOracle(w, caches(), caches(), 40)
    b = do.DecodeOracle(w, caches(), caches(), 40, gemv=cpu_oracle.gemv)
    la = a.step([5], [30])
    lb = b.step([5], [30])
    assert la.shape == (1, cfg.vocab) and np.isfinite(la).all()
    rel, cos = qo.metrics(lb, la)
    assert rel < 1e-6 and cos > 0.999999
