"""Closed forms and special cases that pin the decode-op oracle (RMSNorm, RoPE, SwiGLU,
attention) independently of its own formulas, the decode step's composition against an
independent float64 decoder (transformers' Llama), and a tiny decode step through it.

Each pin is paired with the plausible mistake it must reject, planted in the oracle on the
CPU: the pin is shown to fail on it."""

import numpy as np
import pytest
from scipy.special import expit, softmax

from llmnputest_amd import synth
from oracle import cpu_oracle
from oracle import decode_oracle as do
from oracle import q4nx_oracle as qo
from tests.pins import check_rope_frequencies


def test_rmsnorm_unit_rms_and_weight():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 2560)) * 7
    ones = synth.f32_to_bf16_bits(np.ones(2560, np.float32))
    y = do.rmsnorm(x, ones, 0.0)
    assert np.allclose(np.sqrt((y * y).mean(-1)), 1.0, atol=1e-12)
    w = synth.f32_to_bf16_bits(np.full(2560, 2.0, np.float32))
    assert np.allclose(do.rmsnorm(x, w, 0.0), 2 * y, atol=1e-12)


def test_rmsnorm_eps_closed_form():
    """A constant row c gives y = c / sqrt(c^2 + eps) (granite_rmsnorm.py:113: eps inside the
    square root). At c = 1e-3, eps = 1e-5 that is 0.30151..., while eps added after the
    root would give 0.990...; eps = 0.1 at c = 1 pins it a second way."""
    ones = synth.f32_to_bf16_bits(np.ones(2560, np.float32))
    for c, eps in ((1e-3, 1e-5), (1.0, 0.1), (3.0, 1e-5)):
        y = do.rmsnorm(np.full((2, 2560), c), ones, eps)
        assert np.allclose(y, c / np.sqrt(c * c + eps), rtol=1e-12)
    assert np.isclose(do.rmsnorm(np.full((1, 8), 1e-3), ones[:8], 1e-5)[0, 0], 0.30151134457776363)


def test_rmsnorm_eps_pin_rejects_eps_outside_root(monkeypatch):
    def wrong(x, w_bf16, eps=1e-5):   # planted mistake: 1 / (sqrt(mean x^2) + eps)
        xf = np.asarray(x, np.float64)
        return xf / (np.sqrt((xf * xf).mean(-1, keepdims=True)) + eps) * qo.bf16_to_f32(w_bf16)
    monkeypatch.setattr(do, "rmsnorm", wrong)
    with pytest.raises(AssertionError):
        test_rmsnorm_eps_closed_form()


def test_rope_frequency_closed_forms():
    check_rope_frequencies(do.rope_table)


def test_rope_frequency_pin_rejects_wrong_exponent(monkeypatch):
    def wrong_inv(head_dim, theta):   # planted mistake: theta^(-i/hd)
        return 1.0 / (theta ** (np.arange(0, head_dim // 2, dtype=np.float64) / head_dim))
    monkeypatch.setattr(do, "rope_inv_freq", wrong_inv)
    with pytest.raises(AssertionError):
        check_rope_frequencies(do.rope_table)


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


def _tiny_weights(seed=4):
    cfg = do.DecodeConfig(hidden=256, inter=512, n_layers=2, n_q=4, n_kv=2, head_dim=64,
                          vocab=96)
    rng = np.random.default_rng(seed)
    w = do.DecodeWeights(cfg)
    h, i, q, kv = cfg.hidden, cfg.inter, cfg.n_q * 64, cfg.n_kv * 64
    for _ in range(cfg.n_layers):
        for dst, n, k in ((w.wq, q, h), (w.wk, kv, h), (w.wv, kv, h), (w.wo, h, q), (w.wg, i, h),
                          (w.wu, i, h), (w.wd, h, i)):
            dst.append(synth.q4_tiles(rng, n, k).reshape(-1, 5120))
        w.norm_in.append(synth.f32_to_bf16_bits(1 + 0.1 * rng.standard_normal(h).astype(np.float32)))
        w.norm_post.append(synth.f32_to_bf16_bits(1 + 0.1 * rng.standard_normal(h).astype(np.float32)))
    w.norm_final = synth.f32_to_bf16_bits(np.ones(h, np.float32))
    w.lm_head = synth.q8_tiles(rng, cfg.vocab, h).reshape(-1, 8704)
    return w


def test_forced_step_takes_over_one_ulp_flips_and_rejects_more():
    """The teacher-forced step (DecodeOracle.step(forced=...)): forced with its own bits it is
    the unforced step exactly; a one-ulp change of a value whose ulp lies inside the fp32 bar is
    taken over and counted as a flip; the largest value of a row moved by one ulp (far outside
    the bar), or a point fed another layer's values (a plausible wiring mistake of the caller),
    is refused."""
    w = _tiny_weights()
    caches = lambda: [synth.random_bf16(np.random.default_rng(9), (1, 2, 40, 64)) for _ in range(2)]
    own = do.DecodeOracle(w, caches(), caches(), 40)
    own.recorded = {}
    ref = own.step([5], [30])
    rec = own.recorded
    assert {k[0] for k in rec} == {"xn", "q_pre", "k_pre", "q", "k", "v", "attn", "xn2", "g",
                                   "u", "m"} and {k[1] for k in rec} == {0, 1}
    o = do.DecodeOracle(w, caches(), caches(), 40)
    assert np.array_equal(o.step([5], [30], forced=dict(rec)), ref) and sum(o.flips.values()) == 0
    vals = np.abs(qo.bf16_to_f32(rec[("m", 0)])).reshape(-1)
    small = int(np.argmin(np.where(vals > 0, vals, np.inf)))   # its ulp lies inside the bar
    big = int(np.argmax(vals))                                 # its ulp is far outside it
    m = rec[("m", 0)].copy()
    m.reshape(-1)[small] += 1
    o = do.DecodeOracle(w, caches(), caches(), 40)
    got = o.step([5], [30], forced={("m", 0): m})   # only this point: the flip flows on
    assert o.flips["m"] == 1   # (a value this small moves no fp32 residual: same logits)
    rel, cos = qo.metrics(got, ref)
    assert rel < 1e-3 and cos > 0.9999
    m2 = rec[("m", 0)].copy()
    m2.reshape(-1)[big] += 1
    with pytest.raises(AssertionError, match="not the bf16 rounding"):
        do.DecodeOracle(w, caches(), caches(), 40).step([5], [30], forced={("m", 0): m2})
    crossed = dict(rec)
    crossed[("xn", 1)] = rec[("xn", 0)]
    with pytest.raises(AssertionError, match="xn"):
        do.DecodeOracle(w, caches(), caches(), 40).step([5], [30], forced=crossed)


# ------------------------------------------------------------------ decode-step composition

def _granite_weights(n_layers, vocab, lm_kind, stored_embed, seed, hidden=2560, inter=8192,
                     n_q=40, n_kv=8):
    cfg = do.DecodeConfig(hidden=hidden, inter=inter, n_layers=n_layers, n_q=n_q, n_kv=n_kv,
                          head_dim=64, vocab=vocab)
    rng = np.random.default_rng(seed)
    w = do.DecodeWeights(cfg)
    q, kv = n_q * 64, n_kv * 64
    for _ in range(n_layers):
        w.wq.append(synth.q4_tiles(rng, q, hidden).reshape(-1, 5120))
        w.wk.append(synth.q4_tiles(rng, kv, hidden).reshape(-1, 5120))
        w.wv.append(synth.q4_tiles(rng, kv, hidden).reshape(-1, 5120))
        w.wo.append(synth.q4_tiles(rng, hidden, q).reshape(-1, 5120))
        w.wg.append(synth.q4_tiles(rng, inter, hidden).reshape(-1, 5120))
        w.wu.append(synth.q4_tiles(rng, inter, hidden).reshape(-1, 5120))
        w.wd.append(synth.q4_tiles(rng, hidden, inter).reshape(-1, 5120))
        w.norm_in.append(synth.f32_to_bf16_bits(1 + 0.2 * rng.standard_normal(hidden).astype(np.float32)))
        w.norm_post.append(synth.f32_to_bf16_bits(1 + 0.2 * rng.standard_normal(hidden).astype(np.float32)))
    w.norm_final = synth.f32_to_bf16_bits(1 + 0.2 * rng.standard_normal(hidden).astype(np.float32))
    w.lm_head_kind = lm_kind
    w.lm_head = (synth.q8_tiles(rng, vocab, hidden).reshape(-1, 8704) if lm_kind == "q8"
                 else synth.q4_tiles(rng, vocab, hidden).reshape(-1, 5120))
    if stored_embed:
        w.embed = synth.random_bf16(rng, (vocab, hidden))
    return w


def _llama_from(w):
    """A float64 transformers Llama decoder holding the oracle's dequantised weights
    (pre-norm blocks, rotate-half RoPE with theta 10^4, GQA, SwiGLU MLP, final norm)."""
    torch = pytest.importorskip("torch")
    tr = pytest.importorskip("transformers")
    c = w.cfg
    tied = w.embed is None
    conf = tr.LlamaConfig(hidden_size=c.hidden, intermediate_size=c.inter,
                          num_hidden_layers=c.n_layers, num_attention_heads=c.n_q,
                          num_key_value_heads=c.n_kv, head_dim=c.head_dim, vocab_size=c.vocab,
                          rms_norm_eps=c.eps, rope_theta=c.theta, tie_word_embeddings=tied,
                          max_position_embeddings=64, attention_bias=False, mlp_bias=False)
    torch.manual_seed(0)
    m = tr.LlamaForCausalLM(conf).to(torch.float64).eval()
    t64 = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    kt_h, kt_i, kt_q = c.hidden // 256, c.inter // 256, c.n_q * 64 // 256
    mat = lambda raw, n, kt: t64(_deq(raw, "q4", n // 32, kt))
    lm = t64(_deq(w.lm_head, w.lm_head_kind, c.vocab // 32, kt_h))
    with torch.no_grad():
        m.lm_head.weight.copy_(lm)
        m.model.embed_tokens.weight.copy_(lm if tied else t64(qo.bf16_to_f32(w.embed)))
        m.model.norm.weight.copy_(t64(qo.bf16_to_f32(w.norm_final)))
        for i, L in enumerate(m.model.layers):
            L.self_attn.q_proj.weight.copy_(mat(w.wq[i], c.n_q * 64, kt_h))
            L.self_attn.k_proj.weight.copy_(mat(w.wk[i], c.n_kv * 64, kt_h))
            L.self_attn.v_proj.weight.copy_(mat(w.wv[i], c.n_kv * 64, kt_h))
            L.self_attn.o_proj.weight.copy_(mat(w.wo[i], c.hidden, kt_q))
            L.mlp.gate_proj.weight.copy_(mat(w.wg[i], c.inter, kt_h))
            L.mlp.up_proj.weight.copy_(mat(w.wu[i], c.inter, kt_h))
            L.mlp.down_proj.weight.copy_(mat(w.wd[i], c.hidden, kt_i))
            L.input_layernorm.weight.copy_(t64(qo.bf16_to_f32(w.norm_in[i])))
            L.post_attention_layernorm.weight.copy_(t64(qo.bf16_to_f32(w.norm_post[i])))
        # the rotary frequencies in float64 (transformers builds them in float32)
        rot = m.model.rotary_emb
        inv = t64(do.rope_inv_freq(c.head_dim, c.theta))
        rot.inv_freq = inv
        if hasattr(rot, "original_inv_freq"):
            rot.original_inv_freq = inv
    return m


_MATS: dict = {}   # dequantised float64 matrices shared by the oracles of this module


def _deq(raw, kind, n_t, k_t):
    """The oracle's own dequantised matrix, cached under the key DecodeOracle uses."""
    key = (id(raw), kind)
    if key not in _MATS:
        _MATS[key] = np.asarray(qo.dequant_matrix(raw, kind, n_t, k_t), np.float64)
    return _MATS[key]


def _oracle_logits(w, tokens, narrow=False):
    c = w.cfg
    caches = lambda: [np.zeros((1, c.n_kv, 16, 64), np.uint16) for _ in range(c.n_layers)]
    o = do.DecodeOracle(w, caches(), caches(), 16, narrow=narrow, mats=_MATS,
                        gemv=cpu_oracle.gemv if narrow else None)
    return np.concatenate([o.step([t], [p]) for p, t in enumerate(tokens)])


def _llama_logits(m, tokens):
    import torch
    with torch.no_grad():
        return m(input_ids=torch.tensor([tokens])).logits[0].numpy()


def _assert_step_matches(got, ref, tol=1e-5):
    worst = 0.0
    for p in range(ref.shape[0]):
        rel, cos = qo.metrics(got[p], ref[p])
        worst = max(worst, rel)
        assert rel < tol and cos > 1 - tol * tol, (p, rel, cos)
    print(f"decode-step composition: worst max-rel {worst:.2e} over {ref.shape[0]} positions")


TOKENS = [17, 3, 250, 99, 3, 1, 511, 42]


@pytest.fixture(scope="module")
def granite2_q8():
    w = _granite_weights(2, 512, "q8", False, seed=11)
    return w, _llama_logits(_llama_from(w), TOKENS)


def test_decode_step_composition_vs_float64_llama(granite2_q8):
    """The oracle's decode step without bf16 narrowing equals an independent float64
    transformers Llama decoder on the same dequantised weights at every position of an
    8-token sequence from position 0 (2 granite-width layers, tied q8 lm_head). Llama
    computes its RMSNorm and RoPE angles in float32, hence 1e-5 and not 1e-12."""
    w, ref = granite2_q8
    _assert_step_matches(_oracle_logits(w, TOKENS), ref)
    # the narrowed oracle (the GPU's parity target) stays within bf16 distance of it
    got = _oracle_logits(w, TOKENS, narrow=True)
    for p in range(ref.shape[0]):
        rel, cos = qo.metrics(got[p], ref[p])
        assert rel < 5e-2 and cos > 0.999, (p, rel, cos)


@pytest.mark.parametrize("mistake", ["swapped_norms", "no_final_norm", "interleaved_rope",
                                     "no_attn_residual", "wrong_gqa_map"])
def test_decode_step_composition_pin_rejects(granite2_q8, mistake, monkeypatch):
    w, ref = granite2_q8
    w2 = do.DecodeWeights(w.cfg, **{k: getattr(w, k) for k in
                                    ("wq", "wk", "wv", "wo", "wg", "wu", "wd", "norm_in",
                                     "norm_post", "norm_final", "lm_head", "lm_head_kind",
                                     "embed")})
    if mistake == "swapped_norms":
        w2.norm_in, w2.norm_post = w.norm_post, w.norm_in
    elif mistake == "no_final_norm":
        calls = {"n": 0}
        real = do.rmsnorm
        def rms(x, wb, eps=1e-5):
            calls["n"] += 1
            if calls["n"] % (2 * w.cfg.n_layers + 1) == 0:
                return np.asarray(x, np.float64) * qo.bf16_to_f32(wb)
            return real(x, wb, eps)
        monkeypatch.setattr(do, "rmsnorm", rms)
    elif mistake == "interleaved_rope":
        monkeypatch.setattr(do, "rope", do.rope_interleaved)
    elif mistake == "no_attn_residual":
        real_mv = do.DecodeOracle._mv
        def mv(self, raw, kind, xv, n_t, k_t):
            y = real_mv(self, raw, kind, xv, n_t, k_t)
            if any(raw is r for r in w2.wo):   # o-projection: replace h instead of adding
                return y - self._h_now
            return y
        real_res = do.DecodeOracle._res
        def res(self, a):
            self._h_now = np.asarray(a, np.float64)
            return real_res(self, a)
        monkeypatch.setattr(do.DecodeOracle, "_mv", mv)
        monkeypatch.setattr(do.DecodeOracle, "_res", res)
    elif mistake == "wrong_gqa_map":
        real_att = do.gqa_attention
        def att(q, k, v, lens=None, scale=0.125):   # q head h -> kv head h % Hkv
            hkv = np.asarray(k).shape[1]
            perm = [h % hkv * (q.shape[1] // hkv) + h // hkv for h in range(q.shape[1])]
            return real_att(np.asarray(q)[:, perm], k, v, lens, scale)[:, np.argsort(perm)]
        monkeypatch.setattr(do, "gqa_attention", att)
    got = _oracle_logits(w2, TOKENS)
    with pytest.raises(AssertionError):
        _assert_step_matches(got, ref)
    print(mistake, "max-rel", max(qo.metrics(got[p], ref[p])[0] for p in range(len(TOKENS))))


def test_decode_step_q4_lm_head_stored_embedding_vs_float64_llama():
    """The real granite file's conventions: a q4 lm_head (granite_gemv.h:4-7) and a stored
    embedding matrix (untied), 1 granite-width layer, 5 tokens."""
    w = _granite_weights(1, 256, "q4", True, seed=12)
    toks = TOKENS[:5]
    _assert_step_matches(_oracle_logits(w, [t % 256 for t in toks]),
                         _llama_logits(_llama_from(w), [t % 256 for t in toks]))
