"""CPU pins of the oracle's tile format, dequantisation and GEMV.

Each check is chosen so that a plausible mistake fails it: a swapped nibble parity or
row block permutes rows (brute force, one-hot, pack round trip); a wrong meta index or a
dropped minimum changes values (Q4_1 identity, brute force); a wrong rounding mode shows
on bf16 edge cases (torch's RNE casts); the reference's own compiled CPU GEMV agrees on
the same bytes (golden vectors in tests/golden/).
"""

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from llmnputest_amd import synth
from oracle import cpu_oracle
from oracle import q4nx_oracle as qo

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(0)
    edge = np.array([0.0, -0.0, 1.0, -1.0, 1.00390625, 1.0078125, 1.01171875, 3.0e38, -3.4e38,
                     np.inf, -np.inf, 1e-40, -1e-45, 65504.0, 2 ** -126, 2 ** -133],
                    np.float32)
    # values exactly halfway between bf16 neighbours, both parities
    half = (np.arange(1 << 10, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([edge, half, rng.standard_normal(10000).astype(np.float32) * 100])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(qo.bf16_round(x), want)
    assert np.isnan(qo.bf16_to_f32(qo.bf16_round(np.array([np.nan], np.float32))))[0]


@pytest.mark.parametrize("kind", ["q4", "q8"])
def test_dequant_vs_bruteforce(kind):
    rng = np.random.default_rng(1)
    t = (synth.q4_tiles(rng, 64, 256) if kind == "q4" else synth.q8_tiles(rng, 64, 256))
    flat = t.reshape(-1, t.shape[-1])
    vec = qo.dequant_matrix(flat, kind, 2, 1)
    brute = np.concatenate([qo.dequant_tile_bruteforce(flat[i], kind) for i in range(2)])
    assert np.array_equal(vec.view(np.uint32), brute.view(np.uint32))


def test_pack_roundtrip_known_codes():
    """Codes, scales and minima placed through the format text come back exactly."""
    rng = np.random.default_rng(2)
    codes = rng.integers(0, 16, (32, 256)).astype(np.uint8)
    d = synth.f32_to_bf16_bits(rng.uniform(0.001, 0.05, (32, 8)).astype(np.float32))
    m = synth.f32_to_bf16_bits(-rng.uniform(0.0, 0.5, (32, 8)).astype(np.float32))
    tile = synth.pack_q4_tile(codes, d, m)
    w = qo.dequant_matrix(tile.reshape(1, -1), "q4", 1, 1)
    df = qo.bf16_to_f32(d)[:, np.arange(256) // 32]
    mf = qo.bf16_to_f32(m)[:, np.arange(256) // 32]
    assert np.array_equal(w, (codes.astype(np.float32) * df + mf).astype(np.float32))
    # a single nonzero code lands on exactly one (row, k)
    for row, k in [(0, 0), (1, 0), (15, 255), (16, 3), (31, 200)]:
        c = np.zeros((32, 256), np.uint8)
        c[row, k] = 9
        one = np.ones((32, 8), np.uint16) * synth.f32_to_bf16_bits(np.float32(1.0))
        zero = np.zeros((32, 8), np.uint16)
        wm = qo.dequant_matrix(synth.pack_q4_tile(c, one, zero).reshape(1, -1), "q4", 1, 1)
        assert wm[row, k] == 9.0 and np.count_nonzero(wm) == 1


def test_q4_1_zero_point_identity():
    """Synthetic tiles use m = -8d, so every weight is (code - 8) * d exactly."""
    rng = np.random.default_rng(3)
    t = synth.q4_tiles(rng, 32, 512).reshape(-1, 5120)
    d = qo.bf16_to_f32(t[:, 0:512].copy().view(np.uint16))
    m = qo.bf16_to_f32(t[:, 512:1024].copy().view(np.uint16))
    assert (d > 0).all() and (m < 0).all() and np.array_equal(m, -8 * d)   # tools/q4nx.py:23-26
    codes = qo.unpack_nibbles(t[:, 1024:]).astype(np.float32)
    g = qo.meta_index()
    assert np.array_equal(qo.q4_tiles_f32(t), (codes - 8) * d[:, g])
    assert codes.min() == 0 and codes.max() == 15


@pytest.mark.parametrize("kind", ["q4", "q8"])
def test_gemv_onehot_and_ones(kind):
    rng = np.random.default_rng(4)
    n, k = 64, 512
    t = (synth.q4_tiles(rng, n, k) if kind == "q4" else synth.q8_tiles(rng, n, k))
    raw = t.reshape(-1, t.shape[-1])
    w = qo.dequant_matrix(raw, kind, n // 32, k // 256)
    for kk in (0, 31, 32, 257, 511):
        x = np.zeros(k, np.float32)
        x[kk] = 1
        y = qo.gemv(raw, kind, qo.bf16_round(x), n // 32, k // 256)
        assert np.array_equal(y, w[:, kk])
    ones = qo.gemv(raw, kind, qo.bf16_round(np.ones(k, np.float32)), n // 32, k // 256,
                   acc=np.float64)
    assert np.allclose(ones, w.astype(np.float64).sum(1), rtol=0, atol=1e-9)


def test_untile_row_and_column_order():
    """Row = tr*32 + rb*16 + r and column = kt*256 + k (tools/q4nx.py:146-149)."""
    flat = np.zeros((2 * 3, 8192), np.float32)
    for tr in range(2):
        for kt in range(3):
            for rb in range(2):
                for k in range(0, 256, 37):
                    for r in range(0, 16, 5):
                        flat[tr * 3 + kt, rb * 4096 + k * 16 + r] = tr * 1e6 + kt * 1e4 + rb * 1e3 + k + r / 100
    m = qo.untile(flat, 2, 3)
    for tr in range(2):
        for kt in range(3):
            for rb in range(2):
                for k in range(0, 256, 37):
                    for r in range(0, 16, 5):
                        assert m[tr * 32 + rb * 16 + r, kt * 256 + k] == np.float32(
                            tr * 1e6 + kt * 1e4 + rb * 1e3 + k + r / 100)


def test_reference_cpu_baseline_golden():
    """The reference's own CPU GEMV (built from designs/granite_gemv/cpu_baseline.cpp)
    printed these outputs for these seeded tiles; the oracle must reproduce them to the
    reference's fp32 accumulation error."""
    spec = json.loads((GOLDEN / "ref_cpu_baseline.json").read_text())
    for case in spec["cases"]:
        tiles = synth.q4_tiles(np.random.default_rng(case["seed"]), case["n"], case["k"])
        raw = np.ascontiguousarray(tiles).reshape(-1)
        assert hashlib.sha256(raw.tobytes()).hexdigest() == case["sha256"]
        k_t = case["k"] // 256
        rows = raw.reshape(case["n"] // 32, -1)[case["tile_row"]]
        x = cpu_oracle.ref_baseline_x(case["k"])
        w = qo.dequant_matrix(rows, "q4", 1, k_t).astype(np.float64)
        y = w @ x.astype(np.float64)
        got = np.array(case["y0_3"])
        # printed with 8 decimals; fp32 accumulation over K terms of magnitude ~1
        assert np.allclose(y[:4], got, rtol=0, atol=2e-6 * np.sqrt(case["k"] / 256)), (y[:4], got)


def test_oracle_small_fixture():
    spec = json.loads((GOLDEN / "oracle_small.json").read_text())
    rng = np.random.default_rng(7)
    q4 = synth.q4_tiles(rng, 64, 512).reshape(-1, 5120)
    q8 = synth.q8_tiles(rng, 64, 512).reshape(-1, 8704)
    x = synth.random_bf16(rng, (2, 512))
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    h = spec["sha256"]
    assert (sha(q4), sha(q8), sha(x)) == (h["q4"], h["q8"], h["x"])
    assert sha(qo.dequant_q4_bf16(q4)) == h["q4_bf16"] and sha(qo.dequant_q8_bf16(q8)) == h["q8_bf16"]
    assert np.array_equal(qo.gemv(q4, "q4", x, 2, 2, acc=np.float64), np.array(spec["q4_y"]))
    assert np.array_equal(qo.gemv(q8, "q8", x, 2, 2, acc=np.float64), np.array(spec["q8_y"]))


@pytest.mark.parametrize("kind", ["q4", "q8"])
def test_c_oracle_equals_numpy(kind):
    rng = np.random.default_rng(5)
    n, k = 256, 1024
    t = (synth.q4_tiles(rng, n, k) if kind == "q4" else synth.q8_tiles(rng, n, k))
    raw = t.reshape(-1, t.shape[-1])
    x = synth.random_bf16(rng, (3, k))
    a = cpu_oracle.gemv(raw, kind, x, n // 32, k // 256, threads=4)
    b = qo.gemv(raw, kind, x, n // 32, k // 256, acc=np.float64)
    assert np.allclose(a, b, rtol=1e-13, atol=1e-12)


@pytest.mark.skipif(not cpu_oracle.REF_BASELINE.exists(), reason="reference not built here")
def test_reference_binary_live():
    rng = np.random.default_rng(9)
    n, k = 64, 2560
    raw = synth.q4_tiles(rng, n, k).reshape(-1)
    r = cpu_oracle.run_ref_baseline(raw, n // 32, k // 256, threads=2, iters=1)
    w = qo.dequant_matrix(raw, "q4", n // 32, k // 256).astype(np.float64)
    y = w @ cpu_oracle.ref_baseline_x(k).astype(np.float64)
    assert np.allclose(y[:4], r["y0_3"], rtol=0, atol=1e-5)


def test_q8_cpu_baseline_vs_oracle():
    """The bench's AVX2 q8 CPU baseline (oracle/cpu_q8_baseline.c) against the float64 oracle
    on the same tile bytes: signed codes (a uint8 reading flips them), scales per (row, 32-K
    group) (a wrong group or row-block index moves rows), every thread count giving the same
    bits (each tile-row is summed by one thread in a fixed order)."""
    rng = np.random.default_rng(21)
    n, k = 40 * 32, 1024
    raw = synth.q8_tiles(rng, n, k).reshape(-1)
    x = synth.random_bf16(rng, (k,))
    ref = cpu_oracle.gemv(raw, "q8", x, n // 32, k // 256, threads=4)
    y1 = cpu_oracle.q8_baseline_gemv(raw, x, n // 32, k // 256, threads=1)
    y7 = cpu_oracle.q8_baseline_gemv(raw, x, n // 32, k // 256, threads=7)
    assert np.array_equal(y1.view(np.uint32), y7.view(np.uint32))
    rel, cos = qo.metrics(y1, ref)
    assert rel < 1e-5 and cos > 0.9999999, (rel, cos)
    # one-hot x: each output is exactly one dequantised column, summed in fp32 once per group
    xo = np.zeros(k, np.uint16)
    xo[300] = 0x3F80   # 1.0
    col = qo.dequant_matrix(raw, "q8", n // 32, k // 256)[:, 300]
    assert np.array_equal(cpu_oracle.q8_baseline_gemv(raw, xo, n // 32, k // 256, threads=3),
                          col)


def test_cpu_attention_baseline_vs_oracle():
    """The bench's AVX2 GQA decode attention (oracle/cpu_attn.c, the attention leg of the CPU
    decode baseline) against the float64 oracle attention: fp32 accuracy at one position,
    lengths that end inside and on a block of 8 positions, and a full context; the same
    result on 1 and 5 threads; a constant key row gives the mean of V (uniform softmax)."""
    from oracle import decode_oracle as do
    rng = np.random.default_rng(31)
    q = rng.standard_normal((40, 64)).astype(np.float32)
    k = synth.random_bf16(rng, (8, 300, 64))
    v = synth.random_bf16(rng, (8, 300, 64))
    kf, vf = qo.bf16_to_f32(k), qo.bf16_to_f32(v)
    for length in (1, 7, 8, 9, 257, 300):
        got = cpu_oracle.gqa_decode(q, k, v, length, 0.125, threads=5)
        ref = do.gqa_attention(q[None], kf[None], vf[None], [length], 0.125)[0]
        rel, cos = qo.metrics(got.ravel(), ref.ravel())
        assert rel < 1e-5 and cos > 0.9999999, (length, rel, cos)
        assert np.array_equal(got, cpu_oracle.gqa_decode(q, k, v, length, 0.125, threads=1))
    kc = np.broadcast_to(k[:, :1], k.shape).copy()      # every position the same key
    got = cpu_oracle.gqa_decode(q, kc, v, 200, 0.125, threads=3)
    assert np.allclose(got, np.repeat(vf[:, :200].mean(axis=1), 5, axis=0), rtol=1e-5, atol=1e-6)
