"""GPU parity of dequantisation and the q4/q8 GEMV against the oracle.

Bars: dequant bit-exact; GEMV max|Δ|/max|ref| < 1e-5 against the float64 oracle with
cosine > 0.9999999 (the reference's own GEMV gate, designs/granite_gemv/granite_gemv.py:335);
one-hot activations reproduce a dequantised column exactly (README.md:188-190).
"""

import numpy as np
import pytest
import torch

from llmnputest_amd import ops, synth
from oracle import q4nx_oracle as qo

pytestmark = pytest.mark.gpu

REL = 1e-5
COS = 0.9999999


def _tiles(kind, n, k, seed):
    rng = np.random.default_rng(seed)
    t = synth.q4_tiles(rng, n, k) if kind == "q4" else synth.q8_tiles(rng, n, k)
    return t.reshape(-1, t.shape[-1]), rng


def _dev_u8(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).reshape(-1)).to(dev)


def _dev_bf16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).to(dev).view(torch.bfloat16)


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("kind", ["q4", "q8"])
@pytest.mark.parametrize("untile", [False, True])
def test_dequant_bitexact(dev, kind, untile):
    n, k = 96, 768
    raw, _ = _tiles(kind, n, k, 1)
    w = _dev_u8(raw, dev)
    n_t, k_t = n // 32, k // 256
    got16 = _bits(ops.dequant(w, kind, n_t, k_t, torch.bfloat16, untile))
    got32 = ops.dequant(w, kind, n_t, k_t, torch.float32, untile).cpu().numpy()
    f32 = qo.q4_tiles_f32(raw) if kind == "q4" else qo.q8_tiles_f32(raw)
    if untile:
        f32 = qo.untile(f32, n_t, k_t)
    assert np.array_equal(got32.view(np.uint32), f32.view(np.uint32))
    assert np.array_equal(got16, qo.bf16_round(f32))


@pytest.mark.parametrize("n,k", [(8192, 2560), (2560, 8192)])
def test_dequant_bitexact_full_granite(dev, n, k):
    """Config 2's weights dequantised in full: the gate/up 2560->8192 and down 8192->2560
    tensors (2560 q4 tiles each), fp32 bits and bf16 bits against the oracle's numpy dequant,
    tiled and un-tiled."""
    raw, _ = _tiles("q4", n, k, 8)
    w = _dev_u8(raw, dev)
    n_t, k_t = n // 32, k // 256
    f32 = qo.q4_tiles_f32(raw)
    for untile in (False, True):
        want = qo.untile(f32, n_t, k_t) if untile else f32
        got32 = ops.dequant(w, "q4", n_t, k_t, torch.float32, untile).cpu().numpy()
        assert np.array_equal(got32.view(np.uint32), want.view(np.uint32)), untile
        got16 = _bits(ops.dequant(w, "q4", n_t, k_t, torch.bfloat16, untile))
        assert np.array_equal(got16, qo.bf16_round(want)), untile


@pytest.mark.parametrize("kind", ["q4", "q8"])
def test_onehot_exact(dev, kpath, kind):
    n, k = 64, 1024
    raw, _ = _tiles(kind, n, k, 2)
    w = _dev_u8(raw, dev)
    wm = qo.dequant_matrix(raw, kind, n // 32, k // 256)
    for kk in (0, 1, 31, 32, 255, 256, 511, 777, 1023):
        x = np.zeros(k, np.float32)
        x[kk] = 1.0
        y = ops.gemv(w, kind, _dev_bf16(qo.bf16_round(x), dev), n // 32, k // 256).cpu().numpy()
        assert np.array_equal(y.view(np.uint32), wm[:, kk].view(np.uint32)), kk


@pytest.mark.parametrize("kind,n,k", [
    ("q4", 8192, 2560),   # gate/up
    ("q4", 2560, 8192),   # down
    ("q4", 2560, 2560),   # q/o
    ("q4", 512, 2560),    # k/v
    ("q8", 4096, 1024),
    ("q8", 2048, 2560),
])
def test_gemv_parity(dev, kpath, kind, n, k):
    raw, rng = _tiles(kind, n, k, 3)
    x = synth.random_bf16(rng, k)
    y = ops.gemv(_dev_u8(raw, dev), kind, _dev_bf16(x, dev), n // 32, k // 256).cpu().numpy()
    ref = qo.gemv(raw, kind, x, n // 32, k // 256, acc=np.float64)
    rel, cos = qo.metrics(y, ref)
    assert rel < REL and cos > COS, (rel, cos)


@pytest.mark.parametrize("n,k", [(8192, 2560), (2560, 8192), (2560, 2560), (512, 2560)])
def test_rowblock_q4_precision(dev, valu, n, k):
    """The one-row q4 GEMV at the granite projection shapes stays at fp32 accuracy: max|y -
    y_float64| below 2.5e-7 of max|y| over four seeds (measured 1.06-1.26e-7). Both nibbles
    enter v_dot2_f32_f16 in bits 4-7 of their fp16 operand; with the low nibble left in bits
    0-3 (a plausible saving of one instruction) the same shapes measured 3.7-6.3e-7, since the
    instruction keeps fewer bits of subnormals with leading zeros."""
    for seed in range(4):
        rng = np.random.default_rng(100 + seed)
        raw, _ = _tiles("q4", n, k, 100 + seed)
        x = synth.random_bf16(rng, k)
        y = ops.gemv(_dev_u8(raw, dev), "q4", _dev_bf16(x, dev), n // 32, k // 256).cpu().numpy()
        rel, cos = qo.metrics(y, qo.gemv(raw, "q4", x, n // 32, k // 256, acc=np.float64))
        assert rel < 2.5e-7 and cos > COS, (seed, rel, cos)


def test_gemv_q8_lm_head_full(dev, kpath):
    """Config: y[248320] = W[248320, 1024] @ x, q8 tiles."""
    n, k = 248320, 1024
    raw, rng = _tiles("q8", n, k, 4)
    x = synth.random_bf16(rng, k)
    y = ops.gemv(_dev_u8(raw, dev), "q8", _dev_bf16(x, dev), n // 32, k // 256).cpu().numpy()
    ref = qo.gemv(raw, "q8", x, n // 32, k // 256, acc=np.float64, chunk=1024)
    rel, cos = qo.metrics(y, ref)
    assert rel < REL and cos > COS, (rel, cos)


@pytest.mark.parametrize("kind", ["q4", "q8"])
@pytest.mark.parametrize("batch", [2, 3, 5, 8])
def test_gemv_batch(dev, kpath, kind, batch):
    n, k = 1024, 2560
    raw, rng = _tiles(kind, n, k, 5)
    x = synth.random_bf16(rng, (batch, k))
    y = ops.gemv(_dev_u8(raw, dev), kind, _dev_bf16(x, dev), n // 32, k // 256).cpu().numpy()
    ref = qo.gemv(raw, kind, x, n // 32, k // 256, acc=np.float64)
    for b in range(batch):
        rel, cos = qo.metrics(y[b], ref[b])
        assert rel < REL and cos > COS, (b, rel, cos)


@pytest.mark.parametrize("k,tiles_per_wave", [(2560, 1), (2560, 2), (2560, 4), (8192, 2), (8192, 4),
                                                (1024, 4)])
def test_gemv_tiles_per_wave(dev, general, k, tiles_per_wave):
    """Every wave/tile decomposition of the general VALU GEMV gives the same answer, run after
    run."""
    n = 512
    raw, rng = _tiles("q4", n, k, 6)
    x = synth.random_bf16(rng, k)
    w, xd = _dev_u8(raw, dev), _dev_bf16(x, dev)
    ref = qo.gemv(raw, "q4", x, n // 32, k // 256, acc=np.float64)
    pol = ops.current_policy().replace(gemv_tiles_per_wave=tiles_per_wave)
    y1 = ops.gemv(w, "q4", xd, n // 32, k // 256, policy=pol).cpu().numpy()
    y2 = ops.gemv(w, "q4", xd, n // 32, k // 256, policy=pol).cpu().numpy()
    rel, cos = qo.metrics(y1, ref)
    assert rel < REL and cos > COS, (rel, cos)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))  # deterministic


@pytest.mark.parametrize("kind,n,k,tiles_per_wave", [("q4", 8192, 2560, 1), ("q4", 8192, 2560, 2),
                                                     ("q4", 8192, 2560, 4), ("q4", 2560, 8192, 2),
                                                     ("q4", 2560, 8192, 4), ("q8", 4096, 1024, 2)])
def test_rowblock_tiles_per_wave(dev, valu, kind, n, k, tiles_per_wave):
    """The row-block kernel at every K-tiles-per-wave the policy may ask for: the oracle's
    answer, and the same bits run after run."""
    raw, rng = _tiles(kind, n, k, 7)
    x = synth.random_bf16(rng, k)
    w, xd = _dev_u8(raw, dev), _dev_bf16(x, dev)
    ref = qo.gemv(raw, kind, x, n // 32, k // 256, acc=np.float64)
    pol = ops.current_policy().replace(gemv_tiles_per_wave=tiles_per_wave)
    y1 = ops.gemv(w, kind, xd, n // 32, k // 256, policy=pol).cpu().numpy()
    y2 = ops.gemv(w, kind, xd, n // 32, k // 256, policy=pol).cpu().numpy()
    rel, cos = qo.metrics(y1, ref)
    assert rel < REL and cos > COS, (rel, cos)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


@pytest.mark.parametrize("kind", ["q4", "q8"])
@pytest.mark.parametrize("parts,batch,n,k", [(2, 1, 2560, 2560), (3, 3, 2560, 8192),
                                             (5, 1, 1024, 2560), (8, 8, 512, 8192),
                                             (0, 1, 2560, 8192), (0, 2, 2560, 2560)])
def test_gemv_ksplit(dev, general, kind, parts, batch, n, k):
    """K split over several workgroups per tile-row of the general VALU GEMV (last one adds
    the parts in order): same answer as the oracle, with a residual, bit-identical run after
    run."""
    raw, rng = _tiles(kind, n, k, 11)
    x = synth.random_bf16(rng, (batch, k))
    res = rng.standard_normal((batch, n)).astype(np.float32)
    w, xd, rd = _dev_u8(raw, dev), _dev_bf16(x, dev), torch.from_numpy(res).to(dev)
    ref = qo.gemv(raw, kind, x, n // 32, k // 256, acc=np.float64).reshape(batch, n) + res
    ws = ops.Workspace(1 << 20, device=dev)
    pol = ops.current_policy().replace(gemv_ksplit=parts)
    y1 = ops.gemv(w, kind, xd, n // 32, k // 256, residual=rd, ws=ws, policy=pol).cpu().numpy()
    y2 = ops.gemv(w, kind, xd, n // 32, k // 256, residual=rd, ws=ws, policy=pol).cpu().numpy()
    for b in range(batch):
        rel, cos = qo.metrics(y1[b], ref[b])
        assert rel < REL and cos > COS, (b, rel, cos)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


@pytest.mark.parametrize("batch", [1, 2])
@pytest.mark.parametrize("parts", [0, 1])
def test_gemv_ex_norm_ssq_and_keys(dev, kpath, parts, batch):
    """gemv_ex: RMSNorm prologue from an fp32 residual (with and without the producer's
    per-16 sums of squares), the sums of squares of its own output per 16-row block, and
    argmax keys that decode_advance turns into the first maximal row."""
    rng = np.random.default_rng(12)
    n, k = 2560, 8192
    raw, _ = _tiles("q4", n, k, 12)
    w = _dev_u8(raw, dev)
    h = (rng.standard_normal((batch, k)) * 5).astype(np.float32)
    nw = qo.bf16_round((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32))
    res = rng.standard_normal((batch, n)).astype(np.float32)
    hd, nwd = torch.from_numpy(h).to(dev), _dev_bf16(nw, dev)
    ss_in = torch.from_numpy((h.astype(np.float64).reshape(batch, -1, 16) ** 2).sum(-1)
                             .astype(np.float32)).to(dev)
    ss_out = torch.empty((batch, n // 16), dtype=torch.float32, device=dev)
    keys = torch.zeros((batch, n // 16), dtype=torch.int64, device=dev)
    pol = ops.current_policy().replace(gemv_ksplit=parts)
    ys = []
    for sin in (None, ss_in):
        ys.append(ops.gemv_ex(w, "q4", hd, n // 32, k // 256, norm_w=nwd, eps=1e-5,
                              residual=torch.from_numpy(res).to(dev), ssq_in=sin,
                              ssq_out=ss_out, argmax_keys=keys, policy=pol).cpu().numpy())
    hf = h.astype(np.float64)
    xn = qo.bf16_round((hf / np.sqrt((hf ** 2).mean(1, keepdims=True) + 1e-5)
                        * qo.bf16_to_f32(nw)).astype(np.float32))
    ref = qo.gemv(raw, "q4", xn, n // 32, k // 256, acc=np.float64).reshape(batch, n) + res
    for y in ys:
        for b in range(batch):
            rel, cos = qo.metrics(y[b], ref[b])
            assert rel < 1e-4 and cos > 0.999999, (b, rel, cos)   # xn may flip a bf16 ulp
    y = ys[-1]
    sref = (y.astype(np.float64).reshape(batch, -1, 16) ** 2).sum(-1)
    assert np.abs(ss_out.cpu().numpy() - sref).max() <= 1e-6 * sref.max()
    tok = torch.zeros(batch, dtype=torch.int32, device=dev)
    pos = torch.zeros(batch, dtype=torch.int32, device=dev)
    lens = torch.zeros(batch, dtype=torch.int32, device=dev)
    step = torch.zeros(1, dtype=torch.int32, device=dev)
    ops.decode_advance(keys, n // 16, tok, pos, lens, step)
    assert tok.cpu().numpy().tolist() == np.argmax(y, axis=1).tolist()


def test_gemv_residual_and_ones(dev, kpath):
    n, k = 2560, 2560
    raw, rng = _tiles("q4", n, k, 7)
    w = _dev_u8(raw, dev)
    res = rng.standard_normal(n).astype(np.float32)
    x = qo.bf16_round(np.ones(k, np.float32))
    y = ops.gemv(w, "q4", _dev_bf16(x, dev), n // 32, k // 256,
                 residual=torch.from_numpy(res).to(dev).reshape(1, n)).cpu().numpy()
    rowsum = qo.dequant_matrix(raw, "q4", n // 32, k // 256).astype(np.float64).sum(1)
    rel, cos = qo.metrics(y - res, rowsum)
    assert rel < REL and cos > COS


@pytest.mark.parametrize("scale", [1e-30, 1e-3, 1e4, 1e30])
def test_gemv_activation_range(dev, kpath, scale):
    """The per-workgroup power-of-two fp16 scaling keeps any bf16 range exact."""
    n, k = 256, 2560
    raw, rng = _tiles("q4", n, k, 8)
    xf = rng.standard_normal(k).astype(np.float32) * np.float32(scale)
    xf[::97] *= np.float32(1e-6)   # a spread of magnitudes inside one vector
    x = qo.bf16_round(xf)
    y = ops.gemv(_dev_u8(raw, dev), "q4", _dev_bf16(x, dev), n // 32, k // 256).cpu().numpy()
    ref = qo.gemv(raw, "q4", x, n // 32, k // 256, acc=np.float64)
    rel, cos = qo.metrics(y, ref)
    assert rel < REL and cos > COS, (rel, cos)


@pytest.mark.parametrize("kind", ["q4", "q8"])
@pytest.mark.parametrize("case", range(8))
def test_gemv_random_shapes(dev, kpath, kind, case):
    """Seeded random shapes off the usual grid (tile-row counts that do not fill a split,
    single-tile and long K, odd batches; beyond 8 rows on the matrix cores): every row within
    the bar of the float64 oracle."""
    rng = np.random.default_rng(1000 + 17 * case + (kind == "q8"))
    n_t = int(rng.integers(1, 200))
    k_t = int(rng.choice([1, 2, 3, 5, 7, 10, 13, 32, 40]))
    batch = int(rng.integers(1, 41 if kpath == "mfma" else 9))
    raw, rng2 = _tiles(kind, 32 * n_t, 256 * k_t, 2000 + case)
    x = synth.random_bf16(rng2, (batch, 256 * k_t))
    y = ops.gemv(_dev_u8(raw, dev), kind, _dev_bf16(x, dev), n_t, k_t).cpu().numpy()
    ref = qo.gemv(raw, kind, x, n_t, k_t, acc=np.float64).reshape(batch, -1)
    y = y.reshape(batch, -1)
    for b in range(batch):
        rel, cos = qo.metrics(y[b], ref[b])
        assert rel < REL and cos > COS, (n_t, k_t, batch, b, rel, cos)


@pytest.mark.parametrize("n,k", [(8192, 2560), (2560, 8192)])
@pytest.mark.parametrize("dist", ["student_t2", "outliers"])
def test_gemv_heavy_tailed_activations(dev, kpath, n, k, dist):
    """Heavy-tailed activations at the granite projection shapes: Student-t with 2 degrees
    of freedom, and Gaussians with a few entries 10^3-10^4 times larger (the outlier
    channels real activations have). Every product of the inner product stays exact and the
    per-wave fp16 scale follows the largest entry, so the bar is the same as for Gaussian x."""
    raw, rng = _tiles("q4", n, k, 31 if dist == "outliers" else 32)
    if dist == "student_t2":
        xf = rng.standard_t(2, size=(2, k)).astype(np.float32)
    else:
        xf = rng.standard_normal((2, k)).astype(np.float32)
        idx = rng.choice(k, size=(2, 6), replace=False)
        for b in range(2):
            xf[b, idx[b]] *= rng.choice([1e3, -1e3, 1e4, -1e4], size=6).astype(np.float32)
    x = qo.bf16_round(xf)
    w = _dev_u8(raw, dev)
    ref = qo.gemv(raw, "q4", x, n // 32, k // 256, acc=np.float64)
    for b in range(2):   # one row at a time (the batch-1 kernels), then both rows together
        y = ops.gemv(w, "q4", _dev_bf16(x[b], dev), n // 32, k // 256).cpu().numpy()
        rel, cos = qo.metrics(y, ref[b])
        assert rel < REL and cos > COS, (b, rel, cos)
    y2 = ops.gemv(w, "q4", _dev_bf16(x, dev), n // 32, k // 256).cpu().numpy()
    for b in range(2):
        rel, cos = qo.metrics(y2[b], ref[b])
        assert rel < REL and cos > COS, (b, rel, cos)


@pytest.mark.parametrize("k_t", [64, 65])
def test_gemv_longest_k(dev, kpath, k_t):
    """K = 16384 (64 K-tiles: sixteen waves of four K-tiles, the longest row a row-block
    workgroup covers) and one K-tile more (the general kernel takes it at one row)."""
    n = 256
    raw, rng = _tiles("q4", n, 256 * k_t, 70 + k_t)
    x = synth.random_bf16(rng, 256 * k_t)
    y = ops.gemv(_dev_u8(raw, dev), "q4", _dev_bf16(x, dev), n // 32, k_t).cpu().numpy()
    ref = qo.gemv(raw, "q4", x, n // 32, k_t, acc=np.float64)
    rel, cos = qo.metrics(y, ref)
    assert rel < REL and cos > COS, (rel, cos)
