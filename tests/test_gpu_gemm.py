"""GPU parity of the batched q4/q8 contraction on the matrix cores (`q4nx_gemm`) against the
oracle, for row counts from one (decode) to prefill lengths.

Bars: max|Δ|/max|ref| < 1e-5 against the float64 oracle with cosine > 0.9999999 for every
row (the reference's GEMV gate, designs/granite_gemv/granite_gemv.py:335, and its per-token
check of the batched design, granite_gemv32.py:279-288); one-hot rows reproduce the
float32 dequantised column bit-for-bit; split-K launches are bit-reproducible.
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


def _check_rows(y, ref):
    """Every row on its own, then the whole block."""
    for i in range(ref.shape[0]):
        rel, cos = qo.metrics(y[i], ref[i])
        assert rel < REL and cos > COS, (i, rel, cos)


@pytest.mark.parametrize("kind", ["q4", "q8"])
@pytest.mark.parametrize("m,n,k", [
    (1, 128, 512),
    (5, 128, 512),       # partial m-tile
    (16, 256, 768),
    (17, 256, 2560),     # two m-tiles, one of one row
    (33, 128, 1024),     # K split over two waves, two m-tiles per wave
    (64, 192, 768),
    (65, 256, 1024),     # prefill blocks: 128 rows per workgroup
    (200, 512, 2560),
    (8, 2560, 8192),     # down_proj shape, batch 8: split K across workgroups
])
def test_gemm_parity(dev, kind, m, n, k):
    raw, rng = _tiles(kind, n, k, 11 + m)
    x = synth.random_bf16(rng, (m, k))
    y = ops.gemm(_dev_u8(raw, dev), kind, _dev_bf16(x, dev), n // 32, k // 256).cpu().numpy()
    ref = qo.gemv(raw, kind, x, n // 32, k // 256, acc=np.float64)
    _check_rows(y, ref)


@pytest.mark.parametrize("kind", ["q4", "q8"])
def test_gemm_onehot_exact(dev, kind):
    """Row i of x is the unit vector e_{k_i}: row i of y is column k_i of the float32
    dequantised matrix, bit for bit (code * d + m rounds once, as tools/q4nx.py:127-137)."""
    n, k = 96, 1024
    raw, _ = _tiles(kind, n, k, 2)
    cols = [0, 1, 7, 8, 31, 32, 255, 256, 511, 777, 1000, 1023, 5, 600, 64, 130, 900]
    x = np.zeros((len(cols), k), np.float32)
    x[np.arange(len(cols)), cols] = 1.0
    y = ops.gemm(_dev_u8(raw, dev), kind, _dev_bf16(qo.bf16_round(x), dev), n // 32,
                 k // 256).cpu().numpy()
    wm = qo.dequant_matrix(raw, kind, n // 32, k // 256)
    for i, kk in enumerate(cols):
        assert np.array_equal(y[i].view(np.uint32), wm[:, kk].view(np.uint32)), kk


@pytest.mark.parametrize("scale", [1e-30, 1e-3, 1e4, 1e30])
def test_gemm_activation_range(dev, scale):
    """bf16 x enters the matrix cores unchanged: any bf16 range is exact input."""
    m, n, k = 24, 256, 2560
    raw, rng = _tiles("q4", n, k, 8)
    xf = rng.standard_normal((m, k)).astype(np.float32) * np.float32(scale)
    xf[:, ::97] *= np.float32(1e-6)
    x = qo.bf16_round(xf)
    y = ops.gemm(_dev_u8(raw, dev), "q4", _dev_bf16(x, dev), n // 32, k // 256).cpu().numpy()
    ref = qo.gemv(raw, "q4", x, n // 32, k // 256, acc=np.float64)
    _check_rows(y, ref)


def test_gemm_heavy_tailed(dev):
    """Student-t(2) activations: a few entries dwarf the rest."""
    m, n, k = 12, 512, 8192
    raw, rng = _tiles("q4", n, k, 9)
    x = qo.bf16_round(rng.standard_t(2.0, (m, k)).astype(np.float32))
    y = ops.gemm(_dev_u8(raw, dev), "q4", _dev_bf16(x, dev), n // 32, k // 256).cpu().numpy()
    ref = qo.gemv(raw, "q4", x, n // 32, k // 256, acc=np.float64)
    _check_rows(y, ref)


def test_gemm_residual_strided_x(dev):
    """x rows with a stride longer than K, and a residual added once."""
    m, n, k = 40, 256, 1536
    raw, rng = _tiles("q4", n, k, 10)
    xfull = synth.random_bf16(rng, (m, k + 64))
    xd = _dev_bf16(xfull, dev)[:, :k]
    res = rng.standard_normal((m, n)).astype(np.float32)
    y = ops.gemm(_dev_u8(raw, dev), "q4", xd, n // 32, k // 256,
                 residual=torch.from_numpy(res).to(dev)).cpu().numpy()
    ref = qo.gemv(raw, "q4", np.ascontiguousarray(xfull[:, :k]), n // 32, k // 256,
                  acc=np.float64) + res
    _check_rows(y, ref)


@pytest.mark.parametrize("parts", [1, 2, 3, 5])
@pytest.mark.parametrize("n,m", [(2560, 3), (2560, 30), (2560, 100),
                                 (512, 3), (512, 12)])   # 16 tile-rows: row-block workgroups
def test_gemm_ksplit_deterministic(dev, parts, m, n):
    """Any split of K gives the oracle's result, and the same bits on every call (with 16
    tile-rows and one m-tile the parts are row-block workgroups, two per tile-row)."""
    k = 8192
    raw, rng = _tiles("q4", n, k, 12)
    w = _dev_u8(raw, dev)
    x = synth.random_bf16(rng, (m, k))
    xd = _dev_bf16(x, dev)
    pol = ops.Policy(gemm_ksplit=parts)
    y1 = ops.gemm(w, "q4", xd, n // 32, k // 256, policy=pol).cpu().numpy()
    y2 = ops.gemm(w, "q4", xd, n // 32, k // 256, policy=pol).cpu().numpy()
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    ref = qo.gemv(raw, "q4", x, n // 32, k // 256, acc=np.float64)
    _check_rows(y1, ref)


@pytest.mark.parametrize("parts", [1, 3])
def test_gemm_q8_rowblock_split(dev, parts):
    """q8 tiles on row-block workgroups (16 tile-rows, 3 rows), whole and with K in 3 parts:
    each workgroup stages the scales and its block's 4096 code bytes (the last load of lanes
    32..63 lands in the slot's padding)."""
    n, k, m = 512, 8192, 3
    raw, rng = _tiles("q8", n, k, 15)
    x = synth.random_bf16(rng, (m, k))
    y = ops.gemm(_dev_u8(raw, dev), "q8", _dev_bf16(x, dev), n // 32, k // 256,
                 policy=ops.Policy(gemm_ksplit=parts)).cpu().numpy()
    _check_rows(y, qo.gemv(raw, "q8", x, n // 32, k // 256, acc=np.float64))


@pytest.mark.parametrize("kind", ["q4", "q8"])
def test_gemm_matches_gemv_batch(dev, kind):
    """For the batch sizes both paths take, the two agree to the oracle's bar."""
    n, k, b = 1024, 2560, 8
    raw, rng = _tiles(kind, n, k, 13)
    w = _dev_u8(raw, dev)
    x = synth.random_bf16(rng, (b, k))
    xd = _dev_bf16(x, dev)
    y_mma = ops.gemm(w, kind, xd, n // 32, k // 256).cpu().numpy()
    y_vec = ops.gemv(w, kind, xd, n // 32, k // 256).cpu().numpy()
    ref = qo.gemv(raw, kind, x, n // 32, k // 256, acc=np.float64)
    _check_rows(y_mma, ref)
    _check_rows(y_vec, ref)


def test_gemm_q8_lm_head_prefill(dev):
    """The tied lm_head shape of the granite-3B step (q8 2560 -> 100352) over 48 prompt rows,
    checked against the oracle on a slice of the vocabulary."""
    n, k, m = 100352, 2560, 48
    rng = np.random.default_rng(14)
    raw = synth.q8_tiles(rng, n, k).reshape(-1, qo.Q8_TILE_BYTES)
    x = synth.random_bf16(rng, (m, k))
    y = ops.gemm(_dev_u8(raw, dev), "q8", _dev_bf16(x, dev), n // 32, k // 256).cpu().numpy()
    lo, hi = 96 * 32, 160 * 32   # tile-rows 96..159
    k_t = k // 256
    ref = qo.gemv(raw[lo // 32 * k_t: hi // 32 * k_t], "q8", x, (hi - lo) // 32, k_t,
                  acc=np.float64)
    _check_rows(y[:, lo:hi], ref)


# ------------------------------------------------------------------ prompt blocks (prefill kernel)
# Launches that fill the chip go to the prefill kernel (raw codes on the matrix cores, the
# group scale on the VALU, the minimum as a contraction over per-group sums of x): blocks of
# 128 rows from 768 workgroups of four tile-rows, else 64-row blocks from 512; smaller
# launches stay on the batched kernel above.

def _pf_workgroups(m, n, rows=128):
    return -(-(n // 32) // 4) * -(-m // rows)


def _pf_block_rows(m, n):
    """Row-block size the library picks (0: not the prefill kernel)."""
    if m >= 128 and _pf_workgroups(m, n, 128) >= 768:
        return 128
    if m >= 128 and _pf_workgroups(m, n, 64) >= 512:
        return 64
    return 0


@pytest.mark.parametrize("kind", ["q4", "q8"])
@pytest.mark.parametrize("m,n,k", [
    (4100, 2016, 512),   # 63 tile-rows: the last workgroup's fourth wave has none; ragged rows
    (2048, 4096, 1024),
    (1544, 8192, 768),   # 128-row blocks; ragged rows, a partial chunk of groups (3 K-tiles)
    (3100, 4064, 512),   # 128-row blocks, 127 tile-rows: the last workgroup's last wave has none
])
def test_gemm_prefill_parity(dev, kind, m, n, k):
    """Every row against the float64 oracle at the GEMV bar."""
    assert _pf_block_rows(m, n) > 0
    raw, rng = _tiles(kind, n, k, 21 + m)
    x = synth.random_bf16(rng, (m, k))
    y = ops.gemm(_dev_u8(raw, dev), kind, _dev_bf16(x, dev), n // 32, k // 256).cpu().numpy()
    ref = qo.gemv(raw, kind, x, n // 32, k // 256, acc=np.float64)
    _check_rows(y, ref)


def test_gemm_prefill_long_k(dev):
    """K = 8192 (32 tiles per wave, 256 pipelined steps): every row at the GEMV bar."""
    m, n, k = 2048, 4096, 8192
    raw, rng = _tiles("q4", n, k, 23)
    x = synth.random_bf16(rng, (m, k))
    y = ops.gemm(_dev_u8(raw, dev), "q4", _dev_bf16(x, dev), n // 32, k // 256).cpu().numpy()
    ref = qo.gemv(raw, "q4", x, n // 32, k // 256, acc=np.float64)
    _check_rows(y, ref)


@pytest.mark.parametrize("kind", ["q4", "q8"])
@pytest.mark.parametrize("n,m", [(2048, 4096), (8192, 1536)])   # 64- and 128-row blocks
def test_gemm_prefill_onehot_exact(dev, kind, n, m):
    """One-hot rows reproduce the float32 dequantised column bit for bit: d (16 + c) (q4) or
    s (q + 128) (q8) is exact, and so is its sum with the minimum term."""
    k = 1024
    assert _pf_block_rows(m, n) == (64 if n == 2048 else 128)
    raw, _ = _tiles(kind, n, k, 3)
    cols = np.arange(m) * 5 % k
    x = np.zeros((m, k), np.float32)
    x[np.arange(m), cols] = 1.0
    y = ops.gemm(_dev_u8(raw, dev), kind, _dev_bf16(qo.bf16_round(x), dev), n // 32,
                 k // 256).cpu().numpy()
    wm = qo.dequant_matrix(raw, kind, n // 32, k // 256)
    assert np.array_equal(y.view(np.uint32), wm[:, cols].T.copy().view(np.uint32))


@pytest.mark.parametrize("dist", ["student_t2", "outliers"])
def test_gemm_prefill_heavy_tailed(dev, dist):
    """Heavy-tailed activations on both row-block sizes: a few entries dwarf the rest of their
    32-K group, so the group sums S carry most of the minimum term and the scaled code sums
    cancel against it."""
    k = 1024
    for m, n in ((1536, 8192), (2048, 2048)):
        assert _pf_block_rows(m, n) > 0
        raw, rng = _tiles("q4", n, k, 31 + m)
        if dist == "student_t2":
            xf = rng.standard_t(2.0, (m, k)).astype(np.float32)
        else:
            xf = rng.standard_normal((m, k)).astype(np.float32)
            hit = rng.random((m, k)) < 1e-3
            xf[hit] *= np.float32(1e4)
        x = qo.bf16_round(xf)
        y = ops.gemm(_dev_u8(raw, dev), "q4", _dev_bf16(x, dev), n // 32, k // 256).cpu().numpy()
        ref = qo.gemv(raw, "q4", x, n // 32, k // 256, acc=np.float64)
        _check_rows(y, ref)


@pytest.mark.parametrize("scale", [1e-30, 1e30])
def test_gemm_prefill_activation_range_residual_stride(dev, scale):
    """Extreme activation ranges, rows with a stride longer than K and a residual."""
    m, n, k = 4096, 2048, 512
    assert _pf_block_rows(m, n) > 0
    raw, rng = _tiles("q4", n, k, 14)
    xf = rng.standard_normal((m, k + 64)).astype(np.float32) * np.float32(scale)
    xfull = qo.bf16_round(xf)
    xd = _dev_bf16(xfull, dev)[:, :k]
    res = rng.standard_normal((m, n)).astype(np.float32) * np.float32(scale)
    y = ops.gemm(_dev_u8(raw, dev), "q4", xd, n // 32, k // 256,
                 residual=torch.from_numpy(res).to(dev)).cpu().numpy()
    ref = qo.gemv(raw, "q4", np.ascontiguousarray(xfull[:, :k]), n // 32, k // 256,
                  acc=np.float64) + res
    _check_rows(y, ref)


@pytest.mark.parametrize("kind", ["q4", "q8"])
@pytest.mark.parametrize("m,n,k", [(2048, 4096, 256), (1536, 8192, 512), (2048, 4096, 768)])
def test_gemm_prefill_short_k(dev, kind, m, n, k):
    """One to three K-tiles per tile-row: the first tile's reload, the clamped prefetch of the
    tile after the last and the steps of x past the end all stay unused."""
    assert _pf_block_rows(m, n) > 0
    raw, rng = _tiles(kind, n, k, 41 + k)
    x = synth.random_bf16(rng, (m, k))
    y = ops.gemm(_dev_u8(raw, dev), kind, _dev_bf16(x, dev), n // 32, k // 256).cpu().numpy()
    ref = qo.gemv(raw, kind, x, n // 32, k // 256, acc=np.float64)
    _check_rows(y, ref)


def test_gemm_prefill_without_workspace(dev):
    """A prompt block with no workspace (NULL, 0), or one too small for the per-group sums of
    x, runs on the batched kernel instead: every row at the same bar."""
    from llmnputest_amd import _lib
    m, n, k = 2048, 4096, 512
    assert _pf_block_rows(m, n) > 0
    raw, rng = _tiles("q4", n, k, 43)
    x = synth.random_bf16(rng, (m, k))
    w, xd = _dev_u8(raw, dev), _dev_bf16(x, dev)
    ref = qo.gemv(raw, "q4", x, n // 32, k // 256, acc=np.float64)
    need = _lib.lib().q4nx_gemm_ws_bytes(4, n // 32, k // 256, m, None)
    small = torch.empty(need // 2, dtype=torch.uint8, device=dev)
    for wp, wn in ((None, 0), (small.data_ptr(), small.numel())):
        y = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        _lib.call("q4nx_gemm", 4, w.data_ptr(), n // 32, k // 256, xd.data_ptr(), k, m,
                  y.data_ptr(), n, None, wp, wn, None, ops._stream())
        _check_rows(y.cpu().numpy(), ref)
