"""GPU parity of RMSNorm, RoPE, SwiGLU, the fused groups and GQA decode attention.

fp32 outputs (the pre-rounding values) are held to max|Δ|/max|ref| < 1e-5 against the
float64 oracle with cosine >= 0.9999; bf16 outputs are compared with the oracle rounded
the same way and may differ only by rare 1-ulp flips where the fp32 value sits on a
rounding boundary (see `assert_bf16_close`).
"""

import numpy as np
import pytest
import torch

from llmnputest_amd import ops, synth
from llmnputest_amd._lib import Q4NXError
from oracle import decode_oracle as do
from oracle import q4nx_oracle as qo

pytestmark = pytest.mark.gpu

REL = 1e-5
COS = 0.9999


def bf16_dev(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).to(dev).view(torch.bfloat16)


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def assert_close(got, ref, rel=REL, cos=COS):
    r, c = qo.metrics(got, ref)
    assert r < rel and c >= cos, (r, c)


def assert_bf16_close(got_bits, ref_f64, max_frac=1e-3):
    """bf16 outputs equal the oracle's RNE rounding except for rare 1-ulp boundary flips."""
    want = qo.bf16_round(np.asarray(ref_f64, np.float64).astype(np.float32))
    g = np.asarray(got_bits, np.uint16).ravel().astype(np.int32)
    w = want.ravel().astype(np.int32)
    diff = np.abs(g - w)
    assert diff.max() <= 1, int(diff.max())
    assert (diff > 0).mean() <= max_frac, float((diff > 0).mean())


# ------------------------------------------------------------------ bf16 rounding

def test_round_bf16_bitexact(dev):
    """The device rounding every kernel uses equals the oracle's RNE on every class of
    input: both parities of exact halfway cases, subnormals, infinities, extremes, NaN."""
    rng = np.random.default_rng(9)
    halves = (np.arange(1 << 16, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    near = (np.arange(1 << 16, dtype=np.uint32) << 16 | 0x7FFF).view(np.float32)
    sub = (rng.integers(1, 1 << 23, 20000, dtype=np.uint32)).view(np.float32)
    edge = np.array([0.0, -0.0, np.inf, -np.inf, 3.4028235e38, -3.4028235e38, 1e-45, 2 ** -126,
                     3.3961776e38, 65504.0], np.float32)
    x = np.concatenate([halves, near, sub, -sub, edge,
                        rng.standard_normal(100000).astype(np.float32) * 1e3])
    finite_or_inf = ~np.isnan(x)
    got = bits(ops.round_bf16(torch.from_numpy(x).to(dev)))
    want = qo.bf16_round(x)
    assert np.array_equal(got[finite_or_inf], want[finite_or_inf])
    assert np.isnan(qo.bf16_to_f32(got[~finite_or_inf])).all()


# ------------------------------------------------------------------ RMSNorm

@pytest.mark.parametrize("xdtype", ["bf16", "f32"])
def test_rmsnorm(dev, xdtype):
    rng = np.random.default_rng(10)
    b, c = 3, 2560
    w = synth.f32_to_bf16_bits(1.0 + 0.1 * rng.standard_normal(c).astype(np.float32))
    if xdtype == "bf16":
        xb = synth.random_bf16(rng, (b, c))
        x_host = qo.bf16_to_f32(xb)
        x_dev = bf16_dev(xb, dev)
    else:
        x_host = (rng.standard_normal((b, c)) * 30).astype(np.float32)
        x_dev = torch.from_numpy(x_host).to(dev)
    y, yf = ops.rmsnorm(x_dev, bf16_dev(w, dev), 1e-5, want_f32=True)
    ref = do.rmsnorm(x_host, w, 1e-5)
    assert_close(yf.cpu().numpy(), ref)
    assert_bf16_close(bits(y), ref)
    # the weight is non-uniform, so dropping it would fail (granite_rmsnorm.py:132-134)
    unit = do.rmsnorm(x_host, synth.f32_to_bf16_bits(np.ones(c, np.float32)), 1e-5)
    assert qo.metrics(yf.cpu().numpy(), unit)[0] > 0.05


# ------------------------------------------------------------------ RoPE

def test_rope(dev):
    rng = np.random.default_rng(11)
    b, h = 8, 40
    x = synth.random_bf16(rng, (b, h, 64))
    pos = rng.integers(0, 4096, b).astype(np.int32)
    tab_np = do.rope_table(4096, 64, 10000.0)
    tab = ops.rope_table(4096, 64, 10000.0)
    assert np.allclose(tab.cpu().numpy(), tab_np, rtol=0, atol=1e-7)
    y, yf = ops.rope(bf16_dev(x, dev), torch.from_numpy(pos).to(dev), tab, want_f32=True)
    ref = np.stack([do.rope(qo.bf16_to_f32(x[i]), pos[i], tab_np) for i in range(b)])
    assert_close(yf.cpu().numpy(), ref)
    assert_bf16_close(bits(y), ref)
    alt = np.stack([do.rope_interleaved(qo.bf16_to_f32(x[i]), pos[i], tab_np) for i in range(b)])
    assert qo.metrics(yf.cpu().numpy(), alt)[0] > 0.1     # granite_elementwise.py:153-162
    y0 = ops.rope(bf16_dev(x, dev), torch.zeros(b, dtype=torch.int32, device=dev), tab)
    assert np.array_equal(bits(y0), x)                    # position 0 is the identity


# ------------------------------------------------------------------ SwiGLU

@pytest.mark.parametrize("in_f32", [False, True])
def test_swiglu(dev, in_f32):
    rng = np.random.default_rng(12)
    b, n = 2, 8192
    if in_f32:
        g = (rng.standard_normal((b, n)) * 3).astype(np.float32)
        u = (rng.standard_normal((b, n)) * 3).astype(np.float32)
        gd, ud = torch.from_numpy(g).to(dev), torch.from_numpy(u).to(dev)
        ref = do.swiglu_from_raw(g, u)
    else:
        gb, ub = synth.random_bf16(rng, (b, n), 3.0), synth.random_bf16(rng, (b, n), 3.0)
        gd, ud = bf16_dev(gb, dev), bf16_dev(ub, dev)
        ref = do.swiglu(qo.bf16_to_f32(gb), qo.bf16_to_f32(ub))
    y, yf = ops.swiglu(gd, ud, want_f32=True)
    assert_close(yf.cpu().numpy(), ref)
    assert_bf16_close(bits(y), ref)
    assert (yf.cpu().numpy() != 0).sum() == (ref != 0).sum()   # whole vector processed


# ------------------------------------------------------------------ fused [q,k,v,RoPE]

@pytest.fixture
def ksplit(request, vpath):
    """Force the general GEMV's K-split (0 = automatic) for one test on top of its VALU
    kernel family."""
    with ops.policy_scope(ops.current_policy().replace(gemv_ksplit=request.param)):
        yield request.param


@pytest.mark.parametrize("batch,norm,ksplit", [(1, False, 0), (1, True, 0), (3, True, 0),
                                               (3, True, 1), (2, True, 8)],
                         indirect=["ksplit"])
def test_qkv_rope(dev, vpath, batch, norm, ksplit):
    rng = np.random.default_rng(13)
    hq, hkv, hid, lmax = 40, 8, 2560, 512
    kt = hid // 256
    wq = synth.q4_tiles(rng, hq * 64, hid).reshape(-1, 5120)
    wk = synth.q4_tiles(rng, hkv * 64, hid).reshape(-1, 5120)
    wv = synth.q4_tiles(rng, hkv * 64, hid).reshape(-1, 5120)
    pos = rng.integers(0, lmax, batch).astype(np.int32)
    tab_np = do.rope_table(lmax, 64, 10000.0)
    tab = ops.rope_table(lmax, 64, 10000.0)
    kc = torch.zeros((batch, hkv, lmax, 64), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    nraw = (hq + 2 * hkv) * 64
    raw = torch.empty((batch, nraw), dtype=torch.float32, device=dev)
    xn = torch.empty((batch, hid), dtype=torch.bfloat16, device=dev)
    nw = synth.f32_to_bf16_bits(1.0 + 0.1 * rng.standard_normal(hid).astype(np.float32))
    if norm:
        h = (rng.standard_normal((batch, hid)) * 20).astype(np.float32)
        x_dev = torch.from_numpy(h).to(dev)
        norm_dev = bf16_dev(nw, dev)
    else:
        xb = synth.random_bf16(rng, (batch, hid))
        x_dev = bf16_dev(xb, dev)
        norm_dev = None
    d = lambda a: torch.from_numpy(a.reshape(-1)).to(dev)
    q = ops.qkv_rope(d(wq), d(wk), d(wv), hq, hkv, kt, x_dev, torch.from_numpy(pos).to(dev), tab,
                     kc, vc, norm_w=norm_dev, raw_out=raw, xn_out=xn if norm else None)
    torch.cuda.synchronize()
    if norm:
        ref_xn = do.rmsnorm(h, nw, 1e-5)
        assert_bf16_close(bits(xn), ref_xn, max_frac=2e-3)
        x_used = bits(xn)            # teacher-force the GEMV on the kernel's own input
    else:
        x_used = xb
    raw_np = raw.cpu().numpy()
    ref_q = qo.gemv(wq, "q4", x_used, hq * 2, kt, acc=np.float64).reshape(batch, -1)
    ref_k = qo.gemv(wk, "q4", x_used, hkv * 2, kt, acc=np.float64).reshape(batch, -1)
    ref_v = qo.gemv(wv, "q4", x_used, hkv * 2, kt, acc=np.float64).reshape(batch, -1)
    assert_close(raw_np, np.concatenate([ref_q, ref_k, ref_v], axis=1))
    # epilogue on the kernel's own accumulators: narrow, rotate q and k, narrow v
    qr, kr, vr = do.qkv_rope_from_raw(raw_np[:, :hq * 64], raw_np[:, hq * 64:(hq + hkv) * 64],
                                      raw_np[:, (hq + hkv) * 64:], pos, tab_np)
    assert_bf16_close(bits(q).reshape(batch, hq, 64), qr)
    kcn, vcn = bits(kc), bits(vc)
    for b in range(batch):
        assert_bf16_close(kcn[b, :, pos[b]], kr[b])
        assert np.array_equal(vcn[b, :, pos[b]], qo.bf16_round(vr[b].astype(np.float32)))
        mask = np.ones(lmax, bool)
        mask[pos[b]] = False
        assert not kcn[b][:, mask].any() and not vcn[b][:, mask].any()   # nothing else written


@pytest.mark.parametrize("batch", [1, 3, 8])
def test_qkv_rope_positions_outside_cache(dev, kpath, batch):
    """A row whose position lies outside [0, max_pos) writes neither its q nor the caches (its
    raw GEMV outputs are still written); every other row is bit for bit what the same launch
    writes with all positions valid. Positions -1 and max_pos, on every kernel family."""
    rng = np.random.default_rng(29)
    hq, hkv, hid, lmax = 40, 8, 2560, 64
    kt = hid // 256
    d = lambda a: torch.from_numpy(a.reshape(-1)).to(dev)
    wq = d(synth.q4_tiles(rng, hq * 64, hid))
    wk = d(synth.q4_tiles(rng, hkv * 64, hid))
    wv = d(synth.q4_tiles(rng, hkv * 64, hid))
    x = bf16_dev(synth.random_bf16(rng, (batch, hid)), dev)
    tab = ops.rope_table(lmax, 64, 10000.0)
    good = rng.integers(0, lmax, batch).astype(np.int32)
    bad = good.copy()
    bad[0] = -1
    if batch > 1:
        bad[-1] = lmax
    sentinel = 0x1234

    def run(pos):
        kc = torch.zeros((batch, hkv, lmax, 64), dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        q = torch.full((batch, hq * 64), sentinel, dtype=torch.int16, device=dev).view(torch.bfloat16)
        raw = torch.empty((batch, (hq + 2 * hkv) * 64), dtype=torch.float32, device=dev)
        ops.qkv_rope(wq, wk, wv, hq, hkv, kt, x, torch.from_numpy(pos).to(dev), tab, kc, vc,
                     q_out=q, raw_out=raw)
        torch.cuda.synchronize()
        return bits(q), bits(kc), bits(vc), raw.cpu().numpy()

    q_g, k_g, v_g, raw_g = run(good)
    q_b, k_b, v_b, raw_b = run(bad)
    assert np.array_equal(raw_b, raw_g)
    for b in range(batch):
        if 0 <= bad[b] < lmax:
            assert np.array_equal(q_b[b], q_g[b])
            assert np.array_equal(k_b[b], k_g[b]) and np.array_equal(v_b[b], v_g[b])
        else:
            assert (q_b[b] == sentinel).all()
            assert not k_b[b].any() and not v_b[b].any()
            assert k_g[b].any()   # the valid launch did write this row


@pytest.mark.parametrize("batch,ksplit", [(1, 0), (3, 0), (2, 1)], indirect=["ksplit"])
def test_qkv_rope_ssq_in(dev, vpath, batch, ksplit):
    """The norm fed the producer's per-16 sums of squares gives the same normalised input
    (to bf16 rounding) and GEMV outputs as the oracle on that input."""
    rng = np.random.default_rng(23)
    hq, hkv, hid, lmax = 40, 8, 2560, 128
    kt = hid // 256
    wq = synth.q4_tiles(rng, hq * 64, hid).reshape(-1, 5120)
    wk = synth.q4_tiles(rng, hkv * 64, hid).reshape(-1, 5120)
    wv = synth.q4_tiles(rng, hkv * 64, hid).reshape(-1, 5120)
    pos = rng.integers(0, lmax, batch).astype(np.int32)
    tab = ops.rope_table(lmax, 64, 10000.0)
    kc = torch.zeros((batch, hkv, lmax, 64), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    raw = torch.empty((batch, (hq + 2 * hkv) * 64), dtype=torch.float32, device=dev)
    xn = torch.empty((batch, hid), dtype=torch.bfloat16, device=dev)
    nw = synth.f32_to_bf16_bits(1.0 + 0.1 * rng.standard_normal(hid).astype(np.float32))
    h = (rng.standard_normal((batch, hid)) * 20).astype(np.float32)
    ss = torch.from_numpy(ssq16(h).astype(np.float32)).to(dev)
    d = lambda a: torch.from_numpy(a.reshape(-1)).to(dev)
    ops.qkv_rope(d(wq), d(wk), d(wv), hq, hkv, kt, torch.from_numpy(h).to(dev),
                 torch.from_numpy(pos).to(dev), tab, kc, vc, norm_w=bf16_dev(nw, dev),
                 raw_out=raw, xn_out=xn, ssq_in=ss)
    assert_bf16_close(bits(xn), do.rmsnorm(h, nw, 1e-5), max_frac=2e-3)
    x_used = bits(xn)
    ref = np.concatenate([qo.gemv(w_, "q4", x_used, n, kt, acc=np.float64).reshape(batch, -1)
                          for w_, n in ((wq, hq * 2), (wk, hkv * 2), (wv, hkv * 2))], axis=1)
    assert_close(raw.cpu().numpy(), ref)


# ------------------------------------------------------------------ fused [gate,up,SwiGLU]

@pytest.mark.parametrize("batch,norm,ksplit", [(1, False, 0), (2, True, 0), (1, True, 2),
                                               (3, True, 5)], indirect=["ksplit"])
def test_gate_up_swiglu(dev, vpath, batch, norm, ksplit):
    rng = np.random.default_rng(14)
    hid, inter = 2560, 8192
    kt = hid // 256
    wg = synth.q4_tiles(rng, inter, hid).reshape(-1, 5120)
    wu = synth.q4_tiles(rng, inter, hid).reshape(-1, 5120)
    raw = torch.empty((batch, 2 * inter), dtype=torch.float32, device=dev)
    xn = torch.empty((batch, hid), dtype=torch.bfloat16, device=dev)
    if norm:
        h = (rng.standard_normal((batch, hid)) * 20).astype(np.float32)
        nw = synth.f32_to_bf16_bits(1.0 + 0.1 * rng.standard_normal(hid).astype(np.float32))
        x_dev, norm_dev = torch.from_numpy(h).to(dev), bf16_dev(nw, dev)
    else:
        xb = synth.random_bf16(rng, (batch, hid))
        x_dev, norm_dev = bf16_dev(xb, dev), None
    d = lambda a: torch.from_numpy(a.reshape(-1)).to(dev)
    hout = ops.gate_up_swiglu(d(wg), d(wu), inter // 32, kt, x_dev, norm_w=norm_dev,
                              raw_out=raw, xn_out=xn if norm else None)
    torch.cuda.synchronize()
    if norm:
        assert_bf16_close(bits(xn), do.rmsnorm(h, nw, 1e-5), max_frac=2e-3)
        x_used = bits(xn)
    else:
        x_used = xb
    raw_np = raw.cpu().numpy()
    ref_g = qo.gemv(wg, "q4", x_used, inter // 32, kt, acc=np.float64).reshape(batch, -1)
    ref_u = qo.gemv(wu, "q4", x_used, inter // 32, kt, acc=np.float64).reshape(batch, -1)
    assert_close(raw_np, np.concatenate([ref_g, ref_u], axis=1))
    ref_h = do.swiglu_from_raw(raw_np[:, :inter], raw_np[:, inter:])
    assert_bf16_close(bits(hout), ref_h)


# ------------------------------------------------------------------ attention

@pytest.mark.parametrize("batch,L,ragged", [
    (1, 1, False), (1, 32, False), (1, 100, False), (1, 512, False), (1, 4096, False),
    (8, 512, True), (8, 2112, True), (8, 4096, False), (1, 32768, False),
])
def test_gqa_decode(dev, apath, batch, L, ragged):
    rng = np.random.default_rng(15 + L)
    hq, hkv = 40, 8
    q = synth.random_bf16(rng, (batch, hq, 64))
    k = synth.random_bf16(rng, (batch, hkv, L, 64))
    v = synth.random_bf16(rng, (batch, hkv, L, 64))
    lens = (rng.integers(1, L + 1, batch) if ragged else np.full(batch, L)).astype(np.int32)
    out, of = ops.gqa_decode(bf16_dev(q, dev), bf16_dev(k, dev), bf16_dev(v, dev),
                             torch.from_numpy(lens).to(dev), 0.125, want_f32=True)
    ref = do.gqa_attention(qo.bf16_to_f32(q), qo.bf16_to_f32(k), qo.bf16_to_f32(v), lens, 0.125)
    assert_close(of.cpu().numpy(), ref)
    assert_bf16_close(bits(out), ref)
    if L == 1:
        expect = np.repeat(qo.bf16_to_f32(v)[:, :, 0], hq // hkv, axis=1)
        assert np.array_equal(of.cpu().numpy(), expect)     # one position: out = V[0]


def test_gqa_decode_uniform_softmax(dev, apath):
    """Constant K gives a uniform softmax, so out = mean(V) (a closed form)."""
    rng = np.random.default_rng(16)
    L = 1000
    q = synth.random_bf16(rng, (1, 40, 64))
    k = np.tile(synth.random_bf16(rng, (1, 8, 1, 64)), (1, 1, L, 1))
    v = synth.random_bf16(rng, (1, 8, L, 64))
    of = ops.gqa_decode(bf16_dev(q, dev), bf16_dev(k, dev), bf16_dev(v, dev),
                        torch.full((1,), L, dtype=torch.int32, device=dev), 0.125,
                        want_f32=True)[1]
    expect = np.repeat(qo.bf16_to_f32(v).astype(np.float64).mean(axis=2), 5, axis=1)
    assert_close(of.cpu().numpy(), expect)


def test_gqa_decode_uniform_full_size(dev, apath):
    """The largest attention config (batch 8, 32768 positions, 40 q / 8 kv heads: 537 MB of
    K/V, the streaming-load variant) through a closed form: K constant along the positions
    makes the softmax uniform, so each output is the mean of V over its sequence's length
    (ragged lengths, including one position)."""
    b, hq, hkv, L = 8, 40, 8, 32768
    gen = torch.Generator(device=dev)
    gen.manual_seed(81)
    q = torch.randn(b, hq, 64, device=dev, generator=gen).to(torch.bfloat16)
    krow = torch.randn(b, hkv, 1, 64, device=dev, generator=gen).to(torch.bfloat16)
    k = krow.expand(b, hkv, L, 64).contiguous()
    v = torch.randn(b, hkv, L, 64, device=dev, generator=gen).to(torch.bfloat16)
    lens = torch.tensor([L, 1, 4095, 20000, 32767, 129, 8192, 30001], dtype=torch.int32,
                        device=dev)
    of = ops.gqa_decode(q, k, v, lens, 0.125, want_f32=True)[1]
    ref = torch.empty((b, hq, 64), dtype=torch.float64, device=dev)
    for i in range(b):
        m = v[i, :, :int(lens[i])].double().mean(dim=1)          # [hkv, 64]
        ref[i] = m.repeat_interleave(hq // hkv, dim=0)
    assert_close(of.cpu().numpy(), ref.cpu().numpy())
    del k, v


@pytest.mark.parametrize("hq,hkv,L", [(8, 8, 300), (16, 2, 1500), (64, 8, 700), (24, 8, 129)])
def test_gqa_decode_group_sizes(dev, apath, hq, hkv, L):
    """Other query-group sizes (1, 8, 8, 3 query heads per kv head), called twice on one
    workspace so the split counters must have been left at zero."""
    rng = np.random.default_rng(19 + hq)
    q = synth.random_bf16(rng, (2, hq, 64))
    k = synth.random_bf16(rng, (2, hkv, L, 64))
    v = synth.random_bf16(rng, (2, hkv, L, 64))
    lens = np.array([L, max(1, L // 3)], np.int32)
    ws = ops.Workspace(8 << 20, device=dev)
    args = (bf16_dev(q, dev), bf16_dev(k, dev), bf16_dev(v, dev), torch.from_numpy(lens).to(dev),
            0.125)
    of1 = ops.gqa_decode(*args, want_f32=True, ws=ws)[1].cpu().numpy()
    of2 = ops.gqa_decode(*args, want_f32=True, ws=ws)[1].cpu().numpy()
    ref = do.gqa_attention(qo.bf16_to_f32(q), qo.bf16_to_f32(k), qo.bf16_to_f32(v), lens, 0.125)
    assert_close(of1, ref)
    assert np.array_equal(of1, of2)


@pytest.mark.parametrize("n_split", [1, 2, 3, 7, 33])
def test_gqa_decode_splits(dev, apath, n_split):
    rng = np.random.default_rng(17)
    L = 2100
    q = synth.random_bf16(rng, (2, 40, 64))
    k = synth.random_bf16(rng, (2, 8, L, 64))
    v = synth.random_bf16(rng, (2, 8, L, 64))
    lens = np.array([L, 777], np.int32)
    ws = ops.Workspace(8 << 20, device=dev)
    of = ops.gqa_decode(bf16_dev(q, dev), bf16_dev(k, dev), bf16_dev(v, dev),
                        torch.from_numpy(lens).to(dev), 0.125, n_split=n_split, want_f32=True,
                        ws=ws)[1]
    ref = do.gqa_attention(qo.bf16_to_f32(q), qo.bf16_to_f32(k), qo.bf16_to_f32(v), lens, 0.125)
    assert_close(of.cpu().numpy(), ref)
    # the split arrival counters are back at zero for the next call on this workspace
    assert not ws.buf[:ops.WS_COUNTER_BYTES].cpu().numpy().any()


def test_gqa_decode_split_edges_b8(dev, apath):
    """Batch 8 at a 2176-position cache (the decode step's attention: 3 splits of 728
    positions, two rounds each) with lengths at the edges of splits and rounds: an empty
    sequence (all zeros), one position, the last position of a round and of a split and the
    first past them, and a full cache."""
    rng = np.random.default_rng(23)
    B, hq, hkv, L = 8, 40, 8, 2176
    q = synth.random_bf16(rng, (B, hq, 64))
    k = synth.random_bf16(rng, (B, hkv, L, 64))
    v = synth.random_bf16(rng, (B, hkv, L, 64))
    lens = np.array([0, 1, 384, 385, 728, 729, 1500, 2176], np.int32)
    out, of = ops.gqa_decode(bf16_dev(q, dev), bf16_dev(k, dev), bf16_dev(v, dev),
                             torch.from_numpy(lens).to(dev), 0.125, want_f32=True)
    got = of.cpu().numpy()
    assert not got[0].any()
    ref = do.gqa_attention(qo.bf16_to_f32(q[1:]), qo.bf16_to_f32(k[1:]), qo.bf16_to_f32(v[1:]),
                           lens[1:], 0.125)
    assert_close(got[1:], ref)
    assert_bf16_close(bits(out)[1:], ref)


def test_gqa_decode_length_past_cache(dev, apath):
    """A length beyond the cache reads the whole cache and no further: the same bits as the
    length equal to max_len, at every split count."""
    rng = np.random.default_rng(31)
    L = 640
    q = bf16_dev(synth.random_bf16(rng, (2, 40, 64)), dev)
    k = bf16_dev(synth.random_bf16(rng, (2, 8, L, 64)), dev)
    v = bf16_dev(synth.random_bf16(rng, (2, 8, L, 64)), dev)
    for n_split in (0, 1, 3):
        outs = [ops.gqa_decode(q, k, v, torch.tensor(lens, dtype=torch.int32, device=dev), 0.125,
                               n_split=n_split, want_f32=True)[1].cpu().numpy()
                for lens in ([L, L], [L + 1, 1 << 20])]
        assert np.array_equal(outs[0], outs[1])


def test_gqa_decode_garbage_past_length(dev, apath):
    """Cache rows at and past a sequence's length take no part in the result whatever they
    hold: K = +Inf and V = NaN bit patterns there leave the output equal to the oracle's on
    the clean cache (a masked position contributes p = 0, and 0 * NaN would be NaN)."""
    rng = np.random.default_rng(20)
    L = 700
    q = synth.random_bf16(rng, (2, 40, 64))
    k = synth.random_bf16(rng, (2, 8, L, 64))
    v = synth.random_bf16(rng, (2, 8, L, 64))
    lens = np.array([333, 1], np.int32)
    kg, vg = k.copy(), v.copy()
    for b, n in enumerate(lens):
        kg[b, :, n:] = 0x7F80
        vg[b, :, n:] = 0x7FC1
    for n_split in (0, 1, 3):
        of = ops.gqa_decode(bf16_dev(q, dev), bf16_dev(kg, dev), bf16_dev(vg, dev),
                            torch.from_numpy(lens).to(dev), 0.125, n_split=n_split,
                            want_f32=True)[1]
        ref = do.gqa_attention(qo.bf16_to_f32(q), qo.bf16_to_f32(k), qo.bf16_to_f32(v), lens,
                               0.125)
        assert_close(of.cpu().numpy(), ref)


# ------------------------------------------------------------------ helpers

def ssq16(y):
    """float64 sums of squares over consecutive 16 entries of each row."""
    y = np.asarray(y, np.float64)
    return (y.reshape(y.shape[0], -1, 16) ** 2).sum(-1)


@pytest.mark.parametrize("kind", ["q8", "q4", "bf16"])
def test_embed_and_argmax(dev, kind):
    """Embedding rows from q8 / q4 tiles (a tied lm_head, dequantised exactly as the oracle
    does) or a stored bf16 matrix, with their per-16 sums of squares; a token out of range
    gives a NaN row; the device argmax takes the first maximum."""
    rng = np.random.default_rng(18)
    vocab, hid = 1024, 512
    toks = np.array([0, 31, 32, 1023, 1024], np.int32)
    if kind == "bf16":
        table = synth.random_bf16(rng, (vocab, hid))
        tdev = bf16_dev(table, dev)
        want = qo.bf16_to_f32(table[toks[:4]])
    else:
        tiles = (synth.q8_tiles if kind == "q8" else synth.q4_tiles)(rng, vocab, hid)
        tiles = tiles.reshape(-1, tiles.shape[-1])
        tdev = torch.from_numpy(tiles.reshape(-1)).to(dev)
        want = do.embed_rows(tiles, toks[:4], vocab, hid, kind)
    ss = torch.empty((5, hid // 16), dtype=torch.float32, device=dev)
    h = ops.embed(tdev, kind, torch.from_numpy(toks).to(dev), vocab, hid, ssq_out=ss).cpu().numpy()
    assert np.array_equal(h[:4], want)
    assert np.isnan(h[4]).all()
    assert_close(ss.cpu().numpy()[:4], ssq16(h[:4]), rel=1e-6)
    logits = rng.standard_normal((3, 100352)).astype(np.float32)
    logits[1, 5000] = logits[1, 7000] = 99.0         # first maximum wins
    idx = ops.argmax(torch.from_numpy(logits).to(dev)).cpu().numpy()
    assert idx.tolist() == np.argmax(logits, axis=1).tolist()


@pytest.mark.parametrize("batch", [1, 3, 5, 8, 17, 40])
def test_decode_advance_against_numpy(dev, batch):
    """decode_advance over random keys at batch sizes that give every arrangement of its
    reduction (16, 5, 3, 2 and 1 waves per row, and rows taken in several rounds): the token of
    each row's largest key, positions and lengths advanced, history written at the step, the
    step counter advanced; a row whose largest key appears twice yields that key's token."""
    rng = np.random.default_rng(31 + batch)
    n_slots = 6272
    # keys as the lm_head epilogue writes them: an order-preserving value above, 2^32 - 1 minus
    # the row below (slot i holds the best of rows 16 i .. 16 i + 15)
    rows = np.arange(n_slots, dtype=np.int64) * 16 + rng.integers(0, 16, (batch, n_slots))
    hi = rng.integers(0, 1 << 30, (batch, n_slots), dtype=np.int64)
    hi[0, 100] = hi[0, 5000] = (1 << 30) + 7             # one value at two rows: the first wins
    keys = (hi << 32) | (0xffffffff - rows)
    pos0 = rng.integers(0, 4000, batch).astype(np.int32)
    i32 = lambda a: torch.from_numpy(np.asarray(a, dtype=np.int32)).to(dev)
    tok, pos, lens, step = i32(np.zeros(batch)), i32(pos0), i32(np.zeros(batch)), i32([2])
    hist = torch.full((4, batch), -1, dtype=torch.int32, device=dev)
    ops.decode_advance(torch.from_numpy(keys).to(dev), n_slots, tok, pos, lens, step, hist)
    expect = rows[np.arange(batch), np.argmax(keys, axis=1)]
    assert int(expect[0]) == int(rows[0, 100])
    assert tok.cpu().numpy().tolist() == expect.tolist()
    assert pos.cpu().numpy().tolist() == (pos0 + 1).tolist()
    assert lens.cpu().numpy().tolist() == (pos0 + 2).tolist()
    h = hist.cpu().numpy()
    assert h[2].tolist() == expect.tolist() and (h[[0, 1, 3]] == -1).all()
    assert int(step.cpu()) == 3


@pytest.mark.parametrize("kind,batch", [("q8", 1), ("q4", 3), ("bf16", 2), ("q8", 8), ("q4", 64)])
def test_decode_advance_embed_equals_advance_then_embed(dev, kind, batch):
    """The fused greedy-loop launch (argmax keys -> token, positions, history, then the token's
    embedding row and its sums of squares) writes exactly what decode_advance followed by
    embed writes, including a NaN row for a token past the vocabulary."""
    rng = np.random.default_rng(19 + batch)
    vocab, hid = 1024, 512
    if kind == "bf16":
        table = synth.random_bf16(rng, (vocab, hid))
        tdev = bf16_dev(table, dev)
    else:
        tiles = (synth.q8_tiles if kind == "q8" else synth.q4_tiles)(rng, vocab, hid)
        tdev = torch.from_numpy(tiles.reshape(-1)).to(dev)
    n_slots = vocab // 16 + (1 if batch == 3 else 0)   # batch 3: one extra slot, a token past V
    keys = torch.from_numpy(rng.integers(0, 1 << 62, (batch, n_slots)).astype(np.int64)).to(dev)
    if batch == 3:
        keys[2, -1] = (1 << 63) - 1 - 2000   # the largest key of row 2: token 2000 >= vocab

    def state():
        i32 = lambda a: torch.tensor(a, dtype=torch.int32, device=dev)
        return dict(tokens=i32([0] * batch), pos=i32(list(range(5, 5 + batch))),
                    lens=i32([0] * batch), step=i32([1]),
                    history=torch.full((4, batch), -1, dtype=torch.int32, device=dev),
                    h=torch.zeros((batch, hid), dtype=torch.float32, device=dev),
                    ss=torch.zeros((batch, hid // 16), dtype=torch.float32, device=dev))

    a, f = state(), state()
    ops.decode_advance(keys, n_slots, a["tokens"], a["pos"], a["lens"], a["step"], a["history"])
    ops.embed(tdev, kind, a["tokens"], vocab, hid, out=a["h"], ssq_out=a["ss"])
    ops.decode_advance_embed(keys, n_slots, f["tokens"], f["pos"], f["lens"], f["step"],
                             f["history"], tdev, kind, vocab, hid, f["h"], f["ss"])
    torch.cuda.synchronize()
    for name in a:
        x, y = a[name].cpu().numpy(), f[name].cpu().numpy()
        assert np.array_equal(x.view(np.uint32) if x.dtype == np.float32 else x,
                              y.view(np.uint32) if y.dtype == np.float32 else y), name
    if batch == 3:
        assert int(f["tokens"][2]) == 2000 and np.isnan(f["h"][2].cpu().numpy()).all()


@pytest.mark.parametrize("hq,hkv,L,lmax,n_split,n_out", [
    (40, 8, 2112, 2176, 9, 2560),    # the 3B decode shape at the policy's split count (8 waves)
    (40, 8, 2112, 2176, 3, 2560),    # splits of 728 positions: two rounds of 12 waves
    (40, 8, 2112, 2176, 17, 2560),   # the same with 17 splits (4 waves)
    (40, 8, 2112, 2176, 18, 2560),   # the most splits the merge holds
    (40, 8, 300, 320, 1, 512),       # one split still publishes a record
    (32, 8, 1000, 1024, 5, 512),
    (8, 8, 40, 64, 18, 256),         # splits past the length: records with m = -inf, l = 0
    (16, 2, 0, 64, 3, 512),          # empty sequence: zeros into the projection
    (4, 1, 700, 768, 7, 256),        # one K-tile, four heads sharing one kv head
    (40, 40, 500, 512, 2, 512)])     # no grouping
def test_attn_records_o_proj_equals_chain(dev, apath, hq, hkv, L, lmax, n_split, n_out):
    """Attention publishing split records, then the o-projection merging them in its prologue,
    gives bit for bit what attention with its own merge followed by the o-projection GEMV
    gives (y and the per-16-row sums of squares); the records merge to the oracle's
    attention output."""
    rng = np.random.default_rng(hq * 1000 + L + n_split)
    q = synth.random_bf16(rng, (1, hq, 64))
    k = synth.random_bf16(rng, (1, hkv, lmax, 64))
    v = synth.random_bf16(rng, (1, hkv, lmax, 64))
    wo = synth.q4_tiles(rng, n_out, hq * 64).reshape(-1)
    h0 = (rng.standard_normal((1, n_out)) * 3).astype(np.float32)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    qd, kd, vd, W = bf16_dev(q, dev), bf16_dev(k, dev), bf16_dev(v, dev), d(wo)
    lens = torch.tensor([L], dtype=torch.int32, device=dev)
    ws = ops.Workspace(1 << 20, device=dev)
    nt = n_out // 32

    attn, af = ops.gqa_decode(qd, kd, vd, lens, 0.125, n_split=n_split, want_f32=True, ws=ws)
    h_c = d(h0)
    ss_c = torch.zeros((1, 2 * nt), dtype=torch.float32, device=dev)
    ops.gemv_ex(W, "q4", attn.view(1, hq * 64), nt, hq // 4, residual=h_c, out=h_c,
                ssq_out=ss_c, ws=ws)

    rec = ops.gqa_decode_records(qd, kd, vd, lens, n_split, 0.125, ws=ws)
    assert rec.shape == (1, hkv, n_split, hq // hkv, 68)
    h_f = d(h0)
    ss_f = torch.zeros((1, 2 * nt), dtype=torch.float32, device=dev)
    ops.gemv_attn_q4(W, nt, rec, residual=h_f, out=h_f, ssq_out=ss_f)
    torch.cuda.synchronize()
    assert np.array_equal(h_f.cpu().numpy().view(np.uint32), h_c.cpu().numpy().view(np.uint32))
    assert np.array_equal(ss_f.cpu().numpy().view(np.uint32), ss_c.cpu().numpy().view(np.uint32))
    # the records themselves hold the attention: merged on the host in float64
    r = rec.cpu().numpy().astype(np.float64)[0]             # [hkv][split][g][68]
    m, l_, acc = r[..., 64], r[..., 65], r[..., :64]
    mx = m.max(axis=1, keepdims=True)
    f = np.where(np.isfinite(m), np.exp2(m - np.where(np.isfinite(mx), mx, 0.0)), 0.0)
    lt = (l_ * f).sum(axis=1)
    at = (acc * f[..., None]).sum(axis=1)
    o = np.where(lt[..., None] > 0, at / np.where(lt > 0, lt, 1.0)[..., None], 0.0)
    o = o.reshape(1, hq, 64)
    if L == 0:
        assert not o.any() and not af.cpu().numpy().any()
    else:
        ref = do.gqa_attention(qo.bf16_to_f32(q), qo.bf16_to_f32(k), qo.bf16_to_f32(v),
                               np.array([L], np.int32), 0.125)
        assert_close(o, ref)
    # and the projection of the attention row is the oracle's GEMV of it
    ref_y = h0 + qo.gemv(wo.reshape(-1, 5120), "q4", bits(attn).reshape(1, -1), nt, hq // 4,
                         acc=np.float64).reshape(1, n_out)
    assert_close(h_f.cpu().numpy(), ref_y)


def test_attn_records_o_proj_rejects(dev):
    """Shapes the fused o-projection does not hold are refused before any launch."""
    rng = np.random.default_rng(7)
    W = torch.from_numpy(synth.q4_tiles(rng, 256, 44 * 64).reshape(-1)).to(dev)
    rec = torch.zeros((1, 4, 3, 11, 68), dtype=torch.float32, device=dev)
    with pytest.raises(Q4NXError, match="query heads"):
        ops.gemv_attn_q4(W, 8, rec)               # 44 heads: the row needs 11 K-tiles
    W = torch.from_numpy(synth.q4_tiles(rng, 256, 40 * 64).reshape(-1)).to(dev)
    rec = torch.zeros((1, 8, 19, 5, 68), dtype=torch.float32, device=dev)
    with pytest.raises(Q4NXError, match="n_split"):
        ops.gemv_attn_q4(W, 8, rec)               # 19 splits: more than the merge holds


@pytest.mark.parametrize("case", range(8))
def test_gqa_decode_random_shapes(dev, apath, case):
    """Seeded random batches, head groupings, cache lengths, ragged lengths (including empty
    and single-position sequences) and split counts, against the float64 oracle."""
    rng = np.random.default_rng(500 + case)
    batch = int(rng.integers(1, 13))
    hkv = int(rng.choice([1, 2, 4, 8]))
    hq = hkv * int(rng.integers(1, 9))
    lmax = int(rng.integers(1, 3000))
    lens = rng.integers(0, lmax + 1, batch).astype(np.int32)
    lens[0] = min(lmax, 1 if case % 2 else lmax)
    if batch > 1 and case % 3 == 0:
        lens[-1] = 0
    n_split = int(rng.choice([0, 0, 1, 3, 40]))
    q = synth.random_bf16(rng, (batch, hq, 64))
    k = synth.random_bf16(rng, (batch, hkv, lmax, 64))
    v = synth.random_bf16(rng, (batch, hkv, lmax, 64))
    of = ops.gqa_decode(bf16_dev(q, dev), bf16_dev(k, dev), bf16_dev(v, dev),
                        torch.from_numpy(lens).to(dev), 0.125, n_split=n_split,
                        want_f32=True)[1].cpu().numpy()
    ref = do.gqa_attention(qo.bf16_to_f32(q), qo.bf16_to_f32(k), qo.bf16_to_f32(v),
                           np.maximum(lens, 1), 0.125)   # empty rows are checked apart
    empty = lens == 0
    assert not of[empty].any()                           # no positions: zeros
    if (~empty).any():
        assert_close(of[~empty], ref[~empty])
