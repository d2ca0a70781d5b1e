"""The GEMV and fused entry points on their matrix-core path (policy mfma_rows): RMSNorm
prologue from the producer's sums of squares, the plain epilogue (residual, sums of squares,
argmax keys), [gate, up, SwiGLU] and [q, k, v, RoPE + cache append], for batches inside and
beyond the VALU kernel's 8 rows.

Bars as in test_gpu_ops: fp32 pre-epilogue values within max|Δ|/max|ref| < 1e-5 of the
float64 oracle on a bf16 input; bf16 epilogue outputs equal the oracle's rounding of the
kernel's own fp32 values up to rare 1-ulp flips. With the RMSNorm prologue the fused ops are
teacher-forced on the prologue's own bf16 output (checked against the float64 norm first);
gemv_ex, which has no such output, is held to the 1e-5 bar plus, per output, the exact effect
of one-ulp flips of the normalised entries that sit on a bf16 rounding midpoint.
"""

import numpy as np
import pytest
import torch

from llmnputest_amd import ops, synth
from oracle import decode_oracle as do
from oracle import q4nx_oracle as qo

pytestmark = pytest.mark.gpu

REL = 1e-5
COS = 0.9999999


def bf16_dev(b, dev):
    return torch.from_numpy(np.ascontiguousarray(b, dtype=np.uint16).view(np.int16)).to(dev).view(torch.bfloat16)


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def rows_close(got, ref, rel, cos):
    for i in range(ref.shape[0]):
        r, c = qo.metrics(got[i], ref[i])
        assert r < rel and c > cos, (i, r, c)


def assert_bf16_close(got_bits, ref_f64, max_frac=1e-3):
    want = qo.bf16_round(np.asarray(ref_f64, np.float64).astype(np.float32))
    diff = np.abs(np.asarray(got_bits, np.uint16).ravel().astype(np.int32) - want.ravel().astype(np.int32))
    assert diff.max() <= 1, int(diff.max())
    assert (diff > 0).mean() <= max_frac, float((diff > 0).mean())


def ssq16(y):
    y = np.asarray(y, np.float64)
    return (y.reshape(y.shape[0], -1, 16) ** 2).sum(-1)


def normed_input(rng, batch, k, dev, scale=20.0):
    """fp32 residual rows, their per-16 sums of squares, bf16 norm weights, and the oracle's
    normalised input (float64, before the bf16 rounding)."""
    h = (rng.standard_normal((batch, k)) * scale).astype(np.float32)
    nw = synth.f32_to_bf16_bits(1.0 + 0.1 * rng.standard_normal(k).astype(np.float32))
    return (torch.from_numpy(h).to(dev), torch.from_numpy(ssq16(h).astype(np.float32)).to(dev),
            bf16_dev(nw, dev), do.rmsnorm(h, nw, 1e-5))


def ambiguous_ulps(x64, margin=1e-6):
    """Per entry: one bf16 ulp where the float64 value lies within `margin` (relative) of a
    bf16 rounding midpoint -- the kernel's fp32 arithmetic may round it either way -- else 0."""
    x32 = np.abs(x64).astype(np.float32)
    lo = (x32.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32).astype(np.float64)
    ulp = ((x32.view(np.uint32) & np.uint32(0x7F800000)).view(np.float32).astype(np.float64)
           * 2.0 ** -7)
    mid = lo + ulp / 2
    return np.where(np.abs(np.abs(x64) - mid) <= margin * np.abs(x64), ulp, 0.0)


def assert_close_norm(y, raw, kind, x64, n_t, k_t, res=0.0):
    """y against the oracle on the float64 norm rounded to bf16, allowing each row the effect
    of one-ulp flips of the normalised input where that input sits on a rounding midpoint."""
    xb = qo.bf16_round(x64.astype(np.float32))
    ref = qo.gemv(raw, kind, xb, n_t, k_t, acc=np.float64).reshape(y.shape) + res
    wabs = np.abs(qo.dequant_matrix(raw, kind, n_t, k_t).astype(np.float64))
    slack = ambiguous_ulps(x64) @ wabs.T            # [rows, N]
    for i in range(y.shape[0]):
        err = np.abs(y[i] - ref[i])
        assert (err <= REL * np.abs(ref[i]).max() + slack[i]).all(), \
            (i, float((err - slack[i]).max() / np.abs(ref[i]).max()))
        assert qo.metrics(y[i], ref[i])[1] > COS


@pytest.mark.parametrize("kind", ["q4", "q8"])
@pytest.mark.parametrize("batch", [1, 2, 12, 40])
def test_mfma_gemv_ex_norm_ssq_keys(dev, mfma, kind, batch):
    """Final-norm + lm_head shape of the decode step: RMSNorm prologue, residual, sums of
    squares and argmax keys, all on the matrix cores."""
    rng = np.random.default_rng(40 + batch)
    n, k = 2048, 2560
    t = synth.q4_tiles(rng, n, k) if kind == "q4" else synth.q8_tiles(rng, n, k)
    raw = t.reshape(-1, t.shape[-1])
    w = torch.from_numpy(raw.reshape(-1)).to(dev)
    hd, ss_in, nwd, x64 = normed_input(rng, batch, k, dev)
    res = rng.standard_normal((batch, n)).astype(np.float32)
    ss_out = torch.empty((batch, n // 16), dtype=torch.float32, device=dev)
    keys = torch.zeros((batch, n // 16), dtype=torch.int64, device=dev)
    y = ops.gemv_ex(w, kind, hd, n // 32, k // 256, norm_w=nwd, eps=1e-5,
                    residual=torch.from_numpy(res).to(dev), ssq_in=ss_in, ssq_out=ss_out,
                    argmax_keys=keys).cpu().numpy()
    assert_close_norm(y, raw, kind, x64, n // 32, k // 256, res)
    sref = ssq16(y)
    assert np.abs(ss_out.cpu().numpy() - sref).max() <= 1e-6 * sref.max()
    tok = torch.zeros(batch, dtype=torch.int32, device=dev)
    pos = torch.zeros(batch, dtype=torch.int32, device=dev)
    lens = torch.zeros(batch, dtype=torch.int32, device=dev)
    step = torch.zeros(1, dtype=torch.int32, device=dev)
    ops.decode_advance(keys, n // 16, tok, pos, lens, step)
    assert tok.cpu().numpy().tolist() == np.argmax(y, axis=1).tolist()


@pytest.mark.parametrize("case", range(6))
def test_gemv_ex_random_shapes_all_epilogues(dev, kpath, case):
    """Seeded random shapes with every epilogue of the plain GEMV at once (RMSNorm prologue
    from the producer's sums of squares, a residual added in place, the outputs' sums of
    squares and argmax keys) on each kernel family: tile-row counts that do not fill a grid,
    short and long K, batches up to 16 on the matrix cores (8 on the VALU kernels)."""
    rng = np.random.default_rng(3100 + 7 * case)
    kind = "q8" if case % 3 == 2 else "q4"
    n_t = int(rng.integers(1, 120))
    k_t = int(rng.choice([1, 2, 3, 5, 10, 13]))
    batch = int(rng.integers(1, 17 if kpath == "mfma" else 9))
    n, k = 32 * n_t, 256 * k_t
    t = synth.q4_tiles(rng, n, k) if kind == "q4" else synth.q8_tiles(rng, n, k)
    raw = t.reshape(-1, t.shape[-1])
    w = torch.from_numpy(raw.reshape(-1)).to(dev)
    hd, ss_in, nwd, x64 = normed_input(rng, batch, k, dev)
    res = rng.standard_normal((batch, n)).astype(np.float32)
    y = torch.from_numpy(res.copy()).to(dev)
    ss_out = torch.empty((batch, n // 16), dtype=torch.float32, device=dev)
    keys = torch.zeros((batch, n // 16), dtype=torch.int64, device=dev)
    ops.gemv_ex(w, kind, hd, n_t, k_t, norm_w=nwd, eps=1e-5, residual=y, out=y, ssq_in=ss_in,
                ssq_out=ss_out, argmax_keys=keys)
    got = y.cpu().numpy()
    assert_close_norm(got, raw, kind, x64, n_t, k_t, res)
    sref = ssq16(got)
    assert np.abs(ss_out.cpu().numpy() - sref).max() <= 1e-6 * sref.max()
    z = lambda: torch.zeros(batch, dtype=torch.int32, device=dev)
    tok = z()
    ops.decode_advance(keys, n // 16, tok, z(), z(), torch.zeros(1, dtype=torch.int32, device=dev))
    assert tok.cpu().numpy().tolist() == np.argmax(got, axis=1).tolist()


@pytest.mark.parametrize("batch", [1, 3, 11, 20])
def test_mfma_gemv_plain_keys_only(dev, mfma, batch):
    """argmax keys without an output vector (the decode step's lm_head form)."""
    rng = np.random.default_rng(50 + batch)
    n, k = 4096, 1024
    raw = synth.q8_tiles(rng, n, k).reshape(-1, 8704)
    x = synth.random_bf16(rng, (batch, k))
    keys = torch.zeros((batch, n // 16), dtype=torch.int64, device=dev)
    ops.gemv_ex(torch.from_numpy(raw.reshape(-1)).to(dev), "q8", bf16_dev(x, dev), n // 32,
                k // 256, argmax_keys=keys, want_y=False)
    ref = qo.gemv(raw, "q8", x, n // 32, k // 256, acc=np.float64).reshape(batch, n)
    tok = torch.zeros(batch, dtype=torch.int32, device=dev)
    z = lambda: torch.zeros(batch, dtype=torch.int32, device=dev)
    ops.decode_advance(keys, n // 16, tok, z(), z(), torch.zeros(1, dtype=torch.int32, device=dev))
    got = tok.cpu().numpy()
    for b in range(batch):
        top = np.sort(ref[b])[-2:]
        if top[1] - top[0] > REL * np.abs(ref[b]).max():
            assert got[b] == int(np.argmax(ref[b])), b


@pytest.mark.parametrize("batch,norm", [(2, False), (5, True), (9, False), (17, True)])
def test_mfma_qkv_rope(dev, mfma, batch, norm):
    rng = np.random.default_rng(60 + batch)
    hq, hkv, hid, lmax = 40, 8, 2560, 256
    kt = hid // 256
    wq = synth.q4_tiles(rng, hq * 64, hid).reshape(-1, 5120)
    wk = synth.q4_tiles(rng, hkv * 64, hid).reshape(-1, 5120)
    wv = synth.q4_tiles(rng, hkv * 64, hid).reshape(-1, 5120)
    pos = rng.integers(0, lmax, batch).astype(np.int32)
    tab_np = do.rope_table(lmax, 64, 10000.0)
    tab = ops.rope_table(lmax, 64, 10000.0)
    kc = torch.zeros((batch, hkv, lmax, 64), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    raw = torch.empty((batch, (hq + 2 * hkv) * 64), dtype=torch.float32, device=dev)
    xn = torch.zeros((batch, hid), dtype=torch.bfloat16, device=dev)
    if norm:
        x_dev, ss_in, nwd, x64 = normed_input(rng, batch, hid, dev)
    else:
        x_used = synth.random_bf16(rng, (batch, hid))
        x_dev, ss_in, nwd = bf16_dev(x_used, dev), None, None
    d = lambda a: torch.from_numpy(a.reshape(-1)).to(dev)
    q = ops.qkv_rope(d(wq), d(wk), d(wv), hq, hkv, kt, x_dev, torch.from_numpy(pos).to(dev), tab,
                     kc, vc, norm_w=nwd, raw_out=raw, ssq_in=ss_in,
                     xn_out=xn if norm else None)
    if norm:   # the prologue's own bf16 input, then the GEMV on it at the full bar
        assert_bf16_close(bits(xn), x64, max_frac=2e-3)
        x_used = bits(xn)
    raw_np = raw.cpu().numpy()
    ref = np.concatenate([qo.gemv(w_, "q4", x_used, n, kt, acc=np.float64).reshape(batch, -1)
                          for w_, n in ((wq, hq * 2), (wk, hkv * 2), (wv, hkv * 2))], axis=1)
    rows_close(raw_np, ref, REL, COS)
    qr, kr, vr = do.qkv_rope_from_raw(raw_np[:, :hq * 64], raw_np[:, hq * 64:(hq + hkv) * 64],
                                      raw_np[:, (hq + hkv) * 64:], pos, tab_np)
    assert_bf16_close(bits(q).reshape(batch, hq, 64), qr)
    kcn, vcn = bits(kc), bits(vc)
    for b in range(batch):
        assert_bf16_close(kcn[b, :, pos[b]], kr[b])
        assert np.array_equal(vcn[b, :, pos[b]], qo.bf16_round(vr[b].astype(np.float32)))
        mask = np.ones(lmax, bool)
        mask[pos[b]] = False
        assert not kcn[b][:, mask].any() and not vcn[b][:, mask].any()


@pytest.mark.parametrize("batch,norm", [(2, True), (4, False), (9, True), (33, False)])
def test_mfma_gate_up_swiglu(dev, mfma, batch, norm):
    rng = np.random.default_rng(70 + batch)
    hid, inter = 2560, 8192
    kt = hid // 256
    wg = synth.q4_tiles(rng, inter, hid).reshape(-1, 5120)
    wu = synth.q4_tiles(rng, inter, hid).reshape(-1, 5120)
    raw = torch.empty((batch, 2 * inter), dtype=torch.float32, device=dev)
    xn = torch.zeros((batch, hid), dtype=torch.bfloat16, device=dev)
    if norm:
        x_dev, ss_in, nwd, x64 = normed_input(rng, batch, hid, dev)
    else:
        x_used = synth.random_bf16(rng, (batch, hid))
        x_dev, ss_in, nwd = bf16_dev(x_used, dev), None, None
    d = lambda a: torch.from_numpy(a.reshape(-1)).to(dev)
    hout = ops.gate_up_swiglu(d(wg), d(wu), inter // 32, kt, x_dev, norm_w=nwd, raw_out=raw,
                              ssq_in=ss_in, xn_out=xn if norm else None)
    if norm:
        assert_bf16_close(bits(xn), x64, max_frac=2e-3)
        x_used = bits(xn)
    raw_np = raw.cpu().numpy()
    ref = np.concatenate([qo.gemv(wg, "q4", x_used, inter // 32, kt, acc=np.float64),
                          qo.gemv(wu, "q4", x_used, inter // 32, kt, acc=np.float64)],
                         axis=1).reshape(batch, -1)
    rows_close(raw_np, ref, REL, COS)
    assert_bf16_close(bits(hout), do.swiglu_from_raw(raw_np[:, :inter], raw_np[:, inter:]))


@pytest.mark.parametrize("parts", [1, 3])
def test_mfma_rowblock_split_fused(dev, parts):
    """The fused epilogues on row-block workgroups (two per group: 32 [gate, up] groups and
    12 [q, k, v] heads at 5 rows), whole and with K in 3 parts: gate/up accumulators and q/k/v
    (before RoPE) at the GEMV bar, SwiGLU and the rotated q to the oracle's rounding."""
    rng = np.random.default_rng(95 + parts)
    hid, inter, batch = 2560, 1024, 5
    kt = hid // 256
    pol = ops.Policy(gemm_ksplit=parts)
    d = lambda a: torch.from_numpy(a.reshape(-1)).to(dev)
    x = synth.random_bf16(rng, (batch, hid))
    wg = synth.q4_tiles(rng, inter, hid).reshape(-1, 5120)
    wu = synth.q4_tiles(rng, inter, hid).reshape(-1, 5120)
    raw = torch.empty((batch, 2 * inter), dtype=torch.float32, device=dev)
    hout = ops.gate_up_swiglu(d(wg), d(wu), inter // 32, kt, bf16_dev(x, dev), raw_out=raw,
                              policy=pol)
    raw_np = raw.cpu().numpy()
    ref = np.concatenate([qo.gemv(wg, "q4", x, inter // 32, kt, acc=np.float64),
                          qo.gemv(wu, "q4", x, inter // 32, kt, acc=np.float64)],
                         axis=1).reshape(batch, -1)
    rows_close(raw_np, ref, REL, COS)
    assert_bf16_close(bits(hout), do.swiglu_from_raw(raw_np[:, :inter], raw_np[:, inter:]))
    hq, hkv, lmax = 8, 2, 128
    wq = synth.q4_tiles(rng, hq * 64, hid).reshape(-1, 5120)
    wk = synth.q4_tiles(rng, hkv * 64, hid).reshape(-1, 5120)
    wv = synth.q4_tiles(rng, hkv * 64, hid).reshape(-1, 5120)
    pos = rng.integers(0, lmax, batch).astype(np.int32)
    kc = torch.zeros((batch, hkv, lmax, 64), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    rq = torch.empty((batch, (hq + 2 * hkv) * 64), dtype=torch.float32, device=dev)
    q = ops.qkv_rope(d(wq), d(wk), d(wv), hq, hkv, kt, bf16_dev(x, dev),
                     torch.from_numpy(pos).to(dev), ops.rope_table(lmax, 64, 10000.0), kc, vc,
                     raw_out=rq, policy=pol)
    rq_np = rq.cpu().numpy()
    ref = np.concatenate([qo.gemv(w_, "q4", x, n, kt, acc=np.float64).reshape(batch, -1)
                          for w_, n in ((wq, hq * 2), (wk, hkv * 2), (wv, hkv * 2))], axis=1)
    rows_close(rq_np, ref, REL, COS)
    qr, _, _ = do.qkv_rope_from_raw(rq_np[:, :hq * 64], rq_np[:, hq * 64:(hq + hkv) * 64],
                                    rq_np[:, (hq + hkv) * 64:], pos, do.rope_table(lmax, 64, 10000.0))
    assert_bf16_close(bits(q).reshape(batch, hq, 64), qr)


def test_mfma_and_valu_agree(dev):
    """The two kernel families on the same batch-3 inputs: both within the oracle's bar. (Their
    bf16 outputs are not compared with each other: where g is near zero, a 1e-6 absolute
    difference in the fp32 accumulators moves bf16(g) by several ulps.)"""
    rng = np.random.default_rng(80)
    hid, inter = 2560, 8192
    kt = hid // 256
    wg = synth.q4_tiles(rng, inter, hid).reshape(-1, 5120)
    wu = synth.q4_tiles(rng, inter, hid).reshape(-1, 5120)
    x = synth.random_bf16(rng, (3, hid))
    d = lambda a: torch.from_numpy(a.reshape(-1)).to(dev)
    outs = {}
    for path, rows in (("valu", 0), ("mfma", 1)):
        raw = torch.empty((3, 2 * inter), dtype=torch.float32, device=dev)
        h = ops.gate_up_swiglu(d(wg), d(wu), inter // 32, kt, bf16_dev(x, dev), raw_out=raw,
                               policy=ops.Policy(mfma_rows_q4=rows))
        outs[path] = (raw.cpu().numpy(), bits(h))
    ref = np.concatenate([qo.gemv(wg, "q4", x, inter // 32, kt, acc=np.float64),
                          qo.gemv(wu, "q4", x, inter // 32, kt, acc=np.float64)], axis=1)
    for path, (raw_np, hb) in outs.items():   # each path's epilogue on its own accumulators
        rows_close(raw_np, ref, REL, COS)
        assert_bf16_close(hb, do.swiglu_from_raw(raw_np[:, :inter], raw_np[:, inter:]))


def test_config3_mlp_batch8_default_policy(dev):
    """Config 3's MLP at batch 8 as the decode step runs it, under the library's default policy
    (8 rows go to the matrix cores): [RMSNorm from the producer's sums of squares, gate, up,
    SwiGLU] on 2560 -> 8192, then down 8192 -> 2560 with the residual added and the sums of
    squares of the result written. Each stage is held to its own bar on its own input (the
    reference checks the intermediate h separately, designs/granite_gemv/granite_mlp_full.py:
    231-254): the normalised input to bf16 rounding, gate/up fp32 accumulators and the down
    output at 1e-5 of the float64 oracle, h to the oracle's rounding of SwiGLU on the kernel's
    own accumulators."""
    rng = np.random.default_rng(88)
    batch, hid, inter = 8, 2560, 8192
    pol = ops.Policy()
    assert pol.mfma_rows_q4 <= batch
    wg = synth.q4_tiles(rng, inter, hid).reshape(-1, 5120)
    wu = synth.q4_tiles(rng, inter, hid).reshape(-1, 5120)
    wd = synth.q4_tiles(rng, hid, inter).reshape(-1, 5120)
    x_dev, ss_in, nwd, x64 = normed_input(rng, batch, hid, dev)
    d = lambda a: torch.from_numpy(a.reshape(-1)).to(dev)
    raw = torch.empty((batch, 2 * inter), dtype=torch.float32, device=dev)
    xn = torch.zeros((batch, hid), dtype=torch.bfloat16, device=dev)
    hb = ops.gate_up_swiglu(d(wg), d(wu), inter // 32, hid // 256, x_dev, norm_w=nwd,
                            raw_out=raw, ssq_in=ss_in, xn_out=xn, policy=pol)
    y = torch.empty((batch, hid), dtype=torch.float32, device=dev)
    ss_out = torch.empty((batch, hid // 16), dtype=torch.float32, device=dev)
    ops.gemv_ex(d(wd), "q4", hb, hid // 32, inter // 256, residual=x_dev, out=y, ssq_out=ss_out,
                policy=pol)
    torch.cuda.synchronize()
    assert_bf16_close(bits(xn), x64, max_frac=2e-3)
    x_used = bits(xn)
    raw_np = raw.cpu().numpy()
    ref = np.concatenate([qo.gemv(wg, "q4", x_used, inter // 32, hid // 256, acc=np.float64),
                          qo.gemv(wu, "q4", x_used, inter // 32, hid // 256, acc=np.float64)],
                         axis=1).reshape(batch, -1)
    rows_close(raw_np, ref, REL, COS)
    h_bits = bits(hb)
    assert_bf16_close(h_bits, do.swiglu_from_raw(raw_np[:, :inter], raw_np[:, inter:]))
    ref_y = (x_dev.cpu().numpy().astype(np.float64)
             + qo.gemv(wd, "q4", h_bits, hid // 32, inter // 256, acc=np.float64).reshape(batch, -1))
    y_np = y.cpu().numpy()
    rows_close(y_np, ref_y, REL, COS)
    rows_close(ss_out.cpu().numpy(), ssq16(y_np), REL, COS)
