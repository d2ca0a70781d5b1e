"""The drop-in host surface on the GPU, used the way the reference's callers use it:
`NpuDesign` upload / run / download (reference/npu.py:41-114, designs/lm_head/lm_head.py's
`run_one`), `NpuLmHead.forward` for a decode row and a prefill block (npu.py:117-150), and
`attach_lm_head` on a model object with a `.q4nx` file (npu.py:153-163, chat.py:36-42).

Bar: fp32 logits within max|Δ|/max|ref| < 1e-5 of the float64 oracle, cosine > 0.9999999
(the reference's own gate, designs/lm_head/lm_head.py:191-196 via granite_gemv.py:335).
"""

import types

import numpy as np
import pytest
import torch

from llmnputest_amd import npu, q4nx, synth
from oracle import q4nx_oracle as qo

pytestmark = pytest.mark.gpu

REL = 1e-5
COS = 0.9999999
N, K = 4096, 1024      # a reduced lm_head: 128 tile-rows x 4 K-tiles of q8


def _meta():
    return {"name": "lm_head", "kind": "q8", "n_rows": N, "k": K}


def _rows_close(y, ref):
    for i in range(ref.shape[0]):
        rel, cos = qo.metrics(y[i], ref[i])
        assert rel < REL and cos > COS, (i, rel, cos)


def test_design_upload_run_download(dev):
    rng = np.random.default_rng(90)
    raw = synth.q8_tiles(rng, N, K).reshape(-1, 8704)
    x = synth.random_bf16(rng, K)
    d = npu.NpuDesign("lm_head", meta=_meta())
    d.upload(0, raw.reshape(-1))
    d.upload(1, x)                      # bf16 bits, as lm_head.py uploads ml_dtypes bf16
    d.run()
    y = d.download(2, np.float32, N)
    ref = qo.gemv(raw, "q8", x, N // 32, K // 256, acc=np.float64)
    _rows_close(y.reshape(1, N), ref.reshape(1, N))
    d.close()


@pytest.mark.parametrize("shape", [(1, 1), (1, 37), (3, 50)])
def test_lm_head_decode_and_prefill(dev, shape):
    """[batch, seq, hidden] activations as transformers hands them to lm_head: one row is
    decode, more rows are prefill -- both on the GPU, in the activations' dtype."""
    rng = np.random.default_rng(91)
    raw = synth.q8_tiles(rng, N, K).reshape(-1, 8704)
    fallback = torch.nn.Linear(K, N, bias=False)
    head = npu.NpuLmHead(fallback, meta=_meta())
    head.load_weights(raw.tobytes())
    hb = synth.random_bf16(rng, (*shape, K))
    h = torch.from_numpy(hb.view(np.int16)).view(torch.bfloat16)          # on the host
    out = head(h)
    assert out.shape == (*shape, N) and out.dtype == torch.bfloat16 and out.device == h.device
    ref = qo.gemv(raw, "q8", hb.reshape(-1, K), N // 32, K // 256, acc=np.float64)
    got = out.float().numpy().reshape(-1, N)
    # the module returns h's dtype (bf16): compare at the bf16 rounding of the oracle
    want = qo.bf16_to_f32(qo.bf16_round(ref.astype(np.float32)))
    diff = np.abs(got - want)
    assert (diff <= np.abs(want) * 2.0 ** -7 + REL * np.abs(ref).max()).all()
    rows = shape[0] * shape[1]
    assert head.npu_calls == 1 and head.cpu_calls == 0
    assert head.prefill_calls == (1 if rows > 1 else 0)
    assert head.design.calls == 1 and head.design.seconds > 0


def test_attach_lm_head(dev, tmp_path):
    rng = np.random.default_rng(92)
    w8 = synth.q8_tiles(rng, N, K)
    path = tmp_path / "model.q4nx"
    q4nx.write_q4nx(path, {"lm_head.weight": ("q8", w8)})
    model = types.SimpleNamespace(lm_head=torch.nn.Linear(K, N, bias=False))
    head = npu.attach_lm_head(model, q4nx.Q4NX(path))
    assert model.lm_head is head and isinstance(head, npu.NpuLmHead)
    h = torch.from_numpy(synth.random_bf16(rng, (2, K)).view(np.int16)).view(torch.bfloat16)
    y = head(h.float())
    ref = qo.gemv(w8.reshape(-1, 8704), "q8", h.view(torch.int16).numpy().view(np.uint16),
                  N // 32, K // 256, acc=np.float64)
    _rows_close(y.numpy(), ref)


@pytest.mark.parametrize("kind,n,k", [("q4", 16, 200), ("q8", 40, 300), ("q4", 100, 2560)])
def test_padded_tensor_trim_and_gemv(dev, tmp_path, kind, n, k):
    """A tensor whose N or K is not a tile multiple, stored padded to whole tiles: `tensor`
    with the logical shape returns exactly the oracle's dequantised matrix with the padding
    trimmed (tools/q4nx.py:176-197), and `gemv_trimmed` gives W @ x of the trimmed matrix."""
    from llmnputest_amd import ops
    rng = np.random.default_rng(n + k)
    n_t, k_t = q4nx.padded_shape(n, k)
    t = synth.q4_tiles(rng, n_t * 32, k_t * 256) if kind == "q4" else synth.q8_tiles(rng, n_t * 32, k_t * 256)
    path = tmp_path / "pad.q4nx"
    q4nx.write_q4nx(path, {"w.weight": (kind, t)})
    f = q4nx.Q4NX(path)
    full = qo.dequant_matrix(t.reshape(-1), kind, n_t, k_t)
    got32 = f.tensor("w.weight", (n, k), device=dev, dtype=torch.float32)
    assert got32.shape == (n, k)
    assert np.array_equal(got32.cpu().numpy(), full[:n, :k])
    got16 = f.tensor("w.weight", (n, k), device=dev)
    want16 = qo.bf16_round(full[:n, :k])
    assert np.array_equal(got16.contiguous().view(torch.int16).cpu().numpy().view(np.uint16), want16)
    with pytest.raises(q4nx.Q4NXFormatError):
        f.tensor("w.weight", (n + 32, k), device=dev)
    x = synth.random_bf16(rng, (3, k))
    y = ops.gemv_trimmed(torch.from_numpy(t.reshape(-1)).to(dev), kind,
                         torch.from_numpy(x.view(np.int16)).to(dev).view(torch.bfloat16), n, k)
    assert y.shape == (3, n)
    ref = full[:n, :k].astype(np.float64) @ qo.bf16_to_f32(x).astype(np.float64).T
    rel, cos = qo.metrics(y.cpu().numpy(), ref.T)
    assert rel < 1e-5 and cos > 0.9999999, (rel, cos)
