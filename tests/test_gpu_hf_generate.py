"""The GPU lm_head inside transformers' `generate`, the way chat.py uses the reference's NPU
one (chat.py:36-42, 80-84): a Qwen3 causal LM (tied embeddings, random weights -- no model
files are available offline), its lm_head written to a .q4nx file as q8 tiles, swapped in
with `attach_lm_head`, then greedy generation with the rest of the model in torch on the CPU.

Check: every call of the head (the prompt block, then one row per step) equals the float64
oracle of the same head on the hidden states it received (bf16-rounded, dequantised q8
weights) to max|Δ|/max|ref| < 1e-5, generate takes the head's argmax, and that is the
oracle's argmax unless its top two logits are within the tolerance.
"""

import numpy as np
import pytest
import torch

from llmnputest_amd import npu, q4nx, synth
from oracle import q4nx_oracle as qo

pytestmark = pytest.mark.gpu

REL = 1e-5


def tiny_qwen3():
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen3Config(vocab_size=4096, hidden_size=512, intermediate_size=1024,
                                   num_hidden_layers=2, num_attention_heads=8,
                                   num_key_value_heads=4, head_dim=64,
                                   tie_word_embeddings=True, max_position_embeddings=256)
    torch.manual_seed(0)
    return transformers.Qwen3ForCausalLM(cfg).eval()


def test_generate_with_gpu_lm_head(dev, tmp_path):
    model = tiny_qwen3()
    w = model.lm_head.weight.detach().float().numpy()
    tiles = synth.quantize_q8(w)
    path = tmp_path / "model.q4nx"
    q4nx.write_q4nx(path, {"lm_head.weight": ("q8", tiles)})
    head = npu.attach_lm_head(model, q4nx.Q4NX(path))
    assert model.lm_head is head

    calls = []
    head.register_forward_hook(lambda mod, args, out: calls.append((args[0].detach().clone(),
                                                                    out.detach().clone())))
    prompt = torch.from_numpy(np.random.default_rng(1).integers(0, 4096, (1, 12)))
    with torch.no_grad():
        seq = model.generate(prompt, max_new_tokens=16, do_sample=False, pad_token_id=0)[0]
    assert seq.shape[0] == 12 + 16
    assert len(calls) == 16 and head.npu_calls == 16 and head.cpu_calls == 0

    # each call against the float64 oracle of the head on exactly the hidden states it got
    wd = qo.dequant_matrix(tiles.reshape(-1, 8704), "q8", 4096 // 32, 512 // 256).astype(np.float64)
    for i, (h, logits) in enumerate(calls):
        hb = qo.bf16_round(h.reshape(-1, 512).float().numpy())
        ref = qo.bf16_to_f32(hb).astype(np.float64) @ wd.T
        got = logits.reshape(-1, 4096).float().numpy()
        for r in range(ref.shape[0]):
            rel, cos = qo.metrics(got[r], ref[r])
            assert rel < REL and cos > 0.9999999, (i, r, rel, cos)
        last = ref[-1]
        assert int(seq[12 + i]) == int(np.argmax(got[-1]))     # generate took the head's argmax
        top = np.sort(last)[-2:]
        if top[1] - top[0] > REL * np.abs(last).max():
            assert int(seq[12 + i]) == int(np.argmax(last)), i


def test_generate_qwen35_head_real_shape(dev, tmp_path):
    """The reference's chat model class (Qwen3_5ForCausalLM, reference/from_q4nx.py:140-171)
    at its real head shape, 248320 x 1024 q8 with tied embeddings (random weights, two
    layers: a gated delta-net and a full-attention one), through `chat.tiny_qwen35`, the model
    `chat --hf-tiny` drives. Each head call (the 8-row prompt block, then one row per step)
    is checked against the float64 oracle on the hidden states it received, and generate
    takes the head's argmax."""
    pytest.importorskip("transformers")
    from llmnputest_amd import chat
    from oracle import cpu_oracle

    n, k = 248320, 1024
    model = chat.tiny_qwen35(seed=3, n_layers=2)
    assert model.lm_head.weight.shape == (n, k)
    assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()
    tiles = synth.quantize_q8(model.lm_head.weight.detach().float().numpy())
    path = tmp_path / "model.q4nx"
    q4nx.write_q4nx(path, {"lm_head.weight": ("q8", tiles)})
    head = npu.attach_lm_head(model, q4nx.Q4NX(path))
    assert model.lm_head is head and head.n_rows == n and head.k == k

    calls = []
    head.register_forward_hook(lambda mod, args, out: calls.append((args[0].detach().clone(),
                                                                    out.detach().clone())))
    prompt = torch.from_numpy(np.random.default_rng(4).integers(0, n, (1, 8)))
    new = 6
    with torch.no_grad():
        seq = model.generate(prompt, max_new_tokens=new, do_sample=False, pad_token_id=0)[0]
    assert seq.shape[0] == 8 + new
    assert len(calls) == new and head.npu_calls == new and head.cpu_calls == 0

    raw = tiles.reshape(-1)
    for i, (h, logits) in enumerate(calls):
        hb = qo.bf16_round(h.reshape(-1, k).float().numpy())
        ref = cpu_oracle.gemv(raw, "q8", hb, n // 32, k // 256)
        got = logits.reshape(-1, n).float().numpy()
        assert got.shape == ref.shape
        for r in range(ref.shape[0]):
            rel, cos = qo.metrics(got[r], ref[r])
            assert rel < REL and cos > 0.9999999, (i, r, rel, cos)
        last = ref[-1]
        assert int(seq[8 + i]) == int(np.argmax(got[-1]))
        top = np.sort(last)[-2:]
        if top[1] - top[0] > REL * np.abs(last).max():
            assert int(seq[8 + i]) == int(np.argmax(last)), i
