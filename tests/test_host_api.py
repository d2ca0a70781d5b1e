"""Host logic of the drop-in surface: the q4nx container reader, projection shapes and the
stored-shape cross-check (tools/q4nx.py, designs/granite_gemv/granite_gemv.py:90-102,
282-288), and the design metadata of the GPU NpuDesign (reference/npu.py:41-114)."""

import numpy as np
import pytest

from llmnputest_amd import npu, q4nx, synth

GRANITE = {"hidden_size": 2560, "intermediate_size": 8192, "num_attention_heads": 40,
           "num_key_value_heads": 8, "head_dim": 64, "vocab_size": 100352}


def test_container_roundtrip(tmp_path):
    rng = np.random.default_rng(0)
    w4 = synth.q4_tiles(rng, 64, 512)
    w8 = synth.q8_tiles(rng, 64, 256)
    norm = synth.random_bf16(rng, 512)
    path = tmp_path / "m.q4nx"
    q4nx.write_q4nx(path, {"a.weight": ("q4", w4), "lm_head.weight": ("q8", w8),
                           "model.norm.weight": norm})
    f = q4nx.Q4NX(path)
    assert f.names() == ["a.weight", "lm_head.weight", "model.norm.weight"]
    kind, t = f.tiles("a.weight")
    assert kind == "q4" and np.array_equal(t, w4.reshape(-1, 5120))
    kind, t = f.tiles("lm_head.weight")
    assert kind == "q8" and np.array_equal(t, w8.reshape(-1, 8704))
    assert np.array_equal(f.plain("model.norm.weight"), norm)
    assert f.raw("a.weight") == w4.tobytes()
    with pytest.raises(q4nx.Q4NXFormatError):
        f.tiles("model.norm.weight")


def test_projection_shapes_and_factoring():
    assert q4nx.projection_shape("model.layers.0.mlp.gate_proj.weight", GRANITE) == (8192, 2560)
    assert q4nx.projection_shape("model.layers.3.mlp.down_proj.weight", GRANITE) == (2560, 8192)
    assert q4nx.projection_shape("model.layers.0.self_attn.k_proj.weight", GRANITE) == (512, 2560)
    assert q4nx.projection_shape("lm_head.weight", GRANITE) == (100352, 2560)
    # gate and down are both stored as [2560, 5120]; only the config tells them apart
    q4nx.check_stored_shape([2560, 5120], 8192, 2560)
    q4nx.check_stored_shape([2560, 5120], 2560, 8192)
    q4nx.check_stored_shape([256, 10, 5120], 8192, 2560)
    with pytest.raises(q4nx.Q4NXFormatError):
        q4nx.check_stored_shape([256, 10, 5120], 2560, 8192)   # wrong factoring
    with pytest.raises(q4nx.Q4NXFormatError):
        q4nx.tiled_shape(100, 2560)
    with pytest.raises(q4nx.Q4NXFormatError):
        q4nx.tiled_shape(2560, 1000)
    with pytest.raises(q4nx.Q4NXFormatError):
        q4nx.kind_of_tile_bytes(5121)
    # a tensor whose N or K is not a tile multiple is stored padded to whole tiles
    # (tools/q4nx.py:180-184): N=16 as 32 rows, K=200 as 256
    assert q4nx.padded_shape(16, 200) == (1, 1)
    assert q4nx.padded_shape(40, 300) == (2, 2)
    assert q4nx.padded_shape(8192, 2560) == q4nx.tiled_shape(8192, 2560)
    q4nx.check_stored_shape([1, 1, 5120], 16, 200)
    q4nx.check_stored_shape([4, 8704], 40, 300)
    with pytest.raises(q4nx.Q4NXFormatError):
        q4nx.check_stored_shape([2, 1, 5120], 16, 200)
    q4nx.check_tile_bytes(256 * 10 * 5120, "q4", 8192, 2560)
    with pytest.raises(q4nx.Q4NXFormatError):
        q4nx.check_tile_bytes(256 * 10 * 5120 - 1, "q4", 8192, 2560)


def test_design_meta():
    m = npu._meta_for("lm_head", None)
    assert m["kind"] == "q8" and m["n_rows"] == 248320 and m["k"] == 1024
    assert m["buffers"] == [7760 * 4 * 8704, 2048, 248320 * 4]
    # the reference's design.json has no kind; it follows from the weight buffer size
    m = npu._meta_for("granite", {"n_rows": 8192, "k": 2560, "buffers": [256 * 10 * 5120, 0, 0]})
    assert m["kind"] == "q4" and m["tile_rows"] == 256
    with pytest.raises(SystemExit):
        npu._meta_for("no_such_design", None)
    with pytest.raises(ValueError):
        npu._meta_for("x", {"kind": "q4", "n_rows": 100, "k": 256})


def test_quantize_q8_roundtrip():
    """quantize_q8 writes the q8 tile layout: the oracle's dequantisation of its tiles is the
    input to within half a scale step, element by element, and a tile's brute-force natural
    view agrees."""
    from oracle import q4nx_oracle as qo
    rng = np.random.default_rng(5)
    n, k = 96, 512
    w = (rng.standard_normal((n, k)) * rng.uniform(0.01, 2.0, (n, 1))).astype(np.float32)
    w[3, 40:72] = 0.0                                   # an all-zero group
    t = synth.quantize_q8(w)
    assert t.shape == (n // 32, k // 256, 8704)
    deq = qo.dequant_matrix(t.reshape(-1, 8704), "q8", n // 32, k // 256)
    s = qo.bf16_to_f32(synth.f32_to_bf16_bits(
        np.abs(w.reshape(n, -1, 32)).max(-1) / np.float32(127.0)))
    step = np.repeat(s, 32, axis=1)
    assert (np.abs(deq - w) <= step * 0.5 + 1e-7 + step * 0.01).all()
    assert (deq[3, 40:72] == 0).all()
    nat = qo.dequant_tile_bruteforce(t[1, 1], "q8")
    assert np.array_equal(nat, deq[32:64, 256:512])


def test_missing_library_fails_loudly(tmp_path):
    """No CPU fallback: with the HIP library absent, the first op raises and names the
    missing file (checked in a fresh interpreter whose library path points nowhere)."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("import torch\n"
            "from llmnputest_amd import ops\n"
            "try:\n"
            "    ops.Policy()\n"
            "except RuntimeError as e:\n"
            "    print('RAISED', e)\n"
            "else:\n"
            "    print('NO ERROR')\n")
    env = dict(os.environ, Q4NX_LIB=str(tmp_path / "absent" / "libq4nx_hip.so"))
    r = subprocess.run([sys.executable, "-c", code], cwd=root, env=env, capture_output=True,
                       text=True, timeout=300)
    assert "RAISED" in r.stdout and "is missing" in r.stdout, (r.stdout, r.stderr[-2000:])
