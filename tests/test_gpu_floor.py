"""The weight-stream floors on the GPU: the null GEMV reads exactly the bytes the row-block
GEMV reads, and the streaming read stores nothing for ordinary data.

The null kernel (the reference's --null design, designs/granite_gemv/granite_gemv.py:105-121)
has no arithmetic to check; what it must get right is its reads. Each of its output words is
the XOR of everything lane r (< 16) of the first wave of its workgroup loaded: for every
K-tile of the wave, the 32 code bytes at rb*2048 + 32r past the nibble plane, that lane's two
d and two m words and its four activations. The expected words are computed here from the
same bytes by index arithmetic written from the q4nx tile format (tools/q4nx.py:7-18), so a
wrong tile, row block, lane offset or metadata index shows up as a mismatch.
"""

import numpy as np
import pytest
import torch

from llmnputest_amd import ops, synth

pytestmark = pytest.mark.gpu


def expected_null(raw: np.ndarray, x_bits: np.ndarray, n_t: int, k_t: int) -> np.ndarray:
    """uint32 [32 * n_t]: the null kernel's output words (see the module docstring)."""
    tpw = next(t for t in (1, 2, 4) if -(-k_t // t) <= 16)
    tiles = raw.reshape(n_t, k_t, 5120)
    xw = np.ascontiguousarray(x_bits, dtype=np.uint16).view(np.uint32)   # bf16 pairs
    out = np.zeros(n_t * 32, np.uint32)
    for lane in range(16):
        qq, gk = lane & 7, lane >> 3
        k0 = gk * 32 + qq * 4
        b0, b1, b2 = lane & 1, (lane >> 1) & 1, (lane >> 2) & 1
        gsw = 2 * b2 + (b1 ^ b2)
        r_first = 2 * gsw + 8 * b0
        for rb in range(2):
            mi = gk * 32 + rb * 16 + r_first
            f = np.zeros(n_t, np.uint32)
            for t in range(tpw):
                kt = min(t, k_t - 1)
                codes = tiles[:, kt, 1024 + rb * 2048 + 32 * lane:1024 + rb * 2048 + 32 * lane + 32]
                cw = np.ascontiguousarray(codes).view(np.uint32)            # [n_t, 8]
                f ^= np.bitwise_xor.reduce(cw, axis=1)
                f ^= np.ascontiguousarray(tiles[:, kt, 2 * mi:2 * mi + 4]).view(np.uint32)[:, 0]
                f ^= np.ascontiguousarray(tiles[:, kt, 512 + 2 * mi:512 + 2 * mi + 4]).view(np.uint32)[:, 0]
                xo = (kt * 256 + k0) // 2
                f ^= xw[xo] ^ xw[xo + 1]
            out[np.arange(n_t) * 32 + rb * 16 + lane] = f
    return out


@pytest.mark.parametrize("n,k", [(8192, 2560), (2560, 8192), (512, 2560), (96, 16384)])
def test_null_gemv_reads_the_gemv_bytes(dev, n, k):
    rng = np.random.default_rng(21)
    raw = synth.q4_tiles(rng, n, k).reshape(-1)
    x = synth.random_bf16(rng, k)
    w = torch.from_numpy(raw).to(dev)
    xd = torch.from_numpy(x.view(np.int16)).to(dev).view(torch.bfloat16)
    y = ops.gemv_q4_null(w, xd, n // 32, k // 256)
    got = y.cpu().numpy().view(np.uint32)
    want = expected_null(raw, x, n // 32, k // 256)
    assert np.array_equal(got, want), int(np.flatnonzero(got != want)[0])


def test_stream_read_stores_nothing(dev):
    sink = torch.zeros(64, dtype=torch.int32, device=dev)
    for nbytes in (16, 4096, 13_107_200 + 48):
        buf = torch.zeros(nbytes, dtype=torch.uint8, device=dev)   # every fold is 0
        ops.stream_read(buf, sink)
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0
