"""Closed-form checks shared by the oracle tests and the ABI tests (not a test module)."""

import numpy as np

from oracle import decode_oracle as do


def rope_angles(table, pos, i):
    """Angle by which pair (i, i + 32) turns at `pos`, recovered from the table."""
    return np.arctan2(table[pos, 1, i], table[pos, 0, i])


def check_rope_frequencies(table_fn):
    """Pair i turns by pos * theta^(-2i/64) (granite_elementwise.py:135-136). For theta =
    10^4 the pairs 8, 16, 24 turn by pos/10, pos/100, pos/1000; for theta = 10^6 pair 16
    turns by pos/1000 and pair 8 by pos/sqrt(1000). theta^(-i/64) instead of
    theta^(-2i/64) gives pos/sqrt(10) at pair 16 and fails."""
    cases = (
        (10000.0, 8, 0.1), (10000.0, 16, 0.01), (10000.0, 24, 0.001),
        (1e6, 16, 1e-3), (1e6, 8, 1.0 / np.sqrt(1000.0)),
    )
    for theta, i, f in cases:
        tab = table_fn(4096, 64, theta)
        for pos in (1, 7, 100, 1234, 4095):
            ang = rope_angles(tab, pos, i)
            want = np.arctan2(np.sin(pos * f), np.cos(pos * f))
            d = np.angle(np.exp(1j * (ang - want)))
            assert abs(d) < 2e-6, (theta, i, pos, ang, want)
    # and the rotation applied to x uses those pairs (dims i and i + 32)
    tab = table_fn(4096, 64, 10000.0)
    x = np.zeros((1, 64))
    x[0, 16] = 1.0
    y = do.rope(x, 300, tab)
    assert np.isclose(y[0, 16], np.cos(3.0), atol=1e-6) and np.isclose(y[0, 48], np.sin(3.0), atol=1e-6)
