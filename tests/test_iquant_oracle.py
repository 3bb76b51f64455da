"""Pins of the IQ2_S oracle (oracle/iquants.py), CPU only: the grid's structure, and blocks
assembled byte by byte from the layout description against closed-form weights."""

import numpy as np
import pytest

from oracle import iquants


def test_grid_structure():
    g = iquants.iq2s_grid()
    assert g.shape == (1024, 8)
    assert set(np.unique(g)) == {8, 25, 43}  # the IQ2 magnitudes
    assert len({bytes(r) for r in g}) == 1024  # distinct entries
    assert (g[0] == 8).all()


def iq2s_block(d, idx, signs, nibs):
    """idx [32] 10-bit grid indices, signs [32] sign bytes, nibs [8, 2] 4-bit scales."""
    qs = np.array([i & 255 for i in idx], np.uint8)
    qh = np.zeros(8, np.uint8)
    for ib in range(8):
        for l in range(4):
            qh[ib] |= ((idx[4 * ib + l] >> 8) & 3) << (2 * l)
    sc = np.array([nibs[ib][0] | (nibs[ib][1] << 4) for ib in range(8)], np.uint8)
    return np.concatenate([np.array([d], np.float16).view(np.uint8), qs, np.asarray(signs, np.uint8), qh, sc])


@pytest.mark.parametrize("seed", range(4))
def test_iq2_s_closed_form(seed):
    rng = np.random.default_rng(seed)
    grid = iquants.iq2s_grid()
    idx = rng.integers(0, 1024, 32)
    signs = rng.integers(0, 256, 32)
    nibs = rng.integers(0, 16, (8, 2))
    d = 0.75
    blk = iq2s_block(d, idx, signs, nibs)
    assert blk.size == iquants.IQ2_S_BYTES
    want = np.empty(256)
    for e in range(256):
        grp, j = e // 8, e % 8
        ib, l = grp // 4, grp % 4
        db = d * (0.5 + nibs[ib][l // 2]) / 4
        want[e] = db * grid[idx[grp], j] * (-1.0 if (signs[grp] >> j) & 1 else 1.0)
    np.testing.assert_array_equal(iquants.dequant_iq2_s(blk), want)
    assert np.array_equal(want.astype(np.float32).astype(np.float64), want)  # exact in float32
