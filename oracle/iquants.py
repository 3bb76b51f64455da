"""GGUF IQ2_S super-block decode (numpy oracle).

Test infrastructure only: see the package docstring for who may import this.

IQ2_S, 82 B per 256 weights: d f16 @0, qs[64] @2 (qs[0:32]: low 8 bits of the grid index of each
group of 8 weights; qs[32:64]: their sign bytes), qh[8] @66, scales[8] @74. Sub-block ib
(32 weights, groups 4ib .. 4ib+3):
  db = d * (0.5 + (scales[ib] & 15)) * 0.25 for groups l = 0, 1; (scales[ib] >> 4) for l = 2, 3
  index = qs[4ib + l] | ((qh[ib] >> 2l) & 3) << 8;  grid entry = 8 magnitudes in {8, 25, 43}
  w[8(4ib + l) + j] = db * grid[index][j] * (-1 if bit j of sign byte qs[32 + 4ib + l] else 1)
(llama.cpp ggml-quants.c dequantize_row_iq2_s, MIT, as the reference ports it in
native/kernels/rgemv.vyb:24-80 gemv_iq2s and checks it in native/tools/iq2_s_ref.py). The grid is
llama.cpp's iq2s_grid as the reference holds it (native/gguf/iq2s_tables.py), in
vybforge_amd/data/iq2s_grid.json. Every weight is exact in float32 (at most 22 significant bits).
"""

import json
import os

import numpy as np

GGML_IQ2_S = 22
IQ2_S_BYTES = 82
_GRID_JSON = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "vybforge_amd", "data", "iq2s_grid.json")


def iq2s_grid():
    """uint8 [1024, 8]: entry i, value j."""
    d = json.load(open(_GRID_JSON))
    g = np.array([int(h, 16) for h in d["grid_u64_hex"]], dtype=np.uint64)
    return g.view(np.uint8).reshape(1024, 8)


def dequant_iq2_s(raw, grid=None):
    """IQ2_S -> float64 [nsb * 256]."""
    grid = iq2s_grid() if grid is None else grid
    b = np.frombuffer(bytes(raw) if not isinstance(raw, np.ndarray) else raw.tobytes(), np.uint8)
    if b.size % IQ2_S_BYTES:
        raise ValueError("not a whole number of IQ2_S super-blocks")
    b = b.reshape(-1, IQ2_S_BYTES)
    d = b[:, 0:2].copy().view("<f2")[:, 0].astype(np.float64)
    qs, signs, qh, sc = (b[:, 2:34].astype(np.int64), b[:, 34:66].astype(np.int64), b[:, 66:74].astype(np.int64),
                         b[:, 74:82].astype(np.int64))
    out = np.empty((b.shape[0], 32, 8), np.float64)
    j = np.arange(8)
    for ib in range(8):
        for l in range(4):
            nib = (sc[:, ib] & 15) if l < 2 else (sc[:, ib] >> 4)
            db = d * (0.5 + nib) * 0.25
            idx = qs[:, 4 * ib + l] | (((qh[:, ib] >> (2 * l)) & 3) << 8)
            g = grid[idx].astype(np.float64)                          # [nsb, 8]
            neg = (signs[:, 4 * ib + l, None] >> j) & 1
            out[:, 4 * ib + l] = db[:, None] * g * np.where(neg == 1, -1.0, 1.0)
    return out.reshape(-1)


def matrix_iq2_s(raw, N, K):
    if K % 256:
        raise ValueError("K must be a multiple of 256")
    return dequant_iq2_s(raw).reshape(N, K)
