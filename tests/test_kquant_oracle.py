"""Pins of the K-quant oracle (oracle/kquants.py), CPU only.

The reference checks its ports against the `gguf` package or a compiled llama.cpp, neither of
which is available here, and holds no K-quant fixture (its gates read real model files). So the
decoders are pinned by blocks assembled byte by byte from the layout description (the packing
direction: a transposed index, a swapped nibble or a wrong shift in the decoder changes values),
with the expected weights written in closed form per element, plus cross-type identities.
"""

import numpy as np
import pytest

from oracle import kquants as kq


def pack_scales(sc, m):
    """Inverse of get_scale_min_k4: 8 six-bit (sc, m) pairs -> scales[12]."""
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = m[j] | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return s


def f16_bytes(v):
    return np.array([v], np.float16).view(np.uint8)


@pytest.mark.parametrize("seed", range(5))
def test_scale_min_k4_roundtrip(seed):
    rng = np.random.default_rng(seed)
    sc = rng.integers(0, 64, 8)
    m = rng.integers(0, 64, 8)
    got_sc, got_m = kq.scale_min_k4(pack_scales(sc, m)[None, :])
    np.testing.assert_array_equal(got_sc[0], sc)
    np.testing.assert_array_equal(got_m[0], m)


def q4k_block(d, dmin, sc, m, q):
    qs = np.zeros(128, np.uint8)
    for g in range(4):
        for l in range(32):
            qs[32 * g + l] = q[64 * g + l] | (q[64 * g + 32 + l] << 4)
    return np.concatenate([f16_bytes(d), f16_bytes(dmin), pack_scales(sc, m), qs])


@pytest.mark.parametrize("seed", range(4))
def test_q4_k_closed_form(seed):
    rng = np.random.default_rng(10 + seed)
    d, dmin = 0.5, 0.125  # exact in fp16
    sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    q = rng.integers(0, 16, 256)
    blk = q4k_block(d, dmin, sc, m, q)
    assert blk.size == kq.Q4_K_BYTES
    want = np.array([d * sc[e // 32] * q[e] - dmin * m[e // 32] for e in range(256)])
    np.testing.assert_array_equal(kq.dequant_q4_k(blk), want)


def q5k_block(d, dmin, sc, m, q5):
    qh = np.zeros(32, np.uint8)
    qs = np.zeros(128, np.uint8)
    for j in range(8):
        for l in range(32):
            qh[l] |= ((q5[32 * j + l] >> 4) & 1) << j
    for g in range(4):
        for l in range(32):
            qs[32 * g + l] = (q5[64 * g + l] & 15) | ((q5[64 * g + 32 + l] & 15) << 4)
    return np.concatenate([f16_bytes(d), f16_bytes(dmin), pack_scales(sc, m), qh, qs])


@pytest.mark.parametrize("seed", range(4))
def test_q5_k_closed_form(seed):
    rng = np.random.default_rng(20 + seed)
    d, dmin = 0.25, 0.0625
    sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    q5 = rng.integers(0, 32, 256)
    blk = q5k_block(d, dmin, sc, m, q5)
    assert blk.size == kq.Q5_K_BYTES
    want = np.array([d * sc[e // 32] * q5[e] - dmin * m[e // 32] for e in range(256)])
    np.testing.assert_array_equal(kq.dequant_q5_k(blk), want)


def test_q5_k_without_high_bits_is_q4_k():
    rng = np.random.default_rng(3)
    sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    q = rng.integers(0, 16, 256)
    b4 = q4k_block(0.75, 0.5, sc, m, q)
    b5 = q5k_block(0.75, 0.5, sc, m, q)
    np.testing.assert_array_equal(kq.dequant_q5_k(b5), kq.dequant_q4_k(b4))


def q6k_block(d, sc16, q6):
    """q6 in 0..63 (stored value; the weight is q6 - 32); sc16 int8 [16]."""
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for h in range(2):
        for l in range(32):
            q1, q2, q3, q4 = (q6[128 * h + 32 * i + l] for i in range(4))
            ql[64 * h + l] = (q1 & 15) | ((q3 & 15) << 4)
            ql[64 * h + 32 + l] = (q2 & 15) | ((q4 & 15) << 4)
            qh[32 * h + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    return np.concatenate([ql, qh, np.asarray(sc16, np.int8).view(np.uint8), f16_bytes(d)])


@pytest.mark.parametrize("seed", range(4))
def test_q6_k_closed_form(seed):
    rng = np.random.default_rng(30 + seed)
    d = 0.375
    sc16 = rng.integers(-128, 128, 16)
    q6 = rng.integers(0, 64, 256)
    blk = q6k_block(d, sc16, q6)
    assert blk.size == kq.Q6_K_BYTES
    # element 128h + 32i + l takes scale 8h + l//16 + 2i
    want = np.array([d * sc16[8 * (e // 128) + (e % 32) // 16 + 2 * ((e % 128) // 32)] * (q6[e] - 32)
                     for e in range(256)])
    np.testing.assert_array_equal(kq.dequant_q6_k(blk), want)


def test_multi_block_rows_and_float32_rounding():
    """Rows of several super-blocks decode block by block; the float32 decode is the float64
    value rounded once (Q6_K is exact in float32)."""
    rng = np.random.default_rng(5)
    N, K = 3, 768
    for ty, gen in ((kq.GGML_Q4_K, None), (kq.GGML_Q5_K, None), (kq.GGML_Q6_K, None)):
        nb = N * K // 256
        raw = rng.integers(0, 256, (nb, kq.BLOCK_BYTES[ty]), dtype=np.uint8)
        fp = [0, 2] if ty != kq.GGML_Q6_K else [208]
        for o in fp:
            raw[:, o:o + 2] = np.abs(rng.normal(0, 1e-3, (nb, 1))).astype(np.float16).view(np.uint8)
        w = kq.matrix(ty, raw.reshape(-1), N, K)
        for b in range(nb):
            np.testing.assert_array_equal(w.reshape(-1)[256 * b:256 * b + 256], kq.DEQUANT[ty](raw[b]))
        if ty == kq.GGML_Q6_K:
            assert np.array_equal(w.astype(np.float32).astype(np.float64), w)
