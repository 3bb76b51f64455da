"""GGUF K-quant super-block decode (Q4_K, Q5_K, Q6_K): numpy oracle.

Test infrastructure only: see the package docstring for who may import this.

The three layouts are llama.cpp's (ggml-quants.c dequantize_row_q4_K / q5_K / q6_K, MIT), which
the reference ports in native/kernels/q4k.vyb:1-70 (q4kdeq), native/tools/q4k_ref.py:37-60,
native/kernels/q5k.vyb and native/tools/q5k_ref.py, native/gguf/q6k_verify.py:20-40. The
independent authority those scripts compare against, the ``gguf`` package, is not installed
here; the pins are in tests/test_kquant_oracle.py (blocks assembled from the layout description
byte by byte, closed-form values, and the q4_0 special case).

A super-block holds QK_K = 256 weights; a row of K weights is K/256 super-blocks.

Q4_K, 144 B: d f16 @0, dmin f16 @2, scales[12] @4, qs[128] @16.
  Sub-block j (32 weights, j = 0..7) has a 6-bit scale sc_j and min m_j packed in scales[]
  (get_scale_min_k4); group g = 0..3 takes qs[32g : 32g+32]: the low nibbles are sub-block 2g,
  the high nibbles sub-block 2g+1.  w = d * sc_j * q - dmin * m_j.
Q5_K, 176 B: d f16 @0, dmin f16 @2, scales[12] @4, qh[32] @16, qs[128] @48.
  As Q4_K, with a fifth bit: element l of sub-block j adds 16 when bit j of qh[l] is set.
Q6_K, 210 B: ql[128] @0, qh[64] @128, scales[16] int8 @192, d f16 @208.
  Two halves of 128; half h uses ql[64h : 64h+64], qh[32h : 32h+32], scales[8h : 8h+8]. For
  l = 0..31 (is = l // 16):
    w[128h +      l] = d * sc[8h+is+0] * ((ql[64h+l]    & 15 | (qh[32h+l] >> 0 & 3) << 4) - 32)
    w[128h + 32 + l] = d * sc[8h+is+2] * ((ql[64h+32+l] & 15 | (qh[32h+l] >> 2 & 3) << 4) - 32)
    w[128h + 64 + l] = d * sc[8h+is+4] * ((ql[64h+l]    >> 4 | (qh[32h+l] >> 4 & 3) << 4) - 32)
    w[128h + 96 + l] = d * sc[8h+is+6] * ((ql[64h+32+l] >> 4 | (qh[32h+l] >> 6 & 3) << 4) - 32)

Every weight is exact in float64 (at most 25 significant bits before the Q4_K/Q5_K
subtraction, whose two terms are exact), and rounded once in float32:
``dequant_*`` returns the float64 values, ``.astype(np.float32)`` is the float32 decode.
"""

import numpy as np

QK_K = 256
Q4_K_BYTES = 144
Q5_K_BYTES = 176
Q6_K_BYTES = 210

# GGML type ids (the reference dispatches on these: native/host/ridge_decode.vyb:294-311)
GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K = 2, 8, 12, 13, 14
BLOCK_BYTES = {GGML_Q4_K: Q4_K_BYTES, GGML_Q5_K: Q5_K_BYTES, GGML_Q6_K: Q6_K_BYTES}


def _sblocks(raw, nbytes):
    b = np.frombuffer(bytes(raw) if not isinstance(raw, np.ndarray) else raw.tobytes(), np.uint8)
    if b.size % nbytes:
        raise ValueError(f"buffer of {b.size} B is not a whole number of {nbytes}-B super-blocks")
    return b.reshape(-1, nbytes)


def _f16(b, off):
    return b[:, off:off + 2].copy().view("<f2")[:, 0].astype(np.float64)


def scale_min_k4(scales):
    """get_scale_min_k4 for the eight sub-blocks: uint8 [nsb, 12] -> (sc, m) int [nsb, 8].

    j < 4:  sc = s[j] & 63,                     m = s[j+4] & 63
    j >= 4: sc = (s[j+4] & 15) | (s[j-4] >> 6) << 4,   m = (s[j+4] >> 4) | (s[j] >> 6) << 4
    (native/kernels/q4k.vyb:41-52, native/tools/q4k_ref.py:37-53)
    """
    s = scales.astype(np.int64)
    sc = np.empty((s.shape[0], 8), np.int64)
    mn = np.empty((s.shape[0], 8), np.int64)
    for j in range(8):
        if j < 4:
            sc[:, j] = s[:, j] & 63
            mn[:, j] = s[:, j + 4] & 63
        else:
            sc[:, j] = (s[:, j + 4] & 15) | ((s[:, j - 4] >> 6) << 4)
            mn[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    return sc, mn


def q4_k_quants(raw):
    """Q4_K -> (d, dmin float64 [nsb], sc, m int [nsb, 8], q int [nsb, 256]) in element order."""
    b = _sblocks(raw, Q4_K_BYTES)
    sc, mn = scale_min_k4(b[:, 4:16])
    qs = b[:, 16:].reshape(-1, 4, 32).astype(np.int64)
    q = np.concatenate([qs & 15, qs >> 4], axis=2).reshape(-1, QK_K)  # group g: lo = 2g, hi = 2g+1
    return _f16(b, 0), _f16(b, 2), sc, mn, q


def q5_k_quants(raw):
    """Q5_K -> (d, dmin, sc, m, q) like q4_k_quants, q in 0..31."""
    b = _sblocks(raw, Q5_K_BYTES)
    sc, mn = scale_min_k4(b[:, 4:16])
    qh = b[:, 16:48].astype(np.int64)                      # [nsb, 32]
    qs = b[:, 48:].reshape(-1, 4, 32).astype(np.int64)     # [nsb, group, l]
    q = np.empty((b.shape[0], 8, 32), np.int64)
    for g in range(4):
        q[:, 2 * g] = (qs[:, g] & 15) + 16 * ((qh >> (2 * g)) & 1)
        q[:, 2 * g + 1] = (qs[:, g] >> 4) + 16 * ((qh >> (2 * g + 1)) & 1)
    return _f16(b, 0), _f16(b, 2), sc, mn, q.reshape(-1, QK_K)


def q6_k_quants(raw):
    """Q6_K -> (d float64 [nsb], sc int [nsb, 16], q int [nsb, 256] in -32..31)."""
    b = _sblocks(raw, Q6_K_BYTES)
    ql = b[:, 0:128].astype(np.int64)
    qh = b[:, 128:192].astype(np.int64)
    sc = b[:, 192:208].view(np.int8).astype(np.int64)
    q = np.empty((b.shape[0], 2, 4, 32), np.int64)
    for h in range(2):
        lo, hi, hb = ql[:, 64 * h:64 * h + 32], ql[:, 64 * h + 32:64 * h + 64], qh[:, 32 * h:32 * h + 32]
        q[:, h, 0] = ((lo & 15) | (((hb >> 0) & 3) << 4)) - 32
        q[:, h, 1] = ((hi & 15) | (((hb >> 2) & 3) << 4)) - 32
        q[:, h, 2] = ((lo >> 4) | (((hb >> 4) & 3) << 4)) - 32
        q[:, h, 3] = ((hi >> 4) | (((hb >> 6) & 3) << 4)) - 32
    return _f16(b, 208), sc, q.reshape(-1, QK_K)


def q6_k_element_scales(sc):
    """Per-element scale index of Q6_K: element 128h + 32i + l uses sc[8h + l//16 + 2i]."""
    e = np.arange(QK_K)
    h, i, l = e // 128, (e % 128) // 32, e % 32
    return sc[:, 8 * h + l // 16 + 2 * i]


def dequant_q4_k(raw):
    """Q4_K -> float64 [nsb * 256]: d * sc_j * q - dmin * m_j."""
    d, dmin, sc, mn, q = q4_k_quants(raw)
    j = np.arange(QK_K) // 32
    return (d[:, None] * sc[:, j] * q - dmin[:, None] * mn[:, j]).reshape(-1)


def dequant_q5_k(raw):
    """Q5_K -> float64 [nsb * 256]: d * sc_j * q5 - dmin * m_j."""
    d, dmin, sc, mn, q = q5_k_quants(raw)
    j = np.arange(QK_K) // 32
    return (d[:, None] * sc[:, j] * q - dmin[:, None] * mn[:, j]).reshape(-1)


def dequant_q6_k(raw):
    """Q6_K -> float64 [nsb * 256]: d * sc * q."""
    d, sc, q = q6_k_quants(raw)
    return (d[:, None] * q6_k_element_scales(sc) * q).reshape(-1)


DEQUANT = {GGML_Q4_K: dequant_q4_k, GGML_Q5_K: dequant_q5_k, GGML_Q6_K: dequant_q6_k}


def matrix(wtype, raw, N, K):
    """Rows [N, K] float64 of a packed K-quant matrix (GGUF row layout)."""
    if K % QK_K:
        raise ValueError("K must be a multiple of 256")
    return DEQUANT[wtype](raw).reshape(N, K)
