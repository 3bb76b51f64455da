"""GGUF q4_0 / Q8_0 block decode and the q8 activation quantizer (numpy oracle).

Test infrastructure only: see the package docstring for who may import this.

Block layouts (little-endian, 32 weights per block, rows are K/32 consecutive blocks):
  q4_0: 18 B = [fp16 d][16 B qs];  w = d * (nibble - 8)
  Q8_0: 34 B = [fp16 d][32 x int8]; w = d * q
Both products are exact in float32 (11-bit significand times a 4- or 8-bit integer),
so the float32 decode is the bit-exact gate for the GPU decode.
"""

import numpy as np

QK = 32
Q4_0_BYTES = 18
Q8_0_BYTES = 34

ORDER_GGML = 0         # element j = low nibble of qs[j], element j+16 = high nibble
ORDER_INTERLEAVED = 1  # element 2s = low nibble of qs[s], element 2s+1 = high nibble


def _blocks(raw, nbytes):
    b = np.frombuffer(bytes(raw) if not isinstance(raw, np.ndarray) else raw.tobytes(), np.uint8)
    if b.size % nbytes:
        raise ValueError(f"buffer of {b.size} B is not a whole number of {nbytes}-B blocks")
    return b.reshape(-1, nbytes)


def q4_0_nibbles(raw, order=ORDER_GGML):
    """Packed q4_0 bytes -> uint8 nibble values [nblocks, 32] in element order.

    ORDER_INTERLEAVED is the order the reference's ``deq_q4_0`` intrinsic decodes: its
    only check builds byte s = (2s & 15) | ((2s+1) & 15) << 4 and expects element i to be
    (i % 16) - 8 (native/gguf/mk_fixture.vyb:86-99, native/gguf/dequant_gguf.vyb:118-127).
    ORDER_GGML is the canonical GGUF order of real model files.
    """
    b = _blocks(raw, Q4_0_BYTES)
    qs = b[:, 2:]
    lo = qs & 0x0F
    hi = qs >> 4
    if order == ORDER_GGML:
        return np.concatenate([lo, hi], axis=1)
    if order == ORDER_INTERLEAVED:
        return np.stack([lo, hi], axis=2).reshape(-1, QK)
    raise ValueError(f"unknown q4_0 order {order}")


def q4_0_scales(raw):
    """fp16 block scales as float32 [nblocks]."""
    b = _blocks(raw, Q4_0_BYTES)
    return b[:, 0:2].copy().view("<f2")[:, 0].astype(np.float32)


def dequant_q4_0(raw, order=ORDER_GGML):
    """q4_0 -> float32 [nblocks*32]; w = d * (q - 8) (deq.vyb:4-12 semantics, f32 store)."""
    q = q4_0_nibbles(raw, order).astype(np.int32) - 8
    d = q4_0_scales(raw)
    return (d[:, None] * q.astype(np.float32)).reshape(-1)


def dequant_q8_0(raw):
    """Q8_0 -> float32 [nblocks*32]; w = d * q (q8_0_ref.py:50-56, q8_0.vyb:11-30)."""
    b = _blocks(raw, Q8_0_BYTES)
    d = b[:, 0:2].copy().view("<f2")[:, 0].astype(np.float32)
    qs = b[:, 2:].copy().view(np.int8).astype(np.float32)
    return (qs * d[:, None]).reshape(-1)


def quant_q8_act(x):
    """xq8 activation quantizer (native/kernels/rgemv7.vyb:195-214), per row.

    x float32 [M, K] (or [K]); per 32-value block: a = max|x|, d = a/127 (f32),
    iv = 127/a (0 when a == 0), q = sat_s8(round-half-even(x * iv)).
    Returns (q int8 [M, K], d float32 [M, K/32]).
    """
    x = np.asarray(x, dtype=np.float32)
    squeeze = x.ndim == 1
    x2 = x.reshape(1, -1) if squeeze else x
    M, K = x2.shape
    if K % QK:
        raise ValueError("K must be a multiple of 32")
    xb = x2.reshape(M, K // QK, QK)
    a = np.max(np.abs(xb), axis=2)
    d = (a / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        iv = np.where(a > 0, np.float32(127.0) / np.where(a > 0, a, np.float32(1)), np.float32(0))
    iv = iv.astype(np.float32)
    prod = (xb * iv[:, :, None]).astype(np.float32)
    q = np.clip(np.rint(prod), -128, 127).astype(np.int8).reshape(M, K)
    if squeeze:
        return q.reshape(K), d.reshape(K // QK)
    return q, d


def dequant_q8_act(q, d):
    """Inverse view of quant_q8_act: float32 x' = d_block * q (for the int8-path gate)."""
    q = np.asarray(q)
    squeeze = q.ndim == 1
    q2 = q.reshape(1, -1) if squeeze else q
    M, K = q2.shape
    x = (q2.reshape(M, K // QK, QK).astype(np.float32)
         * np.asarray(d, np.float32).reshape(M, K // QK, 1)).reshape(M, K)
    return x.reshape(K) if squeeze else x


# --- encoders used by tests to build small inputs with known contents -------------------

def pack_q4_0(d, q, order=ORDER_GGML):
    """d float16-representable [nb], q uint8 nibbles [nb, 32] -> packed bytes (uint8 array)."""
    d = np.asarray(d, np.float16).reshape(-1)
    q = np.asarray(q, np.uint8).reshape(-1, QK)
    if np.any(q > 15):
        raise ValueError("nibbles must be < 16")
    nb = q.shape[0]
    out = np.zeros((nb, Q4_0_BYTES), np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    if order == ORDER_GGML:
        out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
    else:
        out[:, 2:] = q[:, 0::2] | (q[:, 1::2] << 4)
    return out.reshape(-1)


def pack_q8_0(d, q):
    d = np.asarray(d, np.float16).reshape(-1)
    q = np.asarray(q, np.int8).reshape(-1, QK)
    nb = q.shape[0]
    out = np.zeros((nb, Q8_0_BYTES), np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)
