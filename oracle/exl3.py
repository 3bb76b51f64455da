"""EXL3 4-bpw trellis decode, Hadamard-128 and full dequant (numpy oracle).

Test infrastructure only: see the package docstring for who may import this.

Restates native/exl3/exl3_ref.py:31-120 and native/exl3/README.md:24-49.
Storage per weight matrix W [K, N] (K = in features, N = out features):
  trellis uint16 [K/16, N/16, 64]: 64 words = 256 nibbles per 16x16 tile, LSB-first
  suh fp16 [K], svh fp16 [N]
Rotated-basis value of tile slot (r, c): a 16-bit window w16 composed from 4 nibbles of
the tile stream by the tile-slot composition table, then
  mcg   (codebook 1):  x = w16 * 0xCBAC1FED mod 2^32
  3inst (codebook 0):  x = (w16 * 89226354 + 64248484) mod 2^32   [QTIP paper; parity unpinned]
  y = (x & 0x8FFF8FFF) ^ 0x3B603B60 ; value = fp16(fp16(y & 0xFFFF) + fp16(y >> 16))
  (the two halves are summed in float32 and rounded once to fp16, exl3_ref.py:46-47)
Reconstruction per 128x128 block: W = diag(suh) (H/sqrt(128)) What (H/sqrt(128)) diag(svh),
H the natural-order Sylvester Hadamard-128.
"""

import json
import os

import numpy as np

MCG_MAGIC = 0xCBAC1FED
INST3_MUL = 89226354
INST3_ADD = 64248484
AND_MASK = 0x8FFF8FFF
XOR_MASK = 0x3B603B60
R_SCALE = 0.08838834764831845  # 1/sqrt(128)

CB_3INST = 0
CB_MCG = 1

_HERE = os.path.dirname(os.path.abspath(__file__))
SLOTMAP_GOLDEN = os.path.join(_HERE, "..", "tests", "golden", "exl3_tile_slot_composition.json")


def hash_window(w16, codebook=CB_MCG):
    """uint16-valued windows -> uint32 y (before the fp16 split)."""
    w = np.asarray(w16).astype(np.uint64)
    if codebook == CB_MCG:
        x = (w * np.uint64(MCG_MAGIC)) & np.uint64(0xFFFFFFFF)
    elif codebook == CB_3INST:
        x = (w * np.uint64(INST3_MUL) + np.uint64(INST3_ADD)) & np.uint64(0xFFFFFFFF)
    else:
        raise ValueError(f"unknown codebook {codebook}")
    return ((x & np.uint64(AND_MASK)) ^ np.uint64(XOR_MASK)).astype(np.uint32)


def decode_window(w16, codebook=CB_MCG):
    """uint16 windows -> fp16 values (exl3_ref.py:37-47)."""
    y = hash_window(w16, codebook)
    lo = (y & np.uint32(0xFFFF)).astype(np.uint16).view(np.float16)
    hi = (y >> np.uint32(16)).astype(np.uint16).view(np.float16)
    return (lo.astype(np.float32) + hi.astype(np.float32)).astype(np.float16)


def load_slot_composition(path=None):
    """Tile-slot composition: (rows[256], cols[256], nib[256,4], pos[256,4]) in (r, c) order.

    Slot (r, c) of a 16x16 tile takes its window as OR_i nibble[nib_i] << 4*pos_i
    (exl3_ref.py:66-80; the table is native/exl3/tile_slot_composition.json).
    """
    raw = json.load(open(path or SLOTMAP_GOLDEN))
    if "slots" in raw:
        items = [((s[0], s[1]), s[2]) for s in raw["slots"]]
    else:
        items = [(tuple(int(v) for v in k.split(",")), v) for k, v in raw.items()]
    items.sort(key=lambda kv: kv[0])
    rows = np.array([k[0] for k, _ in items], np.int64)
    cols = np.array([k[1] for k, _ in items], np.int64)
    nib = np.array([[int(m) for m, _ in v] for _, v in items], np.int64)
    pos = np.array([[int(p) for _, p in v] for _, v in items], np.int64)
    return rows, cols, nib, pos


def tile_nibbles(trellis):
    """uint16 [..., 64] -> uint8 nibble stream [..., 256] (nibble m = bits 4m..4m+3, LSB-first)."""
    t = np.asarray(trellis).view(np.uint16) if np.asarray(trellis).dtype == np.int16 else np.asarray(trellis)
    t = t.astype(np.uint32)
    shifts = np.arange(4, dtype=np.uint32) * np.uint32(4)
    nib = (t[..., :, None] >> shifts) & np.uint32(15)
    return nib.reshape(t.shape[:-1] + (256,)).astype(np.uint8)


def tile_windows(trellis, slotmap=None):
    """trellis [..., 64] -> uint32 windows [..., 256] in slot order."""
    rows, cols, nib_idx, pos = slotmap or load_slot_composition()
    nib = tile_nibbles(trellis).astype(np.uint32)
    w = np.zeros(nib.shape[:-1] + (256,), np.uint32)
    for i in range(4):
        w |= nib[..., nib_idx[:, i]] << (np.uint32(4) * pos[:, i].astype(np.uint32))
    return w


def decode_rotated(trellis, codebook=CB_MCG, slotmap=None):
    """trellis uint16 [K/16, N/16, 64] -> rotated-basis What fp16 [K, N] (exl3deq semantics)."""
    trellis = np.asarray(trellis)
    kb, nb, words = trellis.shape
    if words != 64:
        raise ValueError("trellis last dim must be 64")
    sm = slotmap or load_slot_composition()
    rows, cols = sm[0], sm[1]
    vals = decode_window(tile_windows(trellis, sm), codebook)   # [kb, nb, 256]
    what = np.zeros((kb * 16, nb * 16), np.float16)
    rr = np.arange(kb)[:, None, None] * 16 + rows[None, None, :]
    cc = np.arange(nb)[None, :, None] * 16 + cols[None, None, :]
    what[rr, cc] = vals
    return what


def hadamard128():
    """Natural-order Sylvester H_128 (H[0] = all ones), float64 entries +-1."""
    H = np.ones((1, 1), np.float64)
    while H.shape[0] < 128:
        H = np.block([[H, H], [H, -H]])
    return H


def rotate_blocks(what, suh, svh):
    """W = diag(suh) Hs What Hs diag(svh) per 128x128 block, float64 (exact-math form)."""
    what = np.asarray(what, np.float64)
    K, N = what.shape
    if K % 128 or N % 128:
        raise ValueError("K and N must be multiples of 128")
    Hs = hadamard128() * R_SCALE
    t = what.reshape(K // 128, 128, N // 128, 128)
    t = np.einsum("ab,ibjc,cd->iajd", Hs, t, Hs, optimize=True)
    w = t.reshape(K, N)
    return w * np.asarray(suh, np.float64)[:, None] * np.asarray(svh, np.float64)[None, :]


def dequant_exl3_f64(trellis, suh, svh, codebook=CB_MCG, slotmap=None):
    """Full original-basis W [K, N] in float64 (no final fp16 rounding)."""
    return rotate_blocks(decode_rotated(trellis, codebook, slotmap), suh, svh)


def dequant_exl3(trellis, suh, svh, codebook=CB_MCG, slotmap=None):
    """Full W [K, N] rounded to fp16, as exl3_ref.dequant_exl3 returns it (exl3_ref.py:84-120).

    The reference's float32 einsum order is not reproduced; values can differ from it by
    one fp16 ulp where float32 sums round differently. The bit-exact gate is decode_rotated.
    """
    return dequant_exl3_f64(trellis, suh, svh, codebook, slotmap).astype(np.float16)


def fwht128_rows(x):
    """x [..., 128*m] -> per-128-chunk (x_chunk @ H) / sqrt(128), float64."""
    x = np.asarray(x, np.float64)
    sh = x.shape
    xs = x.reshape(sh[:-1] + (sh[-1] // 128, 128))
    return (xs @ (hadamard128() * R_SCALE)).reshape(sh)


def gemm_exl3_f64(x, trellis, suh, svh, codebook=CB_MCG):
    """y [B, N] = x [B, K] @ W (float64), computed as x @ dequant_exl3_f64."""
    return np.asarray(x, np.float64) @ dequant_exl3_f64(trellis, suh, svh, codebook)
