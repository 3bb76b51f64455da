"""EXL3 4-bpw trellis decode, Hadamard-128 and full dequant (numpy oracle).

Test infrastructure only: see the package docstring for who may import this.

Restates native/exl3/exl3_ref.py:31-120 and native/exl3/README.md:24-49.
Storage per weight matrix W [K, N] (K = in features, N = out features):
  trellis uint16 [K/16, N/16, 64]: 64 words = 256 nibbles per 16x16 tile, LSB-first
  suh fp16 [K], svh fp16 [N]
Rotated-basis value of tile slot (r, c): a 16-bit window w16 composed from 4 nibbles of
the tile stream by the tile-slot composition table, then
  mcg (codebook 1, exllamav3's decode_3inst at cb=1, exl3_ref.py:19-22):
      x = w16 * 0xCBAC1FED mod 2^32
  (the only codebook the reference implements; any other codebook id raises ValueError)
  y = (x & 0x8FFF8FFF) ^ 0x3B603B60 ; value = fp16(fp16(y & 0xFFFF) + fp16(y >> 16))
  (the two halves are summed in float32 and rounded once to fp16, exl3_ref.py:46-47)
Reconstruction per 128x128 block: W = diag(suh) (H/sqrt(128)) What (H/sqrt(128)) diag(svh),
H the natural-order Sylvester Hadamard-128.
"""

import json
import os

import numpy as np

MCG_MAGIC = 0xCBAC1FED
AND_MASK = 0x8FFF8FFF
XOR_MASK = 0x3B603B60
R_SCALE = 0.08838834764831845  # 1/sqrt(128)

CB_MCG = 1

_HERE = os.path.dirname(os.path.abspath(__file__))
SLOTMAP_GOLDEN = os.path.join(_HERE, "..", "tests", "golden", "exl3_tile_slot_composition.json")


def hash_window(w16, codebook=CB_MCG):
    """uint16-valued windows -> uint32 y (before the fp16 split)."""
    w = np.asarray(w16).astype(np.uint64)
    if codebook != CB_MCG:
        raise ValueError(f"unsupported codebook {codebook}: the reference implements only mcg (1)")
    x = (w * np.uint64(MCG_MAGIC)) & np.uint64(0xFFFFFFFF)
    return ((x & np.uint64(AND_MASK)) ^ np.uint64(XOR_MASK)).astype(np.uint32)


def decode_window(w16, codebook=CB_MCG):
    """uint16 windows -> fp16 values (exl3_ref.py:37-47)."""
    y = hash_window(w16, codebook)
    lo = (y & np.uint32(0xFFFF)).astype(np.uint16).view(np.float16)
    hi = (y >> np.uint32(16)).astype(np.uint16).view(np.float16)
    return (lo.astype(np.float32) + hi.astype(np.float32)).astype(np.float16)


def decode_window_f32(w16, codebook=CB_MCG):
    """uint16 windows -> float32 lo + hi without the fp16 rounding (exl3.vyb:305-309 and
    exl3dq.vyb:88-92: w32 = (fp16_to_f64(lo) + fp16_to_f64(hi)) as Float32; the halves never have
    exponent 0 or 31, so the reference's inf/nan and subnormal branches are never taken)."""
    y = hash_window(w16, codebook)
    lo = (y & np.uint32(0xFFFF)).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (y >> np.uint32(16)).astype(np.uint16).view(np.float16).astype(np.float64)
    return (lo + hi).astype(np.float32)


def tile_map_bytes(slotmap=None):
    """The 256 x 16-byte tile-map body of map.bin (native/exl3/gen_map_bin.py:1-9, 32-37): per slot
    in (row, col) order 4 u16 nibble indices, 4 u8 nibble positions, u16 row, u16 col, little-endian."""
    rows, cols, nib, pos = slotmap or load_slot_composition()
    rec = np.zeros((256, 16), np.uint8)
    rec[:, 0:8] = nib.astype("<u2").view(np.uint8).reshape(256, 8)
    rec[:, 8:12] = pos.astype(np.uint8)
    rec[:, 12:14] = rows.astype("<u2").view(np.uint8).reshape(256, 2)
    rec[:, 14:16] = cols.astype("<u2").view(np.uint8).reshape(256, 2)
    return rec.tobytes()


def tile_map_inverse(body):
    """exl3inv (exl3.vyb:318-333): u32 [256], inv[row * 16 + col] = slot, from a map body."""
    rec = np.frombuffer(body, np.uint8).reshape(256, 16)
    r = rec[:, 12].astype(np.int64) | rec[:, 13].astype(np.int64) << 8
    c = rec[:, 14].astype(np.int64) | rec[:, 15].astype(np.int64) << 8
    inv = np.zeros(256, np.uint32)
    inv[r * 16 + c] = np.arange(256, dtype=np.uint32)
    return inv


def map_decode_f32(q, rows, cw, body, inv):
    """exl3dq1's phase 1 (exl3.vyb:286-309; exl3dq.vyb:60-92): the float32 weights What [rows, cw]
    decoded through a tile map: element (row, col) takes slot inv[(row % 16) 16 + col % 16] of
    tile (row / 16) (cw / 16) + col / 16 (128 bytes of q each) and ORs its four nibbles."""
    q = np.frombuffer(q, np.uint8).reshape(rows // 16, cw // 16, 128)
    rec = np.frombuffer(body, np.uint8).reshape(256, 16)
    nidx = rec[:, 0:8].copy().view("<u2").astype(np.int64)          # [256, 4]
    pp = rec[:, 8:12].astype(np.int64)                                # [256, 4]
    r16, c16 = np.meshgrid(np.arange(16), np.arange(16), indexing="ij")
    slot = np.asarray(inv, np.int64)[(r16 * 16 + c16).ravel()].reshape(16, 16)
    w16 = np.zeros((rows // 16, cw // 16, 16, 16), np.uint32)
    for i in range(4):
        n = nidx[slot, i]                                             # [16, 16]
        byte = q[:, :, n // 2].astype(np.uint32)                      # [kb, nb, 16, 16]
        nib = (byte >> (np.uint32(4) * (n % 2).astype(np.uint32))) & np.uint32(15)
        w16 |= nib << (np.uint32(4) * pp[slot, i].astype(np.uint32))
    what = decode_window_f32(w16).transpose(0, 2, 1, 3).reshape(rows, cw)
    return what


def column_transform_f64(what, H):
    """exl3dq1's phase 2 in float64 (exl3.vyb:310-315; exl3dq.vyb:96-112): for each 128-column
    block, T_block = What_block @ H; returned flat in the reference's T order
    (row / 128 * cw / 128 + col / 128) * 16384 + row % 128 * 128 + d (a half band of 64 rows
    keeps its place inside the 128-row band)."""
    what = np.asarray(what, np.float64)
    rows, cw = what.shape
    H = np.asarray(H, np.float64)
    nbc = cw // 128
    out = np.zeros(((rows + 127) // 128) * nbc * 16384)
    for kb in range(0, rows, 128):
        band = what[kb:kb + 128]
        for nb in range(nbc):
            blk = band[:, nb * 128:(nb + 1) * 128] @ H
            base = (kb // 128 * nbc + nb) * 16384
            out[base:base + blk.size] = blk.ravel()
    return out


def map_deq(q, body, cw, ntiles):
    """exl3deq / exl3deq32 (exl3.vyb:375-422, 207-242): slot s of tile t composes its window from
    the four (nibble index, bit position) pairs of map record s and lands at the record's (row, col)
    inside tile t = (t / (cw / 16), t % (cw / 16)); float32 [ntiles / (cw / 16) 16, cw] (the value
    is the exact half sum, the same in float32 and float64). ntiles must fill whole 16-row bands."""
    nbc = cw // 16
    if ntiles % nbc:
        raise ValueError("ntiles must be a multiple of cw / 16")
    q = np.frombuffer(q, np.uint8).reshape(ntiles, 128)
    rec = np.frombuffer(body, np.uint8)[:4096].reshape(256, 16)
    nidx = rec[:, 0:8].copy().view("<u2").astype(np.int64)          # [256, 4]
    pos = rec[:, 8:12].astype(np.int64)                               # [256, 4]
    rr = rec[:, 12:14].copy().view("<u2").astype(np.int64)[:, 0]
    cc = rec[:, 14:16].copy().view("<u2").astype(np.int64)[:, 0]
    w16 = np.zeros((ntiles, 256), np.uint32)
    for i in range(4):
        byte = q[:, nidx[:, i] // 2].astype(np.uint32)                # [ntiles, 256]
        nib = (byte >> (np.uint32(4) * (nidx[:, i] % 2).astype(np.uint32))) & np.uint32(15)
        w16 |= nib << (np.uint32(4) * pos[:, i].astype(np.uint32))
    val = decode_window_f32(w16)
    t = np.arange(ntiles)
    out = np.zeros((ntiles // nbc * 16, cw), np.float32)
    out[16 * (t // nbc)[:, None] + rr[None, :], 16 * (t % nbc)[:, None] + cc[None, :]] = val
    return out


def hgen(dtype=np.float64):
    """exl3hgen / exl3hgen32 (exl3.vyb:36-56, 124-145): H[i][j] = (-1)^popcount(i & j) times the
    constant 0.08838834764831845 rounded to the stage's precision."""
    i, j = np.meshgrid(np.arange(128), np.arange(128), indexing="ij")
    t = i & j
    par = np.zeros_like(t)
    for k in range(7):
        par += (t >> k) & 1
    c = np.asarray(R_SCALE, np.float64).astype(dtype)
    return np.where(par % 2 == 1, -c, c).astype(dtype)


def had1_f64(W, H, cw, nbc, nblocks):
    """exl3had1 / exl3had132 (exl3.vyb:58-86, 147-172) in float64: for block = kb nbc + nb,
    Tmp[block 16384 + b 128 + d] = sum_c W[(128 kb + b) cw + 128 nb + c] H[c][d]."""
    W = np.asarray(W, np.float64).reshape(-1, cw)
    H = np.asarray(H, np.float64).reshape(128, 128)
    out = np.empty(nblocks * 16384)
    for blk in range(nblocks):
        kb, nb = divmod(blk, nbc)
        out[blk * 16384:(blk + 1) * 16384] = (W[128 * kb:128 * kb + 128, 128 * nb:128 * nb + 128] @ H).ravel()
    return out


def had2_f64(tmp, H, suh, svh, cw, nbc, nblocks):
    """exl3had2 / exl3had232 (exl3.vyb:88-118, 174-202) in float64: O[(128 kb + a) cw + 128 nb + d]
    = (sum_b H[a][b] Tmp[block 16384 + b 128 + d]) suh[128 kb + a] svh[128 nb + d]; returns
    O [nblocks / nbc 128, cw] (columns no block writes stay 0)."""
    tmp = np.asarray(tmp, np.float64)
    H = np.asarray(H, np.float64).reshape(128, 128)
    su = np.asarray(suh, np.float64)
    sv = np.asarray(svh, np.float64)
    out = np.zeros((nblocks // nbc * 128, cw))
    for blk in range(nblocks):
        kb, nb = divmod(blk, nbc)
        o = H @ tmp[blk * 16384:(blk + 1) * 16384].reshape(128, 128)
        out[128 * kb:128 * kb + 128, 128 * nb:128 * nb + 128] = (
            o * su[128 * kb:128 * kb + 128, None] * sv[None, 128 * nb:128 * nb + 128])
    return out


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
