"""Pin the numpy oracle: reference-held golden vectors, known answers, and independent
re-derivations chosen so that a plausible mistake (wrong nibble order, dropped offset,
wrong rounding mode, transposed operand) fails one of them. CPU only."""

import json
import os
import struct
from fractions import Fraction

import numpy as np
import pytest

from oracle import exl3, formats, matmul, moe
from tests.conftest import GOLDEN


# ---- independent scalar decoders (pure Python, bit level) ------------------------------

def fp16_bits_exact(b):
    """IEEE binary16 bits -> exact Fraction (no NaN/inf in these formats' scale fields)."""
    s = -1 if b >> 15 else 1
    e = (b >> 10) & 31
    m = b & 1023
    if e == 0:
        return s * Fraction(m, 1 << 24)
    assert e != 31
    return s * Fraction(1024 + m, 1 << 25) * (Fraction(2) ** e)


def q4_0_scalar(block, order):
    d = fp16_bits_exact(block[0] | (block[1] << 8))
    out = []
    for i in range(32):
        if order == formats.ORDER_GGML:
            byte = block[2 + (i % 16)]
            nib = byte & 15 if i < 16 else byte >> 4
        else:
            byte = block[2 + i // 2]
            nib = byte & 15 if i % 2 == 0 else byte >> 4
        out.append(d * (nib - 8))
    return out


# ---- q4_0 ------------------------------------------------------------------------------

def test_q4_0_reference_fixture_interleaved():
    g = json.load(open(os.path.join(GOLDEN, "q4_0_gguf_fixture.json")))
    blk = bytes.fromhex(g["block_hex"])
    assert len(blk) == 18 and blk[:2] == b"\x00\x3c"          # d = 1.0
    got = formats.dequant_q4_0(blk, formats.ORDER_INTERLEAVED)
    np.testing.assert_array_equal(got, np.array(g["expected_interleaved"], np.float32))


def test_q4_0_reference_fixture_contradicts_ggml_order():
    # the frozen fixture decodes to (i % 16) - 8 only in the interleaved order; in the GGUF
    # order element 1 is the low nibble of byte 1 (0x32 & 15 = 2) -> -6
    g = json.load(open(os.path.join(GOLDEN, "q4_0_gguf_fixture.json")))
    got = formats.dequant_q4_0(bytes.fromhex(g["block_hex"]), formats.ORDER_GGML)
    assert got[1] == -6.0 and got[16] == -7.0
    assert not np.array_equal(got, np.array(g["expected_interleaved"], np.float32))


@pytest.mark.parametrize("order", [formats.ORDER_GGML, formats.ORDER_INTERLEAVED])
def test_q4_0_matches_bit_level_decoder(order):
    rng = np.random.default_rng(7)
    raw = rng.integers(0, 256, 18 * 40, dtype=np.uint8)
    raw.reshape(40, 18)[:, 1] &= 0x7B   # keep scales finite (exponent < 31)
    got = formats.dequant_q4_0(raw, order).reshape(40, 32)
    for b in range(40):
        ref = q4_0_scalar(raw[18 * b:18 * b + 18].tolist(), order)
        assert [Fraction(float(v)) for v in got[b]] == ref


@pytest.mark.parametrize("order", [formats.ORDER_GGML, formats.ORDER_INTERLEAVED])
def test_q4_0_pack_roundtrip(order):
    rng = np.random.default_rng(3)
    q = rng.integers(0, 16, (9, 32), dtype=np.uint8)
    d = rng.normal(0, 0.01, 9).astype(np.float16)
    raw = formats.pack_q4_0(d, q, order)
    np.testing.assert_array_equal(formats.q4_0_nibbles(raw, order), q)
    np.testing.assert_array_equal(formats.dequant_q4_0(raw, order).reshape(9, 32),
                                  d.astype(np.float32)[:, None] * (q.astype(np.float32) - 8))


# ---- Q8_0 ------------------------------------------------------------------------------

def test_q8_0_matches_bit_level_decoder():
    rng = np.random.default_rng(11)
    raw = rng.integers(0, 256, 34 * 25, dtype=np.uint8)
    raw.reshape(25, 34)[:, 1] &= 0x7B
    got = formats.dequant_q8_0(raw).reshape(25, 32)
    for b in range(25):
        blk = raw[34 * b:34 * b + 34].tolist()
        d = fp16_bits_exact(blk[0] | (blk[1] << 8))
        ref = [d * (v - 256 if v > 127 else v) for v in blk[2:]]
        assert [Fraction(float(v)) for v in got[b]] == ref


def test_q8_0_pack_roundtrip():
    rng = np.random.default_rng(5)
    q = rng.integers(-128, 128, (6, 32)).astype(np.int8)
    d = np.abs(rng.normal(0, 0.01, 6)).astype(np.float16)
    raw = formats.pack_q8_0(d, q)
    np.testing.assert_array_equal(formats.dequant_q8_0(raw).reshape(6, 32),
                                  d.astype(np.float32)[:, None] * q.astype(np.float32))


# ---- xq8 quantizer ---------------------------------------------------------------------

def test_xq8_round_half_even_and_scale():
    # amax = 127 -> d = 1, iv = 1: q = rint(x) exactly; ties go to even (round-half-away
    # would give 1, 3, -1, -3)
    x = np.zeros(32, np.float32)
    x[:6] = [127.0, 0.5, 2.5, -0.5, -2.5, 1.5]
    q, d = formats.quant_q8_act(x)
    assert d[0] == np.float32(1.0)
    assert q[:6].tolist() == [127, 0, 2, 0, -2, 2]


def test_xq8_zero_block_and_extremes():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(96).astype(np.float32)
    x[32:64] = 0.0
    q, d = formats.quant_q8_act(x)
    assert d[1] == 0.0 and not q[32:64].any()
    for b in (0, 2):
        blk = x[32 * b:32 * b + 32]
        j = int(np.argmax(np.abs(blk)))
        assert abs(int(q[32 * b + j])) == 127
        assert d[b] == np.float32(np.float32(np.max(np.abs(blk))) / np.float32(127))
        # reconstruction error at most half a step (plus float32 rounding of x*iv)
        err = np.abs(q[32 * b:32 * b + 32].astype(np.float64) * d[b] - blk)
        assert err.max() <= 0.5 * d[b] * (1 + 1e-6)


def test_xq8_matches_scalar_restatement():
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((3, 64)) * rng.uniform(0.01, 30, (3, 1))).astype(np.float32)
    q, d = formats.quant_q8_act(x)
    f32 = lambda v: struct.unpack("<f", struct.pack("<f", v))[0]
    for m in range(3):
        for b in range(2):
            blk = [float(v) for v in x[m, 32 * b:32 * b + 32]]
            a = max(abs(v) for v in blk)
            iv = f32(127.0 / a)
            for i, v in enumerate(blk):
                assert int(q[m, 32 * b + i]) == max(-128, min(127, round(f32(v * iv))))  # round() is RNE
            assert float(d[m, b]) == f32(a / 127.0)


# ---- EXL3 ------------------------------------------------------------------------------

def test_exl3_zero_trellis_kat():
    # native/exl3/README.md:40: all-zero trellis -> 1.84375 per weight (0x3B60 = 0.921875, x2)
    w = exl3.decode_rotated(np.zeros((2, 3, 64), np.uint16))
    assert w.shape == (32, 48) and np.all(w == np.float16(1.84375))


def test_exl3_window_decode_exhaustive():
    w = np.arange(65536, dtype=np.uint32)
    got = exl3.decode_window(w).view(np.uint16)
    # independent: Python integer hash, exact float64 sum of the two halves, one rounding
    prod = (w.astype(np.uint64) * 3417055213) % (1 << 32)
    y = (prod & 2415890431) ^ 996162400
    lo = (y & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (y >> 16).astype(np.uint16).view(np.float16).astype(np.float64)
    ref = (lo + hi).astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, ref)
    # the halves always sit in [0.125, 2): no inf/nan/subnormal can occur
    e_lo, e_hi = (y >> 10) & 31, (y >> 26) & 31
    assert e_lo.min() >= 12 and e_lo.max() <= 15 and e_hi.min() >= 12 and e_hi.max() <= 15


def test_exl3_only_mcg_codebook():
    # the reference implements one codebook, mcg (exl3_ref.py:19-22): any other id is rejected
    # rather than decoded with constants nothing in the reference fixes
    w = np.array([0, 1, 65535], np.uint32)
    for cb in (0, 2, -1):
        with pytest.raises(ValueError):
            exl3.hash_window(w, cb)
        with pytest.raises(ValueError):
            exl3.decode_window(w, cb)


def test_exl3_slot_map_invariants():
    rows, cols, nib, pos = exl3.load_slot_composition()
    assert len(rows) == 256
    assert len(set(zip(rows.tolist(), cols.tolist()))) == 256
    assert rows.min() == 0 and rows.max() == 15 and cols.min() == 0 and cols.max() == 15
    for i in range(256):
        assert sorted(pos[i].tolist()) == [0, 1, 2, 3]
        assert len(set(nib[i].tolist())) == 4
        assert nib[i].min() >= 0 and nib[i].max() < 256
    # the published example (native/exl3/README.md): slot (0,1) = {39@0,24@1,25@2,26@3}
    i = int(np.nonzero((rows == 0) & (cols == 1))[0][0])
    assert dict(zip(nib[i].tolist(), pos[i].tolist())) == {39: 0, 24: 1, 25: 2, 26: 3}


def test_exl3_product_slot_map_matches_golden():
    prod = json.load(open(os.path.join(os.path.dirname(GOLDEN), "..", "vybforge_amd", "data",
                                       "exl3_slot_composition.json")))
    gold = json.load(open(os.path.join(GOLDEN, "exl3_tile_slot_composition.json")))
    assert prod["slots"] == gold["slots"]


def test_exl3_single_nibble_probe_reaches_declared_slots():
    # setting one stream nibble changes exactly the slots whose composition lists it
    rows, cols, nib, pos = exl3.load_slot_composition()
    base = exl3.tile_windows(np.zeros(64, np.uint16))
    for m in (0, 7, 39, 130, 255):
        t = np.zeros(64, np.uint16)
        t[m // 4] = np.uint16(5 << (4 * (m % 4)))
        changed = set(np.nonzero(exl3.tile_windows(t) != base)[0].tolist())
        assert changed == set(np.nonzero((nib == m).any(axis=1))[0].tolist())


def test_hadamard128_properties():
    H = exl3.hadamard128()
    assert np.array_equal(H, H.T) and np.all(H[0] == 1) and np.all(H[:, 0] == 1)
    np.testing.assert_array_equal(H @ H, 128 * np.eye(128))
    assert H[1, 1] == -1 and H[64, 64] == -1 and H[3, 5] == (-1) ** bin(3 & 5).count("1")


def test_exl3_dequant_zero_trellis_closed_form():
    # What = c * J per 128-block -> (H/8) J (H/8) = 128 e0 e0^T -> W[0,0] = 128 c * suh*svh
    kb, nb = 16, 16
    suh = np.full(256, 0.5, np.float16)
    svh = np.full(256, -2.0, np.float16)
    w = exl3.dequant_exl3_f64(np.zeros((kb, nb, 64), np.uint16), suh, svh)
    ref = np.zeros((256, 256))
    for i in (0, 128):
        for j in (0, 128):
            ref[i, j] = 128 * 1.84375 * 0.5 * -2.0
    np.testing.assert_allclose(w, ref, atol=1e-12)


def test_exl3_rotation_blockwise_matmul():
    rng = np.random.default_rng(4)
    what = rng.standard_normal((256, 384))
    suh, svh = rng.standard_normal(256), rng.standard_normal(384)
    w = exl3.rotate_blocks(what, suh, svh)
    Hs = exl3.hadamard128() / np.sqrt(128)
    ref = np.zeros_like(what)
    for i in range(2):
        for j in range(3):
            blk = what[128 * i:128 * i + 128, 128 * j:128 * j + 128]
            ref[128 * i:128 * i + 128, 128 * j:128 * j + 128] = Hs @ blk @ Hs
    ref = ref * suh[:, None] * svh[None, :]
    np.testing.assert_allclose(w, ref, rtol=1e-12, atol=1e-12)
    # and the FWHT form used by the fused GEMV: x @ W == fwht(fwht(x*suh) @ What) * svh
    x = rng.standard_normal((2, 256))
    y1 = x @ w
    y2 = exl3.fwht128_rows(exl3.fwht128_rows(x * suh) @ what) * svh
    np.testing.assert_allclose(y1, y2, rtol=1e-10, atol=1e-10)


# ---- MoE -------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def moe_golden():
    return np.load(os.path.join(GOLDEN, "moe_golden.npz"))


def test_moe_route_reproduces_reference(moe_golden):
    z = moe_golden
    idx, w = moe.route_logits(z["logits"], 8, z["bias"], float(z["scale"]))
    np.testing.assert_array_equal(idx, z["ref_idx"])
    assert np.max(np.abs(w - z["ref_w"])) < 1e-6      # ref_w was stored as float32


def test_moe_route_without_bias_is_topk_by_logit(moe_golden):
    logits = moe_golden["logits"]
    idx, w = moe.route_logits(logits, 8)
    np.testing.assert_array_equal(idx, np.argsort(-logits, axis=-1, kind="stable")[:, :8])
    np.testing.assert_allclose(w.sum(axis=1), 2.5, rtol=1e-12)


def test_moe_block_output_reproduces_reference(moe_golden):
    # every lane of the reference fixture uses expert 0's weights (moe_ref.moe_block,
    # prepare_moe_fixture.py:54-70): out = sum_i w_i * ffn_e + ffn_shared
    z = moe_golden
    _, w = moe.route_logits(z["logits"], 8, z["bias"], float(z["scale"]))
    a_e = moe.swiglu(z["g_e"], z["u_e"], float(z["limit"]))
    a_s = moe.swiglu(z["g_s"], z["u_s"], float(z["limit"]))
    out = w.sum(axis=1)[:, None] * (a_e @ z["wd_e_cols"].astype(np.float64)) \
        + a_s @ z["wd_s_cols"].astype(np.float64)
    assert matmul.rel_maxnorm(out, z["ref_out_cols"]) < 1e-6


def test_swiglu_clamp():
    g = np.array([-20.0, 0.0, 5.0, 20.0])
    u = np.array([20.0, 3.0, -20.0, 1.0])
    got = moe.swiglu(g, u, 10.0)
    sil = lambda v: v / (1 + np.exp(-v))
    np.testing.assert_allclose(got, [sil(-20) * 10, 0.0, sil(5) * -10, sil(10) * 1], rtol=1e-14)


def test_bucket_layout():
    idx = np.array([[3, 1], [1, 0], [3, 2]])
    counts, offsets, order = moe.bucket(idx, 4)
    assert counts.tolist() == [1, 2, 1, 2]
    assert offsets.tolist() == [0, 1, 3, 4, 6]
    assert order.tolist() == [3, 1, 2, 5, 0, 4]


def test_moe_forward_matches_dense_loop():
    rng = np.random.default_rng(6)
    T, H, I, E = 3, 64, 32, 5
    x = rng.standard_normal((T, H))
    logits = rng.standard_normal((T, E))
    W = [(rng.standard_normal((I, H)), rng.standard_normal((I, H)), rng.standard_normal((H, I)))
         for _ in range(E + 1)]
    out, idx, w = moe.moe_forward(x, logits, lambda e: W[e], W[E], topk=2)
    ref = np.zeros((T, H))
    for t in range(T):
        for s in range(2):
            wg, wu, wd = W[idx[t, s]]
            ref[t] += w[t, s] * (moe.swiglu(wg @ x[t], wu @ x[t]) @ wd.T)
        wg, wu, wd = W[E]
        ref[t] += moe.swiglu(wg @ x[t], wu @ x[t]) @ wd.T
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)


# ---- gates -----------------------------------------------------------------------------

def test_rel_maxnorm_definition():
    assert matmul.rel_maxnorm([1.0, 2.001], [1.0, 2.0]) == pytest.approx(0.0005)


def test_gemv_orientation():
    # W row n is output n: y = W @ x, not W^T @ x
    rng = np.random.default_rng(8)
    q = rng.integers(0, 16, (3 * 2, 32), dtype=np.uint8)   # N=3 rows, K=64
    d = np.ones(6, np.float16)
    raw = formats.pack_q4_0(d, q)
    x = rng.standard_normal(64)
    W = q.reshape(3, 64).astype(np.float64) - 8
    np.testing.assert_allclose(matmul.gemv_q4_0_f64(raw, x, 3, 64)[0], W @ x, rtol=1e-12)


# ---- exl3dq1 / exl3inv (the fused decode + column transform parameter-block kinds) -------------

def test_exl3_tile_map_bytes_match_reference_map_bin():
    """The map.bin body rebuilt from the slot composition hashes to the reference's own
    (native/exl3/map.bin, sha256 recorded beside the composition fixture)."""
    import hashlib
    gold = json.load(open(os.path.join(GOLDEN, "exl3_tile_slot_composition.json")))
    assert hashlib.sha256(exl3.tile_map_bytes()).hexdigest() == gold["map_bin_body_sha256"]


def test_exl3_window_f32_is_the_exact_half_sum():
    """All 65536 windows: the float32 value is the exact sum of the two fp16 halves, and it rounds
    to the pinned fp16 decode."""
    w = np.arange(65536, dtype=np.uint32)
    y = exl3.hash_window(w)
    lo = (y & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (y >> 16).astype(np.uint16).view(np.float16).astype(np.float64)
    f = exl3.decode_window_f32(w)
    assert np.array_equal(f.astype(np.float64), lo + hi)
    assert np.array_equal(f.astype(np.float16), exl3.decode_window(w))


def test_exl3_map_decode_matches_slot_decode():
    """Decoding through the map bytes and their inverse equals the pinned slot-composition decode
    (up to the fp16 rounding that exl3dq1 does not apply)."""
    rng = np.random.default_rng(7)
    rows, cw = 64, 256
    q = rng.integers(0, 256, (rows // 16) * (cw // 16) * 128, dtype=np.uint8).tobytes()
    body = exl3.tile_map_bytes()
    what = exl3.map_decode_f32(q, rows, cw, body, exl3.tile_map_inverse(body))
    trellis = np.frombuffer(q, "<u2").reshape(rows // 16, cw // 16, 64)
    assert np.array_equal(what.astype(np.float16), exl3.decode_rotated(trellis))


def test_exl3_column_transform_layout():
    """Identity H returns What in the reference's T order; Hadamard H inverts by H^T / 128."""
    rng = np.random.default_rng(8)
    what = rng.standard_normal((192, 256))
    t = exl3.column_transform_f64(what, np.eye(128))
    for row, col in [(0, 0), (5, 130), (127, 255), (128, 7), (191, 200)]:
        off = (row // 128 * 2 + col // 128) * 16384 + row % 128 * 128 + col % 128
        assert t[off] == what[row, col]
    H = exl3.hadamard128()
    th = exl3.column_transform_f64(what, H)
    blk = th[16384:2 * 16384].reshape(128, 128)   # rows 0..127, columns 128..255
    assert np.allclose(blk @ H.T / 128.0, what[:128, 128:256], atol=1e-12)


def test_exl3_map_deq_equals_the_map_decode():
    """exl3deq's slot-driven placement (each record's own row / col) equals the pinned
    inverse-map decode for the reference's map, and the all-zero trellis gives the 1.84375 KAT."""
    rng = np.random.default_rng(11)
    rows, cw = 64, 256
    ntiles = (rows // 16) * (cw // 16)
    q = rng.integers(0, 256, ntiles * 128, dtype=np.uint8).tobytes()
    body = exl3.tile_map_bytes()
    got = exl3.map_deq(q, body, cw, ntiles)
    assert np.array_equal(got, exl3.map_decode_f32(q, rows, cw, body, exl3.tile_map_inverse(body)))
    assert (exl3.map_deq(bytes(ntiles * 128), body, cw, ntiles) == np.float32(1.84375)).all()


def test_exl3_hgen_is_the_scaled_sylvester_matrix():
    """The Sylvester sign pattern times the reference's literal 0.08838834764831845 (one float64
    ulp above 1 / sqrt(128); the float32 roundings agree), orthogonal to rounding."""
    H = exl3.hadamard128()
    c = 0.08838834764831845
    assert np.array_equal(exl3.hgen(np.float64), np.where(H > 0, c, -c))
    assert np.allclose(exl3.hgen(np.float64), H / np.sqrt(128.0), rtol=3e-16, atol=0)
    assert np.array_equal(exl3.hgen(np.float32), (H / np.sqrt(128.0)).astype(np.float32))
    assert np.allclose(exl3.hgen() @ exl3.hgen().T, np.eye(128), atol=1e-14)


def test_exl3_had1_is_the_column_transform_and_had2_completes_the_rotation():
    """exl3had1 with nbc = cw / 128 is the pinned column transform; exl3had2 after it is the pinned
    per-block rotation diag(suh) Hs What Hs diag(svh); a smaller nbc touches only its columns."""
    rng = np.random.default_rng(12)
    rows, cw = 256, 384
    what = rng.standard_normal((rows, cw))
    su = rng.standard_normal(rows)
    sv = rng.standard_normal(cw)
    H = exl3.hgen()
    nbc, nblocks = cw // 128, rows // 128 * (cw // 128)
    t = exl3.had1_f64(what, H, cw, nbc, nblocks)
    assert np.array_equal(t, exl3.column_transform_f64(what, H))
    w = exl3.had2_f64(t, H, su, sv, cw, nbc, nblocks)
    assert np.allclose(w, exl3.rotate_blocks(what, su, sv), rtol=0, atol=1e-12)
    t2 = exl3.had1_f64(what, H, cw, 2, rows // 128 * 2)
    w2 = exl3.had2_f64(t2, H, su, sv, cw, 2, rows // 128 * 2)
    assert np.allclose(w2[:, :256], exl3.rotate_blocks(what[:, :256], su, sv[:256]), rtol=0, atol=1e-12)
    assert (w2[:, 256:] == 0).all()


def test_moe_fixture_block_matches_moe_forward():
    """The fixture semantics (one expert on every routed lane) equal the pinned moe_forward with
    that expert for every id and the same float32-rounded logits."""
    rng = np.random.default_rng(9)
    S, H, I, E = 6, 64, 32, 288
    y = rng.standard_normal((S, H))
    G = rng.standard_normal((E, H)) * 0.2
    b = (rng.standard_normal(E) * 0.1).astype(np.float32)
    ws = [rng.standard_normal(s) * 0.3 for s in [(H, I), (H, I), (I, H), (H, I), (H, I), (I, H)]]
    lg, idx, w, act, out = moe.fixture_block(y, G, b, *ws)
    ref, ridx, rw = moe.moe_forward(y, lg.astype(np.float32).astype(np.float64),
                                    lambda e: (ws[0].T, ws[1].T, ws[2].T), (ws[3].T, ws[4].T, ws[5].T), bias=b)
    assert np.array_equal(idx, ridx)
    assert np.abs(w - rw).max() < 1e-15
    assert np.abs(out - ref).max() <= 1e-12 * np.abs(ref).max()
    assert np.array_equal(act[:, 0], act[:, 7])


def test_moe_fixture_route_empty_round_takes_expert_zero():
    """Choices at or below -1e9 never win (moe.vyb:53-74): an all-excluded token picks expert 0."""
    lg = np.zeros((1, 288), np.float32)
    bias = np.full(288, -2e9, np.float32)
    bias[[5, 9]] = 0.0
    idx, _ = moe.fixture_route(lg, bias)
    assert idx[0, :2].tolist() == [5, 9] and (idx[0, 2:] == 0).all()


# ---- the xq8-activation decode GEMV gate ------------------------------------------------

@pytest.mark.parametrize("ty", [12, 13, 22])
def test_xq8_gemv_gate_equals_factored_integer_form(ty):
    # the gate (decoded rows @ x' in float64) against the reference kernels' factored arithmetic
    # (integer sub-block dots from the packed bytes, scale / min fields in their dword form): a
    # dropped min term, a wrong nibble half or scale field, or a sign applied to the wrong group
    # fails here
    from vybforge_amd import synth
    rng = np.random.default_rng(ty)
    N, K = 24, 768
    raw = synth.kquant_weights(rng, ty, N, K)
    xq, xd = formats.quant_q8_act(rng.standard_normal(K).astype(np.float32) * 3)
    a = matmul.gemv_xq8_f64(ty, raw, xq, xd, N, K)
    b = matmul.gemv_xq8_factored_f64(ty, raw, xq, xd, N, K)
    assert matmul.rel_maxnorm(a, b) < 1e-13


@pytest.mark.parametrize("ty", [12, 13, 22])
def test_xq8_gemv_gate_reduces_to_the_exact_gemv(ty):
    # x = q / 8 with every block's largest |q| = 127 quantizes without loss (d = 1/8, xq = q), so the
    # gate equals the exact-activation GEMV of the decoded rows
    from oracle import iquants, kquants
    from vybforge_amd import synth
    rng = np.random.default_rng(40 + ty)
    N, K = 16, 512
    raw = synth.kquant_weights(rng, ty, N, K)
    q = rng.integers(-127, 128, K)
    q.reshape(-1, 32)[:, 5] = 127
    x = (q / 8.0).astype(np.float32)
    xq, xd = formats.quant_q8_act(x)
    assert np.array_equal(xq, q) and np.all(xd == np.float32(0.125))
    w = iquants.matrix_iq2_s(raw, N, K) if ty == 22 else kquants.matrix(ty, raw, N, K)
    exact = w @ x.astype(np.float64)
    assert matmul.rel_maxnorm(matmul.gemv_xq8_f64(ty, raw, xq, xd, N, K), exact) < 1e-14
