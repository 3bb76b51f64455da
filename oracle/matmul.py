"""fp64 GEMV/GEMM gates and the tolerance metric (numpy oracle).

Test infrastructure only: see the package docstring for who may import this.

Output convention of the reference's packed GEMV/GEMM (native/kernels/rgemv.vyb:13-15,
359-366; native/tools/gen_rpf.py:2-8): Y[m, n] = RS[m, n] + sum_k X[m, k] * W[n, k], W in
GGUF row layout (row n = output n). The gate is max|y - ref| / max|ref| < 2e-3
(native/glm53/verify_layer0.py:134-139; native/FUSED-DQ-GEMM-DESIGN.md:74-90).
"""

import numpy as np

from . import formats

TOL = 2e-3


def rel_maxnorm(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(y - ref)) / max(float(np.max(np.abs(ref))), 1e-300))


def gemm_rows_f64(x, w_rows, residual=None):
    """Y [M, N] = X [M, K] @ W[N, K]^T (+ residual), float64."""
    y = np.asarray(x, np.float64) @ np.asarray(w_rows, np.float64).T
    if residual is not None:
        y = y + np.asarray(residual, np.float64)
    return y


def q4_0_matrix(raw, N, K, order=formats.ORDER_GGML):
    """Packed q4_0 [N rows x K] -> float32 [N, K]."""
    return formats.dequant_q4_0(raw, order).reshape(N, K)


def q8_0_matrix(raw, N, K):
    return formats.dequant_q8_0(raw).reshape(N, K)


def gemv_q4_0_f64(raw, x, N, K, order=formats.ORDER_GGML, residual=None):
    return gemm_rows_f64(np.asarray(x).reshape(-1, K), q4_0_matrix(raw, N, K, order), residual)


def gemv_q8_0_f64(raw, x, N, K, residual=None):
    return gemm_rows_f64(np.asarray(x).reshape(-1, K), q8_0_matrix(raw, N, K), residual)


def gemm_q8_0_int8_f64(raw, xq, xd, N, K):
    """int8 path gate: Y = (xq8-dequantized X) @ W^T in float64."""
    x = formats.dequant_q8_act(xq, xd)
    return gemm_rows_f64(x.reshape(-1, K), q8_0_matrix(raw, N, K))


def gemv_xq8_f64(wtype, raw, xq, xd, N, K, residual=None):
    """Gate of the decode GEMVs on xq8 activations (native/kernels/rgemv7.vyb:3-96 gemv_iq2s_q,
    native/kernels/rq4kq.vyb:7-89 gemv_q4k_q, native/kernels/rq5kq.vyb:8-80 gemv_q5k_q): the float64
    GEMV of the decoded rows with the xq8-dequantized activation x' = xd[k / 32] * xq[k]. The
    reference's kernels compute the same sum as per-sub-block integer dot products times float32
    scales (restated by gemv_xq8_factored_f64)."""
    from . import iquants, kquants
    w = iquants.matrix_iq2_s(raw, N, K) if wtype == iquants.GGML_IQ2_S else kquants.matrix(wtype, raw, N, K)
    # x' in float64: every product of a float32 scale and an int8 is exact there (float32 would round)
    x = (np.asarray(xd, np.float64).reshape(K // 32, 1) * np.asarray(xq, np.float64).reshape(K // 32, 32)).reshape(K)
    return gemm_rows_f64(x.reshape(1, K), w, None if residual is None else np.asarray(residual).reshape(1, N))[0]


def gemv_xq8_factored_f64(wtype, raw, xq, xd, N, K):
    """The same GEMV in the reference kernels' factored form, in float64, from the packed bytes:
    per 32-weight sub-block an integer dot of the raw quants with xq, then the scales:
      Q4_K / Q5_K (rq4kq.vyb:68-69): dx * (d * sc * dot(q, xq) - dmin * m * sum(xq)), q the 4-bit
        (plus bit j of qh[l] as 16 for Q5_K) quants, sc / m the 6-bit scale and min;
      IQ2_S (rgemv7.vyb:82-84): dx * (dlo * (si0 + si1) + dhi * (si2 + si3)), si_l the dot of group l's
        signed grid bytes with xq, dlo / dhi = d * (0.5 + 4-bit scale) / 4."""
    from . import iquants, kquants
    xq = np.asarray(xq, np.int64).reshape(K // 32, 32)
    xd = np.asarray(xd, np.float64).reshape(K // 32)
    nsb = K // 256
    y = np.zeros(N)
    if wtype == iquants.GGML_IQ2_S:
        grid = iquants.iq2s_grid().astype(np.int64)
        b = np.asarray(raw, np.uint8).reshape(N, nsb, iquants.IQ2_S_BYTES).astype(np.int64)
        d = b[:, :, 0:2].astype(np.uint8).copy().view("<f2")[..., 0].astype(np.float64)
        for sb in range(nsb):
            for ib in range(8):
                blk = 8 * sb + ib
                si = np.zeros((N, 4), np.int64)
                for l in range(4):
                    idx = b[:, sb, 2 + 4 * ib + l] | (((b[:, sb, 66 + ib] >> (2 * l)) & 3) << 8)
                    sgn = b[:, sb, 34 + 4 * ib + l]
                    g = grid[idx] * np.where(((sgn[:, None] >> np.arange(8)) & 1) == 1, -1, 1)
                    si[:, l] = g @ xq[blk, 8 * l:8 * l + 8]
                sc = b[:, sb, 74 + ib]
                dlo = d[:, sb] * (0.5 + (sc & 15)) * 0.25
                dhi = d[:, sb] * (0.5 + (sc >> 4)) * 0.25
                y += xd[blk] * (dlo * (si[:, 0] + si[:, 1]) + dhi * (si[:, 2] + si[:, 3]))
        return y
    # Q4_K / Q5_K in the kernels' dword form (rq4kq.vyb:45-66): t = 0..3 selects the qs bytes
    # 32t .. 32t+31 (low nibbles: sub-block 2t, high: 2t+1) and the scale / min bit fields of the
    # header dwords at 4, 8, 12 (shifted by 16 for odd t, the upper 6-bit forms for t >= 2)
    q5 = wtype == kquants.GGML_Q5_K
    bb = kquants.BLOCK_BYTES[wtype]
    qs0 = 48 if q5 else 16
    b = np.asarray(raw, np.uint8).reshape(N, nsb, bb)
    d = b[:, :, 0:2].copy().view("<f2")[..., 0].astype(np.float64)
    dmin = b[:, :, 2:4].copy().view("<f2")[..., 0].astype(np.float64)
    hdr = b[:, :, 4:16].copy().view("<u4").astype(np.int64)  # [N, nsb, 3]
    b64 = b.astype(np.int64)
    for sb in range(nsb):
        ba, bc, be = hdr[:, sb, 0], hdr[:, sb, 1], hdr[:, sb, 2]
        for t in range(4):
            sh = 16 * (t % 2)
            b0, b1, b2 = ba >> sh, bc >> sh, be >> sh
            if t < 2:
                sc = (b0 & 63, (b0 >> 8) & 63)
                mn = (b1 & 63, (b1 >> 8) & 63)
            else:
                sc = ((b2 & 15) | (((b0 >> 6) & 3) << 4), ((b2 >> 8) & 15) | (((b0 >> 14) & 3) << 4))
                mn = (((b2 >> 4) & 15) | (((b1 >> 6) & 3) << 4), ((b2 >> 12) & 15) | (((b1 >> 14) & 3) << 4))
            qsb = b64[:, sb, qs0 + 32 * t:qs0 + 32 * t + 32]
            for h in range(2):
                j = 2 * t + h
                blk = 8 * sb + j
                q = (qsb >> (4 * h)) & 15
                if q5:
                    q = q | (((b64[:, sb, 16:48] >> j) & 1) << 4)
                dot = q @ xq[blk]
                y += xd[blk] * (d[:, sb] * sc[h] * dot - dmin[:, sb] * mn[h] * xq[blk].sum())
    return y
