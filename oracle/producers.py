"""Producer-side q8 activation quantization (numpy oracle): RMSNorm and SwiGLU that also write
the q8 copy of their output, as the reference's rms_blkg (VYB_RMSQ8) and silu32q (VYB_SWQ8) do.

Test infrastructure only: see the package docstring for who may import this.

rms_norm (native/kernels/layer.vyb:989-1066, rms_blkg; same values as rms_blk, layer.vyb:880-987):
  float64 throughout. Thread t of 256 sums x[t]^2, x[t+256]^2, ... in index order (a product,
  then an add); the 256 partials are folded pairwise: strides 128, 64, 32, then 16, 8, 4, 2, 1
  (element i += element i + stride); v = total / N + eps; sq = six Newton steps
  y <- (y + v / y) / 2 from the seed v * bits(0x5FE6EB50C7B537A9 - bits(v) / 2) when
  1e-9 < v < 1e9, else 24 steps from y = v (vmath.vyb:75-83, 0 for v <= 0); r = 1 / sq;
  y_i = x_i * r * w_i. The float32 copy is float32(y_i).
silu (layer.vyb:1551-1590, silu32 / silu32q): h = g * (1 / (1 + vexp(-g))) * u in float64 with
  the reference's own exp (vmath.vyb:7-40: argument clamped to [-20, 20], z = x * log2(e),
  n = z rounded half away from zero, r = z - n, 2^r by a degree-8 polynomial summed left to
  right, then n doublings or halvings). The float32 copy is float32(h).
q8 copy (both): formats.quant_q8_act of the float32 copy (xq8, rgemv7.vyb:195-214).
"""

import numpy as np

from oracle import formats

_SEED = np.int64(6910469410427058089)  # 0x5FE6EB50C7B537A9
_EXP_C = (0.6931471805599453, 0.2402265069591007, 0.05550410866482158, 0.009618129107628478,
          0.001333355814642845, 0.0001540353039338161, 0.000015252733804059856,
          0.0000013215486790144306)


def _sqrt_ref(v):
    v = float(v)
    if 0.000000001 < v < 1000000000.0:
        bits = np.array([v], np.float64).view(np.int64)[0]
        y = v * np.array([_SEED - bits // 2], np.int64).view(np.float64)[0]
        for _ in range(6):
            y = 0.5 * (y + v / y)
        return y
    if v <= 0.0:
        return 0.0
    y = v
    for _ in range(24):
        y = 0.5 * (y + v / y)
    return y


def rms_scale(x, N=None):
    """r = 1 / sqrt(sum x^2 / N + eps) of one row (float64), in the reference's order; returns
    the sum of squares (eps is added by the caller)."""
    x = np.asarray(x, np.float64)
    N = x.size if N is None else N
    part = np.zeros(256, np.float64)
    for k in range(0, N, 256):
        seg = x[k:k + 256]
        part[:seg.size] = part[:seg.size] + seg * seg
    for st in (128, 64, 32, 16, 8, 4, 2, 1):
        part[:st] = part[:st] + part[st:2 * st]
    return part[0]


def rms_norm(x, w, eps):
    """x float64 [M, N] (or [N]), w float64 [N] -> (y float64, y32 float32, q int8, d float32)."""
    x = np.asarray(x, np.float64)
    squeeze = x.ndim == 1
    x2 = x.reshape(1, -1) if squeeze else x
    w = np.asarray(w, np.float64)
    y = np.empty_like(x2)
    for m in range(x2.shape[0]):
        v = rms_scale(x2[m]) / float(x2.shape[1]) + eps
        r = 1.0 / _sqrt_ref(v)
        y[m] = x2[m] * r * w
    y32 = y.astype(np.float32)
    q, d = formats.quant_q8_act(y32) if y.shape[1] % 32 == 0 else (None, None)
    if squeeze:
        return y[0], y32[0], (None if q is None else q[0]), (None if d is None else d[0])
    return y, y32, q, d


def vexp(x):
    """The reference's float64 exp (vmath.vyb:7-40), elementwise."""
    x = np.asarray(x, np.float64)
    xt = np.where(x > 20.0, 20.0, x)
    xt = np.where(xt < -20.0, -20.0, xt)
    z = xt * 1.4426950408889634
    n = np.where(z >= 0.0, np.trunc(z + 0.5), np.trunc(z - 0.5))
    r = z - n
    rp = [r]
    for _ in range(7):
        rp.append(rp[-1] * r)
    p = 1.0 + rp[0] * _EXP_C[0]
    for i in range(1, 8):
        p = p + rp[i] * _EXP_C[i]
    n = np.clip(n, -2048, 2048)
    # n doublings / halvings (exact for the |n| <= 29 a clamped argument gives)
    return p * np.exp2(n)


def silu_mul(g, u):
    """g, u float64 [n] -> (h float64, h32 float32, q int8, d float32)."""
    g = np.asarray(g, np.float64)
    u = np.asarray(u, np.float64)
    sg = 1.0 / (1.0 + vexp(0.0 - g))
    h = g * sg * u
    h32 = h.astype(np.float32)
    q, d = formats.quant_q8_act(h32) if h.size % 32 == 0 else (None, None)
    return h, h32, q, d
