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
