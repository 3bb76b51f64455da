"""The host wrappers check every tensor size against the shape arguments before a launch (the
C-ABI sees only pointers, so a wrong size would become an out-of-bounds device access). CPU only:
each call here is rejected before anything reaches the device."""

import pytest
import torch

from vybforge_amd import ops


def u8(n):
    return torch.zeros(n, dtype=torch.uint8)


def test_gemv_checks():
    N, K = 64, 256
    rb = ops.row_bytes(ops.GGML_Q4_0, K)
    with pytest.raises(ValueError, match="columns"):
        ops.gemv(ops.GGML_Q4_0, u8(N * rb), torch.zeros(K + 32), N, K)
    with pytest.raises(ValueError, match="W holds"):
        ops.gemv(ops.GGML_Q4_0, u8(N * rb - 1), torch.zeros(K), N, K)
    with pytest.raises(ValueError, match="out has"):
        ops.gemv(ops.GGML_Q4_0, u8(N * rb), torch.zeros(K), N, K, out=torch.zeros(N - 1))
    with pytest.raises(ValueError, match="residual"):
        ops.gemv(ops.GGML_Q4_0, u8(N * rb), torch.zeros(K), N, K, residual=torch.zeros(N + 1))
    with pytest.raises(ValueError, match="segment 1 W"):
        ops.gemv_q4_0_seg3(torch.zeros(K), K, [(u8(N * rb), torch.zeros(N), N), (u8(10), torch.zeros(N), N)])
    with pytest.raises(ValueError, match="segment 0"):
        ops.gemv_seg3(ops.GGML_Q8_0, torch.zeros(K), K, [(u8(N * 34 * K // 32), torch.zeros(N - 1), N)])


def test_gemm_checks():
    M, N, K = 64, 128, 512
    rb = ops.row_bytes(ops.GGML_Q8_0, K)
    with pytest.raises(ValueError, match="X must be"):
        ops.gemm(ops.GGML_Q8_0, u8(N * rb), torch.zeros(M, K - 64), N, K)
    with pytest.raises(ValueError, match="W holds"):
        ops.gemm(ops.GGML_Q8_0, u8(N * rb - 34), torch.zeros(M, K), N, K)
    with pytest.raises(ValueError, match="out has"):
        ops.gemm(ops.GGML_Q8_0, u8(N * rb), torch.zeros(M, K), N, K, out=torch.zeros(M, N - 16))
    with pytest.raises(ValueError, match="Xs must be"):
        ops.gemm_q8_0_i8(u8(N * rb), torch.zeros(M, K, dtype=torch.int8), torch.zeros(M, K // 64), N, K)
    with pytest.raises(ValueError, match="Xq must be"):
        ops.quant_q8_act(torch.zeros(M, K), out=(torch.zeros(M, K), torch.zeros(M, K // 32)))


def test_exl3_and_moe_checks():
    K, N = 256, 128
    t = torch.zeros(K // 16, N // 16, 64, dtype=torch.int16)
    suh, svh = torch.zeros(K, dtype=torch.float16), torch.zeros(N, dtype=torch.float16)
    with pytest.raises(ValueError, match="trellis"):
        ops.Exl3Linear(t[:-1], suh, svh, K, N)
    with pytest.raises(ValueError, match="suh"):
        ops.Exl3Linear(t, suh[:-1], svh, K, N)
    H, I, E = 256, 128, 4
    rbh, rbi = ops.row_bytes(ops.GGML_Q4_0, H), ops.row_bytes(ops.GGML_Q4_0, I)
    with pytest.raises(ValueError, match="w_down"):
        ops.MoeLayer(ops.GGML_Q4_0, u8(E * I * rbh), u8(E * I * rbh), u8(E * H * rbi - 1), H, I, E, 2)
    with pytest.raises(ValueError, match="shared up"):
        ops.MoeLayer(ops.GGML_Q4_0, u8(E * I * rbh), u8(E * I * rbh), u8(E * H * rbi), H, I, E, 2,
                     shared=(u8(I * rbh), u8(1), u8(H * rbi)))
    layer = ops.MoeLayer(ops.GGML_Q4_0, u8(E * I * rbh), u8(E * I * rbh), u8(E * H * rbi), H, I, E, 2)
    with pytest.raises(ValueError, match="logits must be"):
        layer(torch.zeros(3, H), torch.zeros(3, E + 1))
    with pytest.raises(ValueError, match="x must be"):
        layer(torch.zeros(3, H + 64), torch.zeros(3, E))
