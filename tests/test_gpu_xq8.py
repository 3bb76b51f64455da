"""GPU parity of the decode GEMVs on xq8 activations (vybdq_gemv_xq8, vybdq_gemv_xq8_seg3) for Q4_K,
Q5_K and IQ2_S rows. The reference treats these as a lossy path (doc/RIDGE-27B.md:75-84): the gate
here is the float64 GEMV of the xq8-dequantized activation x' = dx * xq (oracle/matmul.py
gemv_xq8_f64), which the kernel reproduces up to float32 scaling and accumulation, so the bar is
XQ8_TOL = 1e-5 of max|ref|, far inside the 2e-3 gate; against the exact GEMV of x itself the
difference is the activation quantization (checked loosely)."""

import numpy as np
import pytest
import torch

from oracle import formats, matmul
from vybforge_amd import ops, synth

pytestmark = pytest.mark.gpu

XQ8_TOL = 1e-5
TYPES = [ops.GGML_Q4_K, ops.GGML_Q5_K, ops.GGML_IQ2_S]


def _setup(dev, ty, N, K, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    raw = synth.kquant_weights(rng, ty, N, K)
    x = (rng.standard_normal(K) * scale).astype(np.float32)
    W = torch.from_numpy(raw).to(dev)
    xq, xd = ops.quant_q8_act(torch.from_numpy(x).to(dev))
    return raw, x, W, xq.reshape(K), xd.reshape(K // 32)


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("N,K", [(256, 2560), (9728, 2560), (2560, 9728), (40, 768), (96, 256)])
def test_gemv_xq8_matches_gate(dev, ty, N, K):
    raw, x, W, xq, xd = _setup(dev, ty, N, K, seed=N + K + ty)
    hq, hd = formats.quant_q8_act(x)
    assert np.array_equal(xq.cpu().numpy(), hq) and np.array_equal(xd.cpu().numpy(), hd)  # the producer is bit-exact
    y = ops.gemv_xq8(ty, W, xq, xd, N, K).cpu().numpy()
    ref = matmul.gemv_xq8_f64(ty, raw, hq, hd, N, K)
    assert matmul.rel_maxnorm(y, ref) < XQ8_TOL, (ty, N, K)


@pytest.mark.parametrize("ty", TYPES)
def test_gemv_xq8_against_the_exact_gemv(dev, ty):
    # lossy by the activation quantization only: the exact GEMV of x differs by well under 2%
    N, K = 2048, 4096
    raw, x, W, xq, xd = _setup(dev, ty, N, K, seed=7 + ty)
    y = ops.gemv_xq8(ty, W, xq, xd, N, K).cpu().numpy()
    exact = ops.gemv(ty, W, torch.from_numpy(x).to(dev), N, K).cpu().numpy()
    rel = matmul.rel_maxnorm(y, exact)
    assert 0 < rel < 2e-2, rel


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("ydt", [torch.float64, torch.float16, torch.bfloat16])
def test_gemv_xq8_outputs_and_residual(dev, ty, ydt):
    N, K = 512, 2048
    raw, x, W, xq, xd = _setup(dev, ty, N, K, seed=11 + ty)
    rs = torch.randn(N, device=dev, dtype=torch.float64).to(ydt)
    y = ops.gemv_xq8(ty, W, xq, xd, N, K, y_dtype=ydt, residual=rs).double().cpu().numpy()
    ref = matmul.gemv_xq8_f64(ty, raw, xq.cpu().numpy(), xd.cpu().numpy(), N, K) + rs.double().cpu().numpy()
    bits = {torch.float64: None, torch.float16: 10, torch.bfloat16: 7}[ydt]
    tol = XQ8_TOL if bits is None else 2.0 ** -bits
    assert matmul.rel_maxnorm(y, ref) < tol


@pytest.mark.parametrize("ty", TYPES)
def test_gemv_xq8_seg3(dev, ty):
    # q|k|v-style: three matrices of different heights on one xq8 row, one launch
    K = 2560
    rng = np.random.default_rng(ty)
    x = rng.standard_normal(K).astype(np.float32)
    xq, xd = ops.quant_q8_act(torch.from_numpy(x).to(dev))
    xq, xd = xq.reshape(K), xd.reshape(K // 32)
    segs, host = [], []
    for N in (4096, 1024, 1024):
        raw = synth.kquant_weights(rng, ty, N, K)
        segs.append((torch.from_numpy(raw).to(dev), torch.empty(N, device=dev), N))
        host.append((raw, N))
    ops.gemv_xq8_seg3(ty, xq, xd, K, segs)
    for (raw, N), (_, Y, _) in zip(host, segs):
        ref = matmul.gemv_xq8_f64(ty, raw, xq.cpu().numpy(), xd.cpu().numpy(), N, K)
        assert matmul.rel_maxnorm(Y.cpu().numpy(), ref) < XQ8_TOL, N


@pytest.mark.parametrize("ty", TYPES)
def test_gemv_xq8_largest_k(dev, ty):
    # K = 65536: the x stage needs more than 64 KB of LDS (the raised limit)
    N, K = 64, 65536
    raw, x, W, xq, xd = _setup(dev, ty, N, K, seed=5 + ty)
    y = ops.gemv_xq8(ty, W, xq, xd, N, K).cpu().numpy()
    ref = matmul.gemv_xq8_f64(ty, raw, xq.cpu().numpy(), xd.cpu().numpy(), N, K)
    assert matmul.rel_maxnorm(y, ref) < XQ8_TOL


def test_gemv_xq8_zero_activation_blocks(dev):
    # all-zero x blocks quantize to d = 0, xq = 0 and contribute nothing (min terms included)
    N, K = 128, 1024
    rng = np.random.default_rng(3)
    x = rng.standard_normal(K).astype(np.float32)
    x[256:512] = 0
    for ty in TYPES:
        raw = synth.kquant_weights(rng, ty, N, K)
        xq, xd = ops.quant_q8_act(torch.from_numpy(x).to(dev))
        y = ops.gemv_xq8(ty, torch.from_numpy(raw).to(dev), xq.reshape(K), xd.reshape(K // 32), N, K).cpu().numpy()
        ref = matmul.gemv_xq8_f64(ty, raw, xq.cpu().numpy(), xd.cpu().numpy(), N, K)
        assert matmul.rel_maxnorm(y, ref) < XQ8_TOL, ty
