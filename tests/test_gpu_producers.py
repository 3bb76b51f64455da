"""GPU parity of the producer-side q8 quantization (vybdq_rmsnorm_q8, vybdq_swiglu_q8) against
the oracle: bit-exact float64 / float32 outputs and q8 copies (the kernels evaluate the same
float64 operations in the same order, without contraction)."""

import numpy as np
import pytest
import torch

from oracle import producers
from vybforge_amd import _lib, ops

pytestmark = pytest.mark.gpu

DT = {"f64": torch.float64, "f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


@pytest.mark.parametrize("xdt", ["f64", "f32", "f16", "bf16"])
@pytest.mark.parametrize("M,N", [(1, 5120), (3, 2560), (2, 96), (1, 17408), (2, 8192), (1, 1536)])
def test_rmsnorm_q8(dev, xdt, M, N):
    rng = np.random.default_rng(M * N + len(xdt))
    x = torch.from_numpy(rng.standard_normal((M, N)) * 3).to(DT[xdt])
    w = torch.from_numpy(rng.uniform(0.5, 1.5, N)).to(DT[xdt])
    eps = 1e-6
    Y, Y32, Xq, Xs = ops.rmsnorm_q8(x.to(dev), w.to(dev), eps, y_dtype=torch.float64, f32_copy=True)
    y, y32, q, d = producers.rms_norm(x.to(torch.float64).numpy(), w.to(torch.float64).numpy(), eps)
    np.testing.assert_array_equal(Y.cpu().numpy(), y)
    np.testing.assert_array_equal(Y32.cpu().numpy(), y32)
    np.testing.assert_array_equal(Xq.cpu().numpy(), q)
    np.testing.assert_array_equal(Xs.cpu().numpy(), d)


def test_rmsnorm_outputs_optional_and_16bit(dev):
    """Only a 16-bit Y (no float32 copy, no q8), N not a multiple of 32; large and tiny rows
    (the Newton seed range ends at 1e-9 and 1e9)."""
    rng = np.random.default_rng(9)
    N = 300
    x = rng.standard_normal((3, N))
    x[1] *= 1e6
    x[2] *= 1e-6
    w = rng.uniform(0.5, 1.5, N)
    for ydt in (torch.float16, torch.bfloat16, torch.float32):
        Y, Y32, Xq, Xs = ops.rmsnorm_q8(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev), 0.0,
                                        y_dtype=ydt, q8=False)
        assert Y32 is None and Xq is None
        y, _, _, _ = producers.rms_norm(x, w, 0.0)
        want = torch.from_numpy(y.astype(np.float32)).to(ydt)
        assert torch.equal(Y.cpu(), want)


@pytest.mark.parametrize("gdt", ["f64", "f32", "bf16"])
@pytest.mark.parametrize("n", [17408, 9728, 64])
def test_swiglu_q8(dev, gdt, n):
    rng = np.random.default_rng(n + len(gdt))
    g = rng.standard_normal(n) * 4
    g[::97] = rng.uniform(-30, 30, g[::97].size)  # past the exp clamp at +-20
    u = rng.standard_normal(n)
    gt, ut = torch.from_numpy(g).to(DT[gdt]), torch.from_numpy(u).to(DT[gdt])
    H, Xq, Xs = ops.swiglu_q8(gt.to(dev), ut.to(dev))
    H64, _, _ = ops.swiglu_q8(gt.to(dev), ut.to(dev), h_dtype=torch.float64, q8=False)
    h, h32, q, d = producers.silu_mul(gt.to(torch.float64).numpy(), ut.to(torch.float64).numpy())
    np.testing.assert_array_equal(H64.cpu().numpy(), h)
    np.testing.assert_array_equal(H.cpu().numpy(), h32)
    np.testing.assert_array_equal(Xq.cpu().numpy(), q)
    np.testing.assert_array_equal(Xs.cpu().numpy(), d)


def test_q8_copy_feeds_the_int8_gemm(dev):
    """The rmsnorm q8 copy is the xq8 layout vybdq_gemm_q8_0_i8 reads: identical to quantizing
    the float32 copy with vybdq_quant_q8_act."""
    rng = np.random.default_rng(4)
    x = torch.from_numpy(rng.standard_normal((4, 1024))).to(dev)
    w = torch.from_numpy(rng.uniform(0.5, 1.5, 1024)).to(dev)
    _, Y32, Xq, Xs = ops.rmsnorm_q8(x, w, 1e-6, f32_copy=True)
    q2, s2 = ops.quant_q8_act(Y32)
    assert torch.equal(Xq, q2) and torch.equal(Xs.reshape(-1), s2.reshape(-1))


def test_argument_errors(dev):
    lib = _lib.lib
    x = torch.zeros(64, dtype=torch.float64, device=dev)
    q = torch.zeros(64, dtype=torch.int8, device=dev)
    assert lib.vybdq_rmsnorm_q8(x.data_ptr(), x.data_ptr(), 0, 0, q.data_ptr(), 0, 1, 64, 1e-6, 3, 0, 0) == _lib.ERR_ARG
    assert lib.vybdq_swiglu_q8(x.data_ptr(), x.data_ptr(), 0, q.data_ptr(), x.data_ptr(), 48, 3, 0, 0) == _lib.ERR_SHAPE
