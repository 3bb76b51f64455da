"""GPU parity: q4_0 / Q8_0 decode (bit-exact), fused GEMV (2e-3 of the fp64 gate, per
native/glm53/verify_layer0.py:134-139), xq8 quantizer (bit-exact), through the C-ABI."""

import numpy as np
import pytest
import torch

from oracle import formats, matmul
from vybforge_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu

TOL = matmul.TOL
TDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16, "f64": torch.float64}


def to_dev(a, dev):
    return torch.from_numpy(np.array(a, copy=True)).to(dev)


def gate(y, ref, out_dtype=torch.float32):
    """rel_maxnorm after allowing half an ulp of the output type per element: a 16-bit output
    rounds the float32 accumulator once more, which the 2e-3 accumulation gate does not cover."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    if out_dtype in (torch.float16, torch.bfloat16):
        mant = 10 if out_dtype == torch.float16 else 7
        half_ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - mant - 1)
        err = np.maximum(np.abs(y - ref) - half_ulp, 0.0)
        return float(err.max() / max(np.abs(ref).max(), 1e-300))
    return matmul.rel_maxnorm(y, ref)


def x_as(x32, name, dev):
    """The activation as the GPU sees it, and the same values in float64 for the gate."""
    t = torch.from_numpy(x32).to(TDT[name])
    return t.to(dev), t.to(torch.float64).numpy()


# ---- decode (bit-exact) -----------------------------------------------------------------

@pytest.mark.parametrize("order", [ops.Q4_GGML, ops.Q4_INTERLEAVED])
@pytest.mark.parametrize("odt", ["f32", "f16", "f64"])
def test_dequant_q4_0_bit_exact(dev, order, odt):
    rng = np.random.default_rng(100 + order)
    raw = synth.q4_0_weights(rng, 37, 96)
    nb = raw.size // 18
    got = ops.dequant(ops.GGML_Q4_0, to_dev(raw, dev), nb, TDT[odt], order).cpu().numpy()
    ref = formats.dequant_q4_0(raw, order)
    np.testing.assert_array_equal(got, ref.astype(got.dtype))


def test_dequant_q4_0_reference_fixture(dev):
    import json, os
    from tests.conftest import GOLDEN
    g = json.load(open(os.path.join(GOLDEN, "q4_0_gguf_fixture.json")))
    raw = np.frombuffer(bytes.fromhex(g["block_hex"]), np.uint8)
    got = ops.dequant(ops.GGML_Q4_0, to_dev(raw, dev), 1, torch.float64, ops.Q4_INTERLEAVED).cpu().numpy()
    np.testing.assert_array_equal(got, np.array(g["expected_interleaved"], np.float64))


@pytest.mark.parametrize("odt", ["f32", "f16", "f64"])
def test_dequant_q8_0_bit_exact(dev, odt):
    rng = np.random.default_rng(200)
    raw = synth.q8_0_weights(rng, 29, 128)
    nb = raw.size // 34
    got = ops.dequant(ops.GGML_Q8_0, to_dev(raw, dev), nb, TDT[odt]).cpu().numpy()
    np.testing.assert_array_equal(got, formats.dequant_q8_0(raw).astype(got.dtype))


def test_dequant_full_config1_bit_exact(dev):
    rng = np.random.default_rng(1)
    raw = synth.q4_0_weights(rng, 9728, 2560)
    got = ops.dequant(ops.GGML_Q4_0, to_dev(raw, dev), raw.size // 18).cpu().numpy()
    np.testing.assert_array_equal(got, formats.dequant_q4_0(raw))


# ---- GEMV ----------------------------------------------------------------------------------

GEMV_SHAPES = [(9728, 2560), (64, 64), (100, 96), (2560, 4096), (2560, 9728), (33, 2048), (1, 6144)]


@pytest.mark.parametrize("N,K", GEMV_SHAPES)
@pytest.mark.parametrize("order", [ops.Q4_GGML, ops.Q4_INTERLEAVED])
def test_gemv_q4_0_f32(dev, N, K, order):
    rng = np.random.default_rng(N * 7 + K)
    raw = synth.q4_0_weights(rng, N, K)
    x = synth.activations(rng, (K,))
    y = ops.gemv(ops.GGML_Q4_0, to_dev(raw, dev), to_dev(x, dev), N, K, order=order).cpu().numpy()
    ref = matmul.gemv_q4_0_f64(raw, x, N, K, order)[0]
    assert matmul.rel_maxnorm(y, ref) < TOL


@pytest.mark.parametrize("xdt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("ydt", ["f32", "f16", "bf16", "f64"])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
def test_gemv_q4_0_dtypes_batch(dev, xdt, ydt, M):
    N, K = 96, 2560
    rng = np.random.default_rng(M * 13)
    raw = synth.q4_0_weights(rng, N, K)
    xd, x64 = x_as(synth.activations(rng, (M, K)), xdt, dev)
    y = ops.gemv(ops.GGML_Q4_0, to_dev(raw, dev), xd, N, K, TDT[ydt]).to(torch.float64).cpu().numpy()
    ref = matmul.gemv_q4_0_f64(raw, x64, N, K)
    assert gate(y, ref, TDT[ydt]) < TOL


@pytest.mark.parametrize("ydt", ["f32", "f64", "f16"])
def test_gemv_residual(dev, ydt):
    N, K = 200, 1024
    rng = np.random.default_rng(5)
    raw = synth.q4_0_weights(rng, N, K)
    x = synth.activations(rng, (K,))
    rs = synth.activations(rng, (N,)).astype(np.float64)
    rs_t = torch.from_numpy(rs).to(TDT[ydt])
    y = ops.gemv(ops.GGML_Q4_0, to_dev(raw, dev), to_dev(x, dev), N, K, TDT[ydt],
                 residual=rs_t.to(dev)).to(torch.float64).cpu().numpy()
    ref = matmul.gemv_q4_0_f64(raw, x, N, K, residual=rs_t.to(torch.float64).numpy())[0]
    assert gate(y, ref, TDT[ydt]) < TOL


@pytest.mark.parametrize("N,K", [(5120, 5120), (48, 5120), (4096, 512), (77, 96)])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_gemv_q8_0(dev, N, K, xdt):
    rng = np.random.default_rng(N + K)
    raw = synth.q8_0_weights(rng, N, K)
    xd, x64 = x_as(synth.activations(rng, (K,)), xdt, dev)
    y = ops.gemv(ops.GGML_Q8_0, to_dev(raw, dev), xd, N, K).cpu().numpy()
    ref = matmul.gemv_q8_0_f64(raw, x64, N, K)[0]
    assert matmul.rel_maxnorm(y, ref) < TOL


def test_gemv_q8_0_batch(dev):
    N, K, M = 300, 4096, 6
    rng = np.random.default_rng(77)
    raw = synth.q8_0_weights(rng, N, K)
    x = synth.activations(rng, (M, K))
    y = ops.gemv(ops.GGML_Q8_0, to_dev(raw, dev), to_dev(x, dev), N, K).cpu().numpy()
    assert matmul.rel_maxnorm(y, matmul.gemv_q8_0_f64(raw, x, N, K)) < TOL


def test_gemv_seg3_qkv(dev):
    K = 2560
    rng = np.random.default_rng(42)
    shapes = [4096, 1024, 1024]
    raws = [synth.q4_0_weights(rng, n, K) for n in shapes]
    xd, x64 = x_as(synth.activations(rng, (K,)), "f16", dev)
    ys = [torch.empty(n, dtype=torch.float16, device=dev) for n in shapes]
    ops.gemv_q4_0_seg3(xd, K, [(to_dev(r, dev), y, n) for r, y, n in zip(raws, ys, shapes)])
    for r, y, n in zip(raws, ys, shapes):
        ref = matmul.gemv_q4_0_f64(r, x64, n, K)[0]
        assert gate(y.to(torch.float64).cpu().numpy(), ref, torch.float16) < TOL


@pytest.mark.parametrize("N,K", [(2560, 4096), (2560, 9728)])
def test_gemv_decode_stack_fp16_launches(dev, N, K):
    """The decode stack's fp16-x / fp16-y launches of o (4096 -> 2560) and down (9728 -> 2560), the
    instantiations the benchmark replays, against the float64 oracle on every row."""
    rng = np.random.default_rng(N + K)
    raw = synth.q4_0_weights(rng, N, K)
    xd, x64 = x_as(synth.activations(rng, (K,)), "f16", dev)
    y = ops.gemv(ops.GGML_Q4_0, to_dev(raw, dev), xd, N, K, y_dtype=torch.float16)
    ref = matmul.gemv_q4_0_f64(raw, x64, N, K)[0]
    assert gate(y.to(torch.float64).cpu().numpy(), ref, torch.float16) < TOL


def test_gemv_decode_stack_gate_up_launch(dev):
    """The decode stack's gate|up launch: two 9728-row segments sharing one fp16 x of 2560."""
    K, I = 2560, 9728
    rng = np.random.default_rng(77)
    raws = [synth.q4_0_weights(rng, I, K) for _ in range(2)]
    xd, x64 = x_as(synth.activations(rng, (K,)), "f16", dev)
    ys = [torch.empty(I, dtype=torch.float16, device=dev) for _ in range(2)]
    ops.gemv_q4_0_seg3(xd, K, [(to_dev(r, dev), y, I) for r, y in zip(raws, ys)])
    for r, y in zip(raws, ys):
        ref = matmul.gemv_q4_0_f64(r, x64, I, K)[0]
        assert gate(y.to(torch.float64).cpu().numpy(), ref, torch.float16) < TOL


@pytest.mark.parametrize("plan", ["8,5,256", "8,1,64", "16,3,128", "16,2,256", "32,2,128", "32,5,64",
                                  "64,3,256", "64,1,128"])
@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_gemv_forced_launch_plans(dev, plan, fmt):
    """Every (lanes per row, pairs per batch, threads) shape on ragged rows: lanes past their last
    pair, partial last workgroups and multi-batch rows (batch smaller than the row)."""
    import os
    N, K = 301, 2560
    rng = np.random.default_rng(17)
    if fmt == "q4_0":
        raw, ty, ref_fn = synth.q4_0_weights(rng, N, K), ops.GGML_Q4_0, matmul.gemv_q4_0_f64
    else:
        raw, ty, ref_fn = synth.q8_0_weights(rng, N, K), ops.GGML_Q8_0, matmul.gemv_q8_0_f64
        g, u, t = plan.split(",")
        plan = ",".join([g, str(min(int(u), 3)), t])
    x = synth.activations(rng, (K,))
    os.environ["VYBDQ_GEMV_PLAN"] = plan
    try:
        y = ops.gemv(ty, to_dev(raw, dev), to_dev(x, dev), N, K).cpu().numpy()
    finally:
        os.environ.pop("VYBDQ_GEMV_PLAN", None)
    assert matmul.rel_maxnorm(y, ref_fn(raw, x, N, K)[0]) < TOL


def test_gemv_deterministic(dev):
    N, K = 4096, 4096
    rng = np.random.default_rng(3)
    W = to_dev(synth.q4_0_weights(rng, N, K), dev)
    x = to_dev(synth.activations(rng, (K,)), dev)
    a = ops.gemv(ops.GGML_Q4_0, W, x, N, K)
    b = ops.gemv(ops.GGML_Q4_0, W, x, N, K)
    assert torch.equal(a, b)


def test_gemv_rejects_misaligned_w(dev):
    W = torch.zeros(18 * 2 * 64 + 2, dtype=torch.uint8, device=dev)
    x = torch.zeros(64, dtype=torch.float32, device=dev)
    y = torch.zeros(2, dtype=torch.float32, device=dev)
    rc = _lib.lib.vybdq_gemv_q4_0(W.data_ptr() + 2, x.data_ptr(), y.data_ptr(), 1, 2, 64,
                                  _lib.F32, _lib.F32, 0, 0, 0)
    assert rc == _lib.ERR_ALIGN


# ---- xq8 quantizer (bit-exact) ------------------------------------------------------------

@pytest.mark.parametrize("xdt", ["f32", "f16", "bf16"])
def test_quant_q8_act_bit_exact(dev, xdt):
    rng = np.random.default_rng(17)
    x32 = (rng.standard_normal((5, 512)) * rng.uniform(0.01, 50, (5, 1))).astype(np.float32)
    x32[1, 64:96] = 0.0
    x32[2, 0:32] = np.linspace(-127, 127, 32).astype(np.float32) * 0.5  # exact .5 ties
    xd, x64 = x_as(x32, xdt, dev)
    q, d = ops.quant_q8_act(xd)
    rq, rd = formats.quant_q8_act(x64.astype(np.float32))
    np.testing.assert_array_equal(q.cpu().numpy(), rq)
    np.testing.assert_array_equal(d.cpu().numpy(), rd)
