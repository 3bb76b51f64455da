"""GPU parity for the GGUF super-block types (Q4_K, Q5_K, Q6_K, IQ2_S) through the type-id entry points
vybdq_dequant (bit-exact against the oracle) and vybdq_gemv (2e-3 of the float64 gate,
native/glm53/verify_layer0.py:134-139)."""

import numpy as np
import pytest
import torch

from oracle import iquants, kquants, matmul
from tests.test_gpu_gguf import TDT, gate, to_dev, x_as
from vybforge_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu

KQ = [ops.GGML_Q4_K, ops.GGML_Q5_K, ops.GGML_Q6_K, ops.GGML_IQ2_S]
TOL = matmul.TOL
BLOCK = {**kquants.BLOCK_BYTES, ops.GGML_IQ2_S: iquants.IQ2_S_BYTES}


def dequant_ref(ty, raw):
    return iquants.dequant_iq2_s(raw) if ty == ops.GGML_IQ2_S else kquants.DEQUANT[ty](raw)


def matrix_ref(ty, raw, N, K):
    return dequant_ref(ty, raw).reshape(N, K)


@pytest.mark.parametrize("ty", KQ)
@pytest.mark.parametrize("odt", [torch.float64, torch.float32, torch.float16])
def test_dequant_bit_exact(dev, ty, odt):
    rng = np.random.default_rng(ty)
    raw = synth.kquant_weights(rng, ty, 7, 768)
    got = ops.dequant_any(ty, to_dev(raw, dev), 7 * 768, odt).cpu().numpy()
    ref = dequant_ref(ty, raw)
    want = ref if odt == torch.float64 else ref.astype(np.float32)
    if odt == torch.float16:
        want = want.astype(np.float16)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("ty", KQ)
def test_dequant_extreme_fields(dev, ty):
    """Every byte value in the scale/quant fields and fp16 scales from subnormal to large."""
    rng = np.random.default_rng(100 + ty)
    nb = 64
    raw = rng.integers(0, 256, (nb, BLOCK[ty]), dtype=np.uint8)
    fp = {ops.GGML_Q6_K: [208], ops.GGML_IQ2_S: [0]}.get(ty, [0, 2])
    vals = np.array([6e-8, 1e-5, 0.001, 0.5, 2.0, 100.0, -0.25, 0.0], np.float16)
    for o in fp:
        raw[:, o:o + 2] = vals[rng.integers(0, vals.size, nb)].view(np.uint8).reshape(nb, 2)
    raw = raw.reshape(-1)
    got = ops.dequant_any(ty, to_dev(raw, dev), nb * 256, torch.float64).cpu().numpy()
    np.testing.assert_array_equal(got, dequant_ref(ty, raw))


@pytest.mark.parametrize("ty", KQ)
@pytest.mark.parametrize("N,K", [(256, 256), (300, 2560), (64, 4096), (1000, 768), (17, 9728)])
@pytest.mark.parametrize("M", [1, 3])
def test_gemv(dev, ty, N, K, M):
    """Odd super-block counts per row (K = 768: Q6_K rows start 2 bytes past a dword boundary
    every other row), ragged row counts, long rows, several X rows."""
    rng = np.random.default_rng(N * 7 + K + M + ty)
    raw = synth.kquant_weights(rng, ty, N, K)
    x = synth.activations(rng, (M, K))
    y = ops.gemv(ty, to_dev(raw, dev), torch.from_numpy(x).to(dev), N, K).cpu().numpy()
    ref = x.astype(np.float64) @ matrix_ref(ty, raw, N, K).T
    assert matmul.rel_maxnorm(y, ref) < TOL


@pytest.mark.parametrize("ty", KQ)
@pytest.mark.parametrize("xdt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("ydt", ["f32", "f16", "bf16", "f64"])
def test_gemv_dtypes_residual(dev, ty, xdt, ydt):
    rng = np.random.default_rng(ty * 3 + len(xdt) + len(ydt))
    N, K, M = 320, 1536, 2
    raw = synth.kquant_weights(rng, ty, N, K)
    xd, x64 = x_as(synth.activations(rng, (M, K)), xdt, dev)
    rs = torch.from_numpy(rng.standard_normal((M, N))).to(TDT[ydt])
    y = ops.gemv(ty, to_dev(raw, dev), xd, N, K, TDT[ydt], residual=rs.to(dev))
    ref = x64 @ matrix_ref(ty, raw, N, K).T + rs.to(torch.float64).numpy()
    assert gate(y.to(torch.float64).cpu().numpy(), ref, TDT[ydt]) < TOL


@pytest.mark.parametrize("ty", KQ)
@pytest.mark.parametrize("plan", ["8,1,64", "16,2,128", "32,2,256", "64,1,256"])
def test_gemv_forced_plans(dev, monkeypatch, ty, plan):
    """Launch shapes the planner does not pick (lanes per row, units per batch, threads)."""
    monkeypatch.setenv("VYBDQ_GEMV_PLAN", plan)
    rng = np.random.default_rng(ty + len(plan))
    N, K = 200, 3328
    raw = synth.kquant_weights(rng, ty, N, K)
    x = synth.activations(rng, (K,))
    y = ops.gemv(ty, to_dev(raw, dev), torch.from_numpy(x).to(dev), N, K).cpu().numpy()
    ref = matrix_ref(ty, raw, N, K) @ x.astype(np.float64)
    assert matmul.rel_maxnorm(y, ref) < TOL


def test_type_id_errors(dev):
    x = torch.zeros(256, device=dev)
    y = torch.zeros(4, device=dev)
    w = torch.zeros(4 * 210, dtype=torch.uint8, device=dev)
    lib = _lib.lib
    assert lib.vybdq_gemv(3, w.data_ptr(), x.data_ptr(), y.data_ptr(), 1, 4, 256, 0, 0, 0, 0) == _lib.ERR_ARG
    assert lib.vybdq_gemv(14, w.data_ptr(), x.data_ptr(), y.data_ptr(), 1, 4, 128, 0, 0, 0, 0) == _lib.ERR_SHAPE
    assert lib.vybdq_dequant(12, w.data_ptr(), y.data_ptr(), 100, 0, 0) == _lib.ERR_SHAPE


SEG_TYPES = [ops.GGML_Q4_0, ops.GGML_Q8_0] + KQ


def _weights(ty, rng, N, K):
    if ty == ops.GGML_Q4_0:
        return synth.q4_0_weights(rng, N, K)
    if ty == ops.GGML_Q8_0:
        return synth.q8_0_weights(rng, N, K)
    return synth.kquant_weights(rng, ty, N, K)


def _rows(ty, raw, N, K):
    if ty == ops.GGML_Q4_0:
        return matmul.q4_0_matrix(raw, N, K)
    if ty == ops.GGML_Q8_0:
        return matmul.q8_0_matrix(raw, N, K)
    return matrix_ref(ty, raw, N, K)


@pytest.mark.parametrize("ty", SEG_TYPES)
@pytest.mark.parametrize("shapes,K,M,xdt", [([4096, 1024, 1024], 2560, 1, "f16"),   # q|k|v
                                            ([9728, 9728], 2560, 1, "bf16"),         # gate|up
                                            ([5120, 5120], 5120, 1, "f32"),          # two Q8_0 matrices per launch
                                            ([300, 77, 1000], 768, 3, "f32"),        # ragged segments, 3 rows
                                            ([64, 0, 128], 1024, 6, "f16")])         # an absent middle segment, 6 rows
def test_gemv_seg3_every_type(dev, ty, shapes, K, M, xdt):
    """vybdq_gemv_seg3: up to three matrices of one GGUF type sharing X in one launch, each with its
    own output dtype and residual, against the float64 gate (native/kernels/qwen3.vyb:416-436)."""
    rng = np.random.default_rng(sum(shapes) + K + M + ty)
    x = synth.activations(rng, (M, K))
    xd, x64 = x_as(x, xdt, dev)
    ydts = [torch.float32, torch.float16, torch.float64]
    segs, refs = [], []
    for i, n in enumerate(shapes):
        raw = _weights(ty, rng, max(n, 1), K)
        ydt = ydts[i]
        rs = torch.from_numpy(synth.activations(rng, (M, max(n, 1))).astype(np.float64)).to(ydt)
        y = torch.empty((M, max(n, 1)), dtype=ydt, device=dev)
        segs.append((to_dev(raw, dev), y, n, rs.to(dev)))
        refs.append(None if n == 0 else matmul.gemm_rows_f64(x64.reshape(M, K), _rows(ty, raw, n, K),
                                                             rs.to(torch.float64).numpy()))
    ops.gemv_seg3(ty, xd.reshape(M, K), K, segs)
    for (W, y, n, rs), ref in zip(segs, refs):
        if n:
            assert gate(y.to(torch.float64).cpu().numpy(), ref, y.dtype) < TOL, (n, y.dtype)


@pytest.mark.parametrize("ty", KQ)
@pytest.mark.parametrize("M,N,K", [(1, 64, 256), (7, 192, 768), (64, 128, 2560), (100, 64, 1024), (130, 320, 512)])
@pytest.mark.parametrize("xdt", ["bf16", "f32", "f16"])
def test_gemm_superblock_types(dev, ty, M, N, K, xdt):
    """vybdq_gemm on the super-block types (the reference's gemm_h type dispatch,
    native/host/ridge_decode.vyb:295-302): partial m-tiles, odd super-block counts per row (K = 768:
    Q6_K / IQ2_S rows 2 bytes past a dword boundary), every activation type."""
    rng = np.random.default_rng(M * 3 + N + K + ty)
    raw = synth.kquant_weights(rng, ty, N, K)
    x = synth.activations(rng, (M, K))
    xd, x64 = x_as(x, xdt, dev)
    y = ops.gemm(ty, to_dev(raw, dev), xd.reshape(M, K), N, K).cpu().numpy()
    ref = matmul.gemm_rows_f64(x64.reshape(M, K), matrix_ref(ty, raw, N, K))
    assert matmul.rel_maxnorm(y, ref) < TOL


@pytest.mark.parametrize("ty", KQ)
@pytest.mark.parametrize("ydt", [torch.float16, torch.float64])
def test_gemm_superblock_residual_ldy(dev, ty, ydt):
    """Residual of the output type and an output row stride wider than N."""
    M, N, K, ldy = 70, 128, 512, 200
    rng = np.random.default_rng(ty + 11)
    raw = synth.kquant_weights(rng, ty, N, K)
    x = synth.activations(rng, (M, K))
    rs = torch.from_numpy(synth.activations(rng, (M, ldy)).astype(np.float64)).to(ydt)
    y = rs.clone().to(dev)
    Wd, Xd = to_dev(raw, dev), to_dev(x, dev)  # held until the launch has run
    from vybforge_amd._lib import call
    call("vybdq_gemm", ty, Wd.data_ptr(), Xd.data_ptr(), y.data_ptr(), M, N, K,
         ops.F32, ops._dt(ydt), ldy, y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    got = y.to(torch.float64).cpu().numpy()
    ref = matmul.gemm_rows_f64(x, matrix_ref(ty, raw, N, K), rs.to(torch.float64).numpy()[:, :N])
    assert gate(got[:, :N], ref, ydt) < TOL
    np.testing.assert_array_equal(got[:, N:], rs.to(torch.float64).numpy()[:, N:])  # columns past N untouched


@pytest.mark.parametrize("ty", KQ)
@pytest.mark.parametrize("N,K", [(17408, 5120), (5120, 17408)])
def test_gemm_superblock_prefill_shape(dev, ty, N, K):
    """The prefill shapes M = 512 x K x N (up 5120 -> 17408, down 17408 -> 5120) with bf16 X: every
    output computed on the device, 256 columns from the first and the last weight tiles checked
    against the float64 oracle."""
    M = 512
    rng = np.random.default_rng(N + ty)
    raw = synth.kquant_weights(rng, ty, N, K)
    x = torch.from_numpy(synth.activations(rng, (M, K))).to(torch.bfloat16)
    y = ops.gemm(ty, to_dev(raw, dev), x.to(dev), N, K).cpu().numpy()
    x64 = x.to(torch.float64).numpy()
    rb = BLOCK[ty] * (K // 256)
    for c0 in (0, N - 256):
        wrows = matrix_ref(ty, raw[c0 * rb:(c0 + 256) * rb], 256, K)
        assert matmul.rel_maxnorm(y[:, c0:c0 + 256], matmul.gemm_rows_f64(x64, wrows)) < TOL, c0


def _x_pattern(kind, rng, M, K):
    x = rng.standard_normal((M, K))
    if kind == "outlier":        # one channel a million times the rest
        x[:, K // 3] = 1e6
    elif kind == "offset":       # a large common offset
        x = x + 1000.0
    elif kind == "fp16_limit":   # around and past the largest fp16 (65504)
        x = x * 3e4 + np.where(rng.random((M, K)) < 0.05, 7e4, 0.0)
    elif kind == "tiny":         # below the fp16 normal range
        x = x * 1e-7
    elif kind == "huge":
        x = x * 1e12
    return x.astype(np.float32)


@pytest.mark.parametrize("ty", SEG_TYPES)
@pytest.mark.parametrize("kind", ["outlier", "offset", "fp16_limit", "tiny", "huge"])
@pytest.mark.parametrize("xdt,M", [("f32", 1), ("bf16", 1), ("f32", 3)])
def test_gemv_activation_range(dev, ty, kind, xdt, M):
    """float32 / bf16 activations of any magnitude: each 32-element block is staged as fp16 after a
    power-of-two scale, so nothing overflows to inf or flushes to zero (the reference multiplies
    float32 x directly, native/kernels/rgemv.vyb:299-368)."""
    N, K = 300, 2560
    kinds = ["outlier", "offset", "fp16_limit", "tiny", "huge"]
    rng = np.random.default_rng(1000 * ty + 10 * kinds.index(kind) + M + (5 if xdt == "bf16" else 0))
    raw = _weights(ty, rng, N, K)
    xd, x64 = x_as(_x_pattern(kind, rng, M, K), xdt, dev)
    y = ops.gemv(ty, to_dev(raw, dev), xd.reshape(M, K), N, K).cpu().numpy()
    ref = matmul.gemm_rows_f64(x64.reshape(M, K), _rows(ty, raw, N, K))
    assert np.all(np.isfinite(y))
    assert matmul.rel_maxnorm(y, ref) < TOL


def _gemm_ws(ty, W, xd, N, K, dev):
    M = xd.shape[0]
    ws = ops.GemmWorkspace([(M, N, K)], dev, ty)
    assert ws.nbytes > 0 or xd.dtype == torch.float16
    return ops.gemm(ty, W, xd, N, K, workspace=ws)


REG_BODY = [ops.GGML_Q4_K, ops.GGML_Q5_K]


@pytest.mark.parametrize("ty", REG_BODY)
@pytest.mark.parametrize("N,K", [(17408, 5120), (5120, 17408)])
def test_gemm_q4k_register_body_prefill_shape(dev, ty, N, K):
    """Q4_K / Q5_K at the prefill shapes through vybdq_gemm_ws (bf16 X converted once into the
    workspace, the 8-wave tile body with the weights dequantized into the MFMA operand registers
    and the super-block heads (Q5_K: with the high bits) staged in LDS; 17408 -> 5120 splits K):
    256 columns of the first and the last weight tiles against the float64 oracle."""
    M = 512
    rng = np.random.default_rng(N + 7)
    raw = synth.kquant_weights(rng, ty, N, K)
    x = torch.from_numpy(synth.activations(rng, (M, K))).to(torch.bfloat16)
    y = _gemm_ws(ty, to_dev(raw, dev), x.to(dev), N, K, dev).cpu().numpy()
    x64 = x.to(torch.float64).numpy()
    rb = BLOCK[ty] * (K // 256)
    for c0 in (0, N - 256):
        wrows = matrix_ref(ty, raw[c0 * rb:(c0 + 256) * rb], 256, K)
        assert matmul.rel_maxnorm(y[:, c0:c0 + 256], matmul.gemm_rows_f64(x64, wrows)) < TOL, c0


@pytest.mark.parametrize("ty", REG_BODY)
@pytest.mark.parametrize("M,N,K", [(64, 64, 256), (100, 320, 512), (130, 1088, 768), (200, 256, 16384),
                                   (513, 2112, 2560)])
@pytest.mark.parametrize("xdt", ["f16", "bf16_ws", "f32_ws"])
def test_gemm_q4k_register_body_edges(dev, ty, M, N, K, xdt):
    """The Q4_K / Q5_K register-operand body: partial m-tiles (100, 130, 513 rows), a partial last
    n-tile, odd super-step counts per split (K = 768), a long K that splits (16384), fp16 X directly
    and bf16 / f32 X through the workspace; every output against the float64 oracle."""
    rng = np.random.default_rng(M + N + K + ty)
    raw = synth.kquant_weights(rng, ty, N, K)
    x = synth.activations(rng, (M, K))
    xd, x64 = x_as(x, xdt.split("_")[0], dev)
    W = to_dev(raw, dev)
    y = (_gemm_ws(ty, W, xd.reshape(M, K), N, K, dev) if xdt.endswith("_ws")
         else ops.gemm(ty, W, xd.reshape(M, K), N, K)).cpu().numpy()
    ref = matmul.gemm_rows_f64(x64.reshape(M, K), matrix_ref(ty, raw, N, K))
    assert matmul.rel_maxnorm(y, ref) < TOL


@pytest.mark.parametrize("ty", REG_BODY)
@pytest.mark.parametrize("kind", ["outlier", "offset", "fp16_limit", "tiny", "huge"])
def test_gemm_q4k_register_body_activation_range(dev, ty, kind):
    """f32 X of any magnitude through the workspace: each row is converted to fp16 after a
    power-of-two scale that is multiplied back into its outputs."""
    M, N, K = 128, 512, 2560
    kinds = ["outlier", "offset", "fp16_limit", "tiny", "huge"]
    rng = np.random.default_rng(300 + 10 * ty + kinds.index(kind))
    raw = synth.kquant_weights(rng, ty, N, K)
    x = _x_pattern(kind, rng, M, K)
    y = _gemm_ws(ty, to_dev(raw, dev), to_dev(x, dev), N, K, dev).cpu().numpy()
    ref = matmul.gemm_rows_f64(x.astype(np.float64), matrix_ref(ty, raw, N, K))
    assert np.all(np.isfinite(y))
    assert matmul.rel_maxnorm(y, ref) < TOL


TILE128 = [ops.GGML_Q6_K, ops.GGML_IQ2_S]


@pytest.mark.parametrize("ty", TILE128)
@pytest.mark.parametrize("N,K", [(17408, 5120), (5120, 17408)])
def test_gemm_128row_tiles_prefill_shape(dev, ty, N, K):
    """Q6_K / IQ2_S at the prefill shapes through vybdq_gemm_ws: bf16 X converted once into the
    workspace, 128-row tiles with the planner's tile width and K split; 256 columns of the first
    and the last weight tiles against the float64 oracle."""
    M = 512
    rng = np.random.default_rng(N + 17 + ty)
    raw = synth.kquant_weights(rng, ty, N, K)
    x = torch.from_numpy(synth.activations(rng, (M, K))).to(torch.bfloat16)
    y = _gemm_ws(ty, to_dev(raw, dev), x.to(dev), N, K, dev).cpu().numpy()
    x64 = x.to(torch.float64).numpy()
    rb = BLOCK[ty] * (K // 256)
    for c0 in (0, N - 256):
        wrows = matrix_ref(ty, raw[c0 * rb:(c0 + 256) * rb], 256, K)
        assert matmul.rel_maxnorm(y[:, c0:c0 + 256], matmul.gemm_rows_f64(x64, wrows)) < TOL, c0


@pytest.mark.parametrize("ty", TILE128)
@pytest.mark.parametrize("M,N,K", [(96, 64, 256), (130, 320, 768), (200, 256, 4096), (513, 1152, 2560)])
@pytest.mark.parametrize("xdt,splits", [("f16", None), ("bf16_ws", "1"), ("bf16_ws", "3"), ("f32_ws", "2"),
                                        ("f32_ws", None)])
def test_gemm_128row_tiles_edges(dev, monkeypatch, ty, M, N, K, xdt, splits):
    """The 128-row tile path: partial m-tiles (96, 130, 200, 513 rows), odd super-block counts per
    row (K = 768: rows 2 bytes past a dword boundary), K splits reduced in the workspace, fp16 X
    directly and bf16 / f32 X through the workspace; every output against the float64 oracle."""
    if splits is not None:
        monkeypatch.setenv("VYBDQ_KQ2_SPLITS", splits)
    rng = np.random.default_rng(M + N + K + ty + 5)
    raw = synth.kquant_weights(rng, ty, N, K)
    x = synth.activations(rng, (M, K))
    xd, x64 = x_as(x, xdt.split("_")[0], dev)
    W = to_dev(raw, dev)
    y = (_gemm_ws(ty, W, xd.reshape(M, K), N, K, dev) if xdt.endswith("_ws")
         else ops.gemm(ty, W, xd.reshape(M, K), N, K)).cpu().numpy()
    ref = matmul.gemm_rows_f64(x64.reshape(M, K), matrix_ref(ty, raw, N, K))
    assert matmul.rel_maxnorm(y, ref) < TOL


@pytest.mark.parametrize("ty", TILE128)
@pytest.mark.parametrize("ydt", [torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("splits", ["1", "3"])
def test_gemm_128row_tiles_residual_ldy(dev, monkeypatch, ty, ydt, splits):
    """Residual of the output type and a row stride wider than N, in the tile epilogue (one split)
    and in the split reduce."""
    monkeypatch.setenv("VYBDQ_KQ2_SPLITS", splits)
    M, N, K, ldy = 150, 256, 1024, 300
    rng = np.random.default_rng(ty + 21 + int(splits))
    raw = synth.kquant_weights(rng, ty, N, K)
    x = synth.activations(rng, (M, K))
    rs = torch.from_numpy(synth.activations(rng, (M, ldy)).astype(np.float64)).to(ydt)
    y = rs.clone().to(dev)
    Wd, Xd = to_dev(raw, dev), to_dev(x, dev)  # held until the launch has run
    ws = ops.GemmWorkspace([(M, N, K)], dev, ty)
    from vybforge_amd._lib import call
    call("vybdq_gemm_ws", ty, Wd.data_ptr(), Xd.data_ptr(), y.data_ptr(), M, N, K, ops.F32, ops._dt(ydt), ldy,
         y.data_ptr(), ws.ptr, ws.nbytes, torch.cuda.current_stream().cuda_stream)
    got = y.to(torch.float64).cpu().numpy()
    ref = matmul.gemm_rows_f64(x, matrix_ref(ty, raw, N, K), rs.to(torch.float64).numpy()[:, :N])
    assert gate(got[:, :N], ref, ydt) < TOL
    np.testing.assert_array_equal(got[:, N:], rs.to(torch.float64).numpy()[:, N:])  # columns past N untouched


@pytest.mark.parametrize("ty", TILE128)
@pytest.mark.parametrize("kind", ["outlier", "offset", "fp16_limit", "tiny", "huge"])
def test_gemm_128row_tiles_activation_range(dev, ty, kind):
    """f32 X of any magnitude through the workspace: each row is converted to fp16 after a
    power-of-two scale that is multiplied back into its outputs."""
    M, N, K = 128, 512, 2560
    kinds = ["outlier", "offset", "fp16_limit", "tiny", "huge"]
    rng = np.random.default_rng(400 + 10 * ty + kinds.index(kind))
    raw = synth.kquant_weights(rng, ty, N, K)
    x = _x_pattern(kind, rng, M, K)
    y = _gemm_ws(ty, to_dev(raw, dev), to_dev(x, dev), N, K, dev).cpu().numpy()
    ref = matmul.gemm_rows_f64(x.astype(np.float64), matrix_ref(ty, raw, N, K))
    assert np.all(np.isfinite(y))
    assert matmul.rel_maxnorm(y, ref) < TOL


@pytest.mark.parametrize("ty", TILE128)
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
@pytest.mark.parametrize("room", ["x_only", "none"])
def test_gemm_128row_tiles_small_workspace(dev, monkeypatch, ty, xdt, room):
    """vybdq_gemm_ws with less workspace than the planned K split needs: room for the fp16 copy of
    X only (one split), or for nothing (bf16 X converted in the tile, f32 X on the 64-row tiles);
    every output against the float64 oracle."""
    monkeypatch.setenv("VYBDQ_KQ2_SPLITS", "3")
    M, N, K = 200, 320, 3072
    rng = np.random.default_rng(ty + len(xdt) + len(room))
    raw = synth.kquant_weights(rng, ty, N, K)
    x = synth.activations(rng, (M, K))
    xd, x64 = x_as(x, xdt, dev)
    Wd = to_dev(raw, dev)
    full = _lib.lib.vybdq_gemm_workspace_size(ty, M, N, K)
    nb = 0 if room == "none" else (M * K * 2 + 255) // 256 * 256 + (M * 4 + 255) // 256 * 256
    assert nb < full
    ws = torch.zeros(nb + 256, dtype=torch.uint8, device=dev)
    wp = (ws.data_ptr() + 255) // 256 * 256 if nb else 0
    y = torch.empty(M, N, dtype=torch.float32, device=dev)
    _lib.call("vybdq_gemm_ws", ty, Wd.data_ptr(), xd.data_ptr(), y.data_ptr(), M, N, K, ops._dt(xd.dtype), ops.F32,
              0, 0, wp, nb, torch.cuda.current_stream().cuda_stream)
    ref = matmul.gemm_rows_f64(x64.reshape(M, K), matrix_ref(ty, raw, N, K))
    assert matmul.rel_maxnorm(y.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("ty", TILE128)
def test_gemm_ws_x_past_2_32_elements(dev, ty):
    """bf16 X of more than 2^32 elements through vybdq_gemm_ws (M = 2^20 + 128 rows, K = 4096, so
    the rows from 2^20 on start past element 2^32): the conversion into the fp16 workspace copy
    addresses every row from a 64-bit base, so the last rows are their own (a 32-bit element offset
    would wrap them onto the first rows). The first and the last 128 rows against the float64
    oracle."""
    M, N, K = (1 << 20) + 128, 64, 4096
    rng = np.random.default_rng(90 + ty)
    raw = synth.kquant_weights(rng, ty, N, K)
    g = torch.Generator(device=dev)
    g.manual_seed(91)
    x = torch.empty((M, K), dtype=torch.bfloat16, device=dev).normal_(generator=g)
    y = _gemm_ws(ty, to_dev(raw, dev), x, N, K, dev)
    wref = matrix_ref(ty, raw, N, K)
    for r0 in (0, M - 128):
        x64 = x[r0:r0 + 128].to(torch.float64).cpu().numpy()
        got = y[r0:r0 + 128].cpu().numpy()
        assert matmul.rel_maxnorm(got, matmul.gemm_rows_f64(x64, wref)) < TOL, r0
    del x, y
    torch.cuda.empty_cache()
