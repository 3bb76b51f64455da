"""GPU parity: dequant MFMA GEMM (q4_0 / Q8_0, 2e-3 of the float64 gate) and the MoE layer
(router against the reference's committed goldens; full layer against the oracle)."""

import os

import numpy as np
import pytest
import torch

from oracle import formats, matmul, moe
from tests.conftest import GOLDEN
from vybforge_amd import ops, synth

pytestmark = pytest.mark.gpu
TOL = matmul.TOL
TDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def dev_t(a, dev):
    return torch.from_numpy(np.array(a, copy=True)).to(dev)


def gate16(y, ref, dtype):
    y = np.asarray(y, np.float64)
    if dtype in (torch.float16, torch.bfloat16):
        mant = 10 if dtype == torch.float16 else 7
        half = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - mant - 1)
        return float(np.maximum(np.abs(y - ref) - half, 0).max() / np.abs(ref).max())
    return matmul.rel_maxnorm(y, ref)


def weights(ty, rng, N, K):
    return synth.q4_0_weights(rng, N, K) if ty == ops.GGML_Q4_0 else synth.q8_0_weights(rng, N, K)


def ref_rows(ty, raw, N, K):
    return matmul.q4_0_matrix(raw, N, K) if ty == ops.GGML_Q4_0 else matmul.q8_0_matrix(raw, N, K)


@pytest.mark.parametrize("ty", [ops.GGML_Q4_0, ops.GGML_Q8_0])
@pytest.mark.parametrize("M,N,K", [(512, 256, 5120), (16, 128, 256), (64, 192, 128), (200, 256, 512), (1, 64, 64),
                                   (130, 128, 1024)])
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_gemm(dev, ty, M, N, K, xdt):
    rng = np.random.default_rng(M + N + K + ty)
    raw = weights(ty, rng, N, K)
    x = torch.from_numpy(synth.activations(rng, (M, K))).to(TDT[xdt])
    y = ops.gemm(ty, dev_t(raw, dev), x.to(dev), N, K).cpu().numpy()
    ref = matmul.gemm_rows_f64(x.to(torch.float64).numpy(), ref_rows(ty, raw, N, K))
    assert matmul.rel_maxnorm(y, ref) < TOL


@pytest.mark.parametrize("ty,K", [(ops.GGML_Q8_0, 5120), (ops.GGML_Q8_0, 17408)])
def test_gemm_config3_rows(dev, ty, K):
    # the prefill shapes M=512 x K x N: a 512-row slice of N checked against float64
    rng = np.random.default_rng(K)
    M, N = 512, 512
    raw = weights(ty, rng, N, K)
    x = torch.from_numpy(synth.activations(rng, (M, K))).to(torch.bfloat16)
    y = ops.gemm(ty, dev_t(raw, dev), x.to(dev), N, K, torch.bfloat16).to(torch.float64).cpu().numpy()
    ref = matmul.gemm_rows_f64(x.to(torch.float64).numpy(), ref_rows(ty, raw, N, K))
    assert gate16(y, ref, torch.bfloat16) < TOL


@pytest.mark.parametrize("ty", [ops.GGML_Q4_0, ops.GGML_Q8_0])
@pytest.mark.parametrize("M,N,K", [(64, 16, 256), (128, 272, 512), (200, 320, 1024), (77, 48, 768),
                                   (128, 256, 8192), (300, 64, 4096)])
@pytest.mark.parametrize("xdt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("split", [False, True])
def test_gemm_mfma_tiles(dev, ty, M, N, K, xdt, split):
    """The register-B MFMA GEMM (K % 256 == 0, M >= 64): odd fragment counts per tile, partial
    M tiles, and long K split across workgroups through the workspace."""
    rng = np.random.default_rng(M * 7 + N + K + ty)
    raw = weights(ty, rng, N, K)
    x = torch.from_numpy(synth.activations(rng, (M, K))).to(TDT[xdt])
    ws = ops.GemmWorkspace([(M, N, K)], dev, ty) if split else None
    W = dev_t(raw, dev)
    y = ops.gemm(ty, W, x.to(dev), N, K, workspace=ws).cpu().numpy()
    ref = matmul.gemm_rows_f64(x.to(torch.float64).numpy(), ref_rows(ty, raw, N, K))
    assert matmul.rel_maxnorm(y, ref) < TOL
    if split:
        # deterministic, and the counters are left zeroed for the next call
        y2 = ops.gemm(ty, W, x.to(dev), N, K, workspace=ws).cpu().numpy()
        np.testing.assert_array_equal(y, y2)


@pytest.mark.parametrize("F", [1, 2, 3, 5, 6, 7, 9, 11, 13, 15, 17, 18, 19, 20])
@pytest.mark.parametrize("splits", [1, 3])
def test_gemm_mfma_forced_tiles(dev, monkeypatch, F, splits):
    """Every per-wave fragment count (0..5) and a ragged last tile, with and without a K split."""
    monkeypatch.setenv("VYBDQ_MMQ_PLAN", f"{F},{splits}")
    ty = ops.GGML_Q8_0 if F % 2 else ops.GGML_Q4_0
    M, N, K = 150, 16 * (2 * F + 3), 768
    rng = np.random.default_rng(F * 10 + splits)
    raw = weights(ty, rng, N, K)
    x = torch.from_numpy(synth.activations(rng, (M, K))).to(torch.bfloat16)
    ws = ops.GemmWorkspace([(M, N, K)], dev, ty) if splits > 1 else None
    if ws is not None:
        # the override applies to the workspace query as well
        assert ws.nbytes > 0
    y = ops.gemm(ty, dev_t(raw, dev), x.to(dev), N, K, workspace=ws).cpu().numpy()
    ref = matmul.gemm_rows_f64(x.to(torch.float64).numpy(), ref_rows(ty, raw, N, K))
    assert matmul.rel_maxnorm(y, ref) < TOL


@pytest.mark.parametrize("N,K,cols", [(17408, 5120, 320), (5120, 17408, 256)])
def test_gemm_config3_full_shape(dev, N, K, cols):
    """The prefill shapes at full size (the benchmark's tiling and K split), checked against float64
    on a column slice taken from the start and the end of N."""
    rng = np.random.default_rng(N + K)
    M = 512
    raw = synth.q8_0_weights(rng, N, K)
    x = torch.from_numpy(synth.activations(rng, (M, K))).to(torch.bfloat16)
    ws = ops.GemmWorkspace([(M, N, K)], dev, ops.GGML_Q8_0)
    y = ops.gemm(ops.GGML_Q8_0, dev_t(raw, dev), x.to(dev), N, K, workspace=ws).cpu().numpy()
    rows = raw.reshape(N, -1)
    x64 = x.to(torch.float64).numpy()
    for c0 in (0, N - cols):
        ref = matmul.gemm_rows_f64(x64, ref_rows(ops.GGML_Q8_0, rows[c0:c0 + cols].reshape(-1), cols, K))
        assert matmul.rel_maxnorm(y[:, c0:c0 + cols], ref) < TOL


@pytest.mark.parametrize("M,N,K", [(1, 16, 256), (64, 48, 768), (130, 272, 512), (200, 256, 5120), (77, 320, 1024),
                                   (128, 64, 8192)])
@pytest.mark.parametrize("split", [False, True])
def test_gemm_int8_path(dev, M, N, K, split):
    """int8 path: xq8 on the GPU, then the int8 MFMA GEMM, against the float64 gate of the
    dequantized activations and weights."""
    rng = np.random.default_rng(M * 3 + N + K)
    raw = synth.q8_0_weights(rng, N, K)
    x = synth.activations(rng, (M, K))
    xq, xs = ops.quant_q8_act(dev_t(x, dev))
    ref_q, ref_s = formats.quant_q8_act(x.reshape(-1, K))
    np.testing.assert_array_equal(xq.cpu().numpy(), ref_q.reshape(M, K))
    ws = ops.GemmWorkspace([(M, N, K)], dev, int8=True) if split else None
    W = dev_t(raw, dev)
    y = ops.gemm_q8_0_i8(W, xq, xs, N, K, workspace=ws).cpu().numpy()
    ref = matmul.gemm_q8_0_int8_f64(raw, ref_q, ref_s, N, K).reshape(M, N)
    assert matmul.rel_maxnorm(y, ref) < TOL
    if split:
        np.testing.assert_array_equal(y, ops.gemm_q8_0_i8(W, xq, xs, N, K, workspace=ws).cpu().numpy())


@pytest.mark.parametrize("F,splits", [(1, 1), (3, 2), (5, 1), (7, 3), (13, 1), (16, 2)])
def test_gemm_int8_forced_tiles(dev, monkeypatch, F, splits):
    monkeypatch.setenv("VYBDQ_MMQ_PLAN", f"{F},{splits}")
    M, N, K = 150, 16 * (2 * F + 3), 768
    rng = np.random.default_rng(F * 11 + splits)
    raw = synth.q8_0_weights(rng, N, K)
    x = synth.activations(rng, (M, K))
    xq, xs = ops.quant_q8_act(dev_t(x, dev))
    ws = ops.GemmWorkspace([(M, N, K)], dev, int8=True) if splits > 1 else None
    y = ops.gemm_q8_0_i8(dev_t(raw, dev), xq, xs, N, K, workspace=ws).cpu().numpy()
    ref_q, ref_s = formats.quant_q8_act(x.reshape(-1, K))
    ref = matmul.gemm_q8_0_int8_f64(raw, ref_q, ref_s, N, K).reshape(M, N)
    assert matmul.rel_maxnorm(y, ref) < TOL


@pytest.mark.parametrize("N,K,cols", [(17408, 5120, 272), (5120, 17408, 256)])
def test_gemm_int8_config3_full_shape(dev, N, K, cols):
    rng = np.random.default_rng(N * 2 + K)
    M = 512
    raw = synth.q8_0_weights(rng, N, K)
    x = synth.activations(rng, (M, K))
    xq, xs = ops.quant_q8_act(dev_t(x, dev))
    ws = ops.GemmWorkspace([(M, N, K)], dev, int8=True)
    y = ops.gemm_q8_0_i8(dev_t(raw, dev), xq, xs, N, K, workspace=ws).cpu().numpy()
    ref_q, ref_s = formats.quant_q8_act(x.reshape(-1, K))
    rows = raw.reshape(N, -1)
    for c0 in (0, N - cols):
        ref = matmul.gemm_q8_0_int8_f64(rows[c0:c0 + cols].reshape(-1), ref_q, ref_s, cols, K).reshape(M, cols)
        assert matmul.rel_maxnorm(y[:, c0:c0 + cols], ref) < TOL


def test_gemm_residual_f64(dev):
    rng = np.random.default_rng(5)
    M, N, K = 70, 128, 256
    raw = synth.q4_0_weights(rng, N, K)
    x = synth.activations(rng, (M, K))
    rs = rng.standard_normal((M, N))
    y = ops.gemm(ops.GGML_Q4_0, dev_t(raw, dev), dev_t(x, dev), N, K, torch.float64,
                 residual=dev_t(rs, dev)).cpu().numpy()
    ref = matmul.gemm_rows_f64(x, ref_rows(ops.GGML_Q4_0, raw, N, K), rs)
    assert matmul.rel_maxnorm(y, ref) < TOL


# ---- MoE -----------------------------------------------------------------------------------

def test_moe_route_reference_goldens(dev):
    z = np.load(os.path.join(GOLDEN, "moe_golden.npz"))
    logits = dev_t(z["logits"].astype(np.float32), dev)
    bias = dev_t(z["bias"].astype(np.float32), dev)
    idx, w = ops.moe_route(logits, 8, bias, float(z["scale"]))
    np.testing.assert_array_equal(idx.cpu().numpy(), z["ref_idx"])
    assert np.abs(w.cpu().numpy() - z["ref_w"]).max() < 1e-4     # verify_moe_vyb.py:59


@pytest.mark.parametrize("T,E,k", [(1, 256, 8), (37, 256, 8), (5, 16, 4), (300, 64, 6)])
def test_moe_route_oracle(dev, T, E, k):
    rng = np.random.default_rng(T * E)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    idx, w = ops.moe_route(dev_t(logits, dev), k)
    ridx, rw = moe.route_logits(logits.astype(np.float64), k)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    assert np.abs(w.cpu().numpy() - rw).max() < 1e-6


@pytest.mark.parametrize("ldt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("E,k", [(256, 8), (300, 8), (1024, 16), (7, 7)])
def test_moe_route_ties_and_types(dev, ldt, E, k):
    """Logits on a coarse grid (many exact ties: the lower expert id must win), every logit dtype,
    E up to 1024 and k = E."""
    rng = np.random.default_rng(E + k)
    logits = (rng.integers(-6, 7, (5, E)) * 0.5).astype(np.float32)
    zero = logits == 0
    logits[zero] *= rng.choice(np.array([-1.0, 1.0], np.float32), int(zero.sum()))  # -0 ties with +0
    lt = torch.from_numpy(logits).to(ldt)
    idx, w = ops.moe_route(lt.to(dev), k)
    ridx, rw = moe.route_logits(lt.to(torch.float64).numpy(), k)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    assert np.abs(w.cpu().numpy() - rw).max() < 1e-6


def test_moe_route_zero_bias_matches_unbiased(dev):
    """A zero bias (the double-precision selection path) and no bias (the logit path) agree."""
    rng = np.random.default_rng(9)
    logits = dev_t(rng.standard_normal((64, 256)).astype(np.float32), dev)
    i0, w0 = ops.moe_route(logits, 8)
    i1, w1 = ops.moe_route(logits, 8, dev_t(np.zeros(256, np.float32), dev))
    assert torch.equal(i0, i1)
    assert torch.equal(w0, w1)


def moe_case(dev, ty, T, H, I, E, k, seed, shared=True, xdtype=torch.bfloat16):
    rng = np.random.default_rng(seed)
    gate = [weights(ty, rng, I, H) for _ in range(E)]
    up = [weights(ty, rng, I, H) for _ in range(E)]
    down = [weights(ty, rng, H, I) for _ in range(E)]
    sh = (weights(ty, rng, I, H), weights(ty, rng, I, H), weights(ty, rng, H, I)) if shared else None
    x = (rng.standard_normal((T, H)) * 0.5).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    layer = ops.MoeLayer(ty, dev_t(np.concatenate(gate), dev), dev_t(np.concatenate(up), dev),
                         dev_t(np.concatenate(down), dev), H, I, E, k,
                         shared=tuple(dev_t(a, dev) for a in sh) if sh else None)
    xb = torch.from_numpy(x).to(xdtype)
    out, idx, w = layer(xb.to(dev), dev_t(logits, dev), routing=True)
    experts = lambda e: (ref_rows(ty, gate[e], I, H), ref_rows(ty, up[e], I, H), ref_rows(ty, down[e], H, I))
    shared_w = tuple(ref_rows(ty, a, n, kk) for a, n, kk in zip(sh, (I, I, H), (H, H, I))) if sh else None
    x64 = xb.to(torch.float64).numpy()
    if shared_w is None:
        ref, ridx, rw = moe.moe_forward(x64, logits.astype(np.float64), experts,
                                        (np.zeros((1, H)), np.zeros((1, H)), np.zeros((H, 1))), topk=k)
    else:
        ref, ridx, rw = moe.moe_forward(x64, logits.astype(np.float64), experts, shared_w, topk=k)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    assert np.abs(w.cpu().numpy() - rw).max() < 1e-6
    return out.cpu().numpy(), ref


@pytest.mark.parametrize("ty", [ops.GGML_Q4_0, ops.GGML_Q8_0])
@pytest.mark.parametrize("T", [1, 5, 40])
def test_moe_layer_small(dev, ty, T):
    out, ref = moe_case(dev, ty, T, H=256, I=128, E=16, k=4, seed=T + ty)
    assert matmul.rel_maxnorm(out, ref) < TOL


def test_moe_layer_no_shared(dev):
    out, ref = moe_case(dev, ops.GGML_Q4_0, 9, H=128, I=64, E=8, k=2, seed=3, shared=False)
    assert matmul.rel_maxnorm(out, ref) < TOL


@pytest.mark.parametrize("ty", [ops.GGML_Q4_0, ops.GGML_Q8_0])
@pytest.mark.parametrize("T", [1, 7, 16, 17, 40, 48])
@pytest.mark.parametrize("shared", [True, False])
def test_moe_layer_grouped_mfma(dev, ty, T, shared):
    """H and I multiples of 256: the grouped MFMA paths. q4_0: the grouped GEMV at one token, the
    LDS-staged body with 16-row m-tiles while the experts average at most 20 rows (T <= 40 here),
    the register-operand body with 32-row m-tiles above; Q8_0: the register-operand body, 16-row
    m-tiles up to 16 tokens. With 8 experts and top-4 several experts get more rows than one m-tile,
    and the shared expert is one more group over all tokens."""
    out, ref = moe_case(dev, ty, T, H=512, I=256, E=8, k=4, seed=100 + T + ty, shared=shared)
    assert matmul.rel_maxnorm(out, ref) < TOL


@pytest.mark.parametrize("T,rows4", [(2, None), (3, None), (4, None), (7, "64"), (16, "64"), (17, "64"),
                                     (40, "64")])
@pytest.mark.parametrize("shared", [True, False])
def test_moe_layer_q4_four_row_tiles(dev, monkeypatch, T, rows4, shared):
    """q4_0 on 4-row tiles (the LDS-staged body with four stages): by default while the experts hit
    average at most two rows (T <= 4 here), forced above (VYBDQ_MOE_ROWS4), where experts hold
    several 4-row tiles, tiles end mid-tile, and the shared expert spans ceil(T / 4) tiles."""
    if rows4:
        monkeypatch.setenv("VYBDQ_MOE_ROWS4", rows4)
    out, ref = moe_case(dev, ops.GGML_Q4_0, T, H=512, I=256, E=8, k=4, seed=400 + T, shared=shared)
    assert matmul.rel_maxnorm(out, ref) < TOL


@pytest.mark.parametrize("ty,T", [(ops.GGML_Q4_0, 9), (ops.GGML_Q4_0, 40), (ops.GGML_Q8_0, 80)])
@pytest.mark.parametrize("H", [512, 6144])
@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float32])
def test_moe_layer_x_copy_in_bucket_launch(dev, monkeypatch, ty, T, H, xdtype):
    """More than 8 tokens with bf16 / f32 x on the MFMA GEMM: the fp16 copy of x made by workgroups
    1..T of the bucketing launch and made in its own launch (VYBDQ_MOE_XH_SEP=1) give bit-identical
    outputs, both within the oracle's gate (H = 512 and 6144: two and three 8-element chunks per
    thread of the row conversion)."""
    outs = []
    for sep in (None, "1"):
        if sep:
            monkeypatch.setenv("VYBDQ_MOE_XH_SEP", sep)
        out, ref = moe_case(dev, ty, T, H=H, I=256, E=8, k=4, seed=900 + T + H, xdtype=xdtype)
        assert matmul.rel_maxnorm(out, ref) < TOL
        outs.append(out)
    np.testing.assert_array_equal(outs[0], outs[1])


@pytest.mark.parametrize("T,mt", [(7, "1"), (17, "1"), (40, "2")])
def test_moe_layer_q4_register_body(dev, monkeypatch, T, mt):
    """q4_0 through the register-operand body (VYBDQ_MOE_LDS=0) at both m-tile heights."""
    monkeypatch.setenv("VYBDQ_MOE_LDS", "0")
    monkeypatch.setenv("VYBDQ_MOE_MT", mt)
    out, ref = moe_case(dev, ops.GGML_Q4_0, T, H=512, I=256, E=8, k=4, seed=150 + T, shared=True)
    assert matmul.rel_maxnorm(out, ref) < TOL


@pytest.mark.parametrize("ty", [ops.GGML_Q4_0, ops.GGML_Q8_0])
@pytest.mark.parametrize("T,gemv_max_t", [(1, 16), (7, 0), (16, 16), (40, 64), (40, 0)])
def test_moe_layer_expert_paths(dev, ty, T, gemv_max_t):
    """Both grouped expert kernels, forced through VYBDQ_MOE_GEMV_MAX_T: the multi-token GEMV
    (groups of up to 4 tokens per x stage; 40 tokens over 8 experts gives groups of several
    chunks and a 10-chunk shared expert) and the MFMA GEMM (0)."""
    import os
    os.environ["VYBDQ_MOE_GEMV_MAX_T"] = str(gemv_max_t)
    try:
        out, ref = moe_case(dev, ty, T, H=512, I=256, E=8, k=4, seed=200 + T + ty)
    finally:
        os.environ.pop("VYBDQ_MOE_GEMV_MAX_T", None)
    assert matmul.rel_maxnorm(out, ref) < TOL


@pytest.mark.parametrize("ty", [ops.GGML_Q4_0, ops.GGML_Q8_0])
@pytest.mark.parametrize("T", [1, 3, 7, 17])
@pytest.mark.parametrize("cols,grid", [("-1,-1", "1,1"), ("-1,-1", "3,5"), ("-1,-1", "-3,-2"), ("8,32", "0,0")])
def test_moe_gemv_work_splits(dev, monkeypatch, ty, T, cols, grid):
    """The multi-token GEMV's two ways of cutting the work, forced through VYBDQ_MOE_GEMV_COLS /
    VYBDQ_MOE_GEMV_GRID: equal ranges over grids of several sizes (ranges that span groups, a
    grid of one workgroup per CU, multiples of the resident count) and small column blocks."""
    monkeypatch.setenv("VYBDQ_MOE_GEMV_COLS", cols)
    monkeypatch.setenv("VYBDQ_MOE_GEMV_GRID", grid)
    out, ref = moe_case(dev, ty, T, H=512, I=256, E=8, k=4, seed=300 + T + ty)
    assert matmul.rel_maxnorm(out, ref) < TOL


@pytest.mark.parametrize("xdtype", [torch.float32, torch.float16])
def test_moe_layer_grouped_mfma_x_dtypes(dev, xdtype):
    out, ref = moe_case(dev, ops.GGML_Q4_0, 12, H=768, I=512, E=16, k=8, seed=5, xdtype=xdtype)
    assert matmul.rel_maxnorm(out, ref) < TOL


def test_moe_layer_glm_shapes(dev):
    # GLM-5 expert shapes (H 6144, I 2048) with few experts so the float64 oracle stays cheap
    out, ref = moe_case(dev, ops.GGML_Q4_0, 16, H=6144, I=2048, E=4, k=2, seed=7)
    assert matmul.rel_maxnorm(out, ref) < TOL


@pytest.mark.parametrize("ty", [ops.GGML_Q4_0, ops.GGML_Q8_0])
@pytest.mark.parametrize("kind", ["outlier", "offset", "fp16_limit", "tiny", "huge"])
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
@pytest.mark.parametrize("M,N,K", [(200, 256, 4096), (512, 128, 5120)])
def test_gemm_ws_activation_range(dev, ty, kind, xdt, M, N, K):
    """vybdq_gemm_ws converts X to fp16 once, each row scaled by the power of two that brings its
    largest |x| into [2^14, 2^15) (multiplied back in the epilogue and the split-K reduce): bf16 /
    float32 activations of any magnitude neither overflow nor flush to zero."""
    from tests.test_gpu_kquant import _x_pattern
    kinds = ["outlier", "offset", "fp16_limit", "tiny", "huge"]
    rng = np.random.default_rng(77 + 10 * kinds.index(kind) + ty + M)
    raw = weights(ty, rng, N, K)
    x = torch.from_numpy(_x_pattern(kind, rng, M, K)).to(TDT[xdt])
    ws = ops.GemmWorkspace([(M, N, K)], dev, ty)
    y = ops.gemm(ty, dev_t(raw, dev), x.to(dev), N, K, workspace=ws).cpu().numpy()
    ref = matmul.gemm_rows_f64(x.to(torch.float64).numpy(), ref_rows(ty, raw, N, K))
    assert np.all(np.isfinite(y))
    assert matmul.rel_maxnorm(y, ref) < TOL
