"""GPU parity of the persistent GEMV chain: dependent stages (stage s reads stage s-1's
output) against the fp64 oracle on the exact inputs each stage saw, multi-segment stages,
mixed dtypes, residual, Q8_0, repeated calls and the workspace protocol."""

import numpy as np
import pytest
import torch

from oracle import matmul
from vybforge_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu
TOL = matmul.TOL


def dev_bytes(a, dev):
    return torch.from_numpy(np.array(a, copy=True)).to(dev)


def gate16(y, ref):
    y = np.asarray(y, np.float64)
    half_ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 11)
    return float(np.maximum(np.abs(y - ref) - half_ulp, 0).max() / np.abs(ref).max())


def test_chain_dependent_stages_q4_0(dev):
    rng = np.random.default_rng(11)
    f16 = torch.float16
    # stage 0: x0[2560] -> (y0a[1024] | y0b[1536] | y0c[512]); stage 1: y0 (3072 as one buffer)...
    # build a dependent chain: each stage's X is the previous stage's Y
    dims = [2560, 3072, 4096, 2560, 9728, 2560]
    xs = [torch.from_numpy(synth.activations(rng, (dims[0],))).to(f16).to(dev)]
    raws, Ws, Ys, pbs = [], [], [], []
    for s in range(len(dims) - 1):
        K, N = dims[s], dims[s + 1]
        raw = synth.q4_0_weights(rng, N, K)
        W = dev_bytes(raw, dev)
        Y = torch.empty(N, dtype=f16, device=dev)
        raws.append(raw); Ws.append(W); Ys.append(Y)
        pbs.append(ops.pblock(xs[-1], K, [(W, Y, N)]))
        xs.append(Y)
    ch = ops.GemvChain(ops.GGML_Q4_0, pbs, dev)
    for rep in range(3):
        for Y in Ys:
            Y.fill_(float("nan"))
        ch()
        assert ch.status() == 0, _lib.last_error()
        for s in range(len(Ws)):
            K, N = dims[s], dims[s + 1]
            x_in = xs[s].to(torch.float64).cpu().numpy()
            ref = matmul.gemv_q4_0_f64(raws[s], x_in, N, K)[0]
            y = Ys[s].to(torch.float64).cpu().numpy()
            assert gate16(y, ref) < TOL, (rep, s)
    assert int(ch.ws.abs().sum()) == 0     # counters reset by the last workgroup


def test_chain_segments_dtypes_residual(dev):
    rng = np.random.default_rng(12)
    K = 2048
    x = torch.from_numpy(synth.activations(rng, (K,))).to(dev)          # f32 x
    shapes = [777, 64, 1500]
    raws = [synth.q4_0_weights(rng, n, K) for n in shapes]
    Ws = [dev_bytes(r, dev) for r in raws]
    Y0 = torch.empty(shapes[0], dtype=torch.float64, device=dev)
    RS = torch.from_numpy(rng.standard_normal(shapes[0])).to(dev)
    Y1 = torch.empty(shapes[1], dtype=torch.float32, device=dev)
    Y2 = torch.empty(shapes[2], dtype=torch.bfloat16, device=dev)
    pb0 = ops.pblock(x, K, [(Ws[0], Y0, shapes[0]), (Ws[1], Y1, shapes[1]), (Ws[2], Y2, shapes[2])],
                     residual=RS)
    # a second stage reading the first stage's f32 segment
    raw_b = synth.q4_0_weights(rng, 256, 64)
    Yb = torch.empty(256, dtype=torch.float32, device=dev)
    pb1 = ops.pblock(Y1, 64, [(dev_bytes(raw_b, dev), Yb, 256)])
    ch = ops.GemvChain(ops.GGML_Q4_0, [pb0, pb1], dev)
    ch()
    assert ch.status() == 0, _lib.last_error()
    x64 = x.to(torch.float64).cpu().numpy()
    ref0 = matmul.gemv_q4_0_f64(raws[0], x64, shapes[0], K, residual=RS.cpu().numpy())[0]
    assert matmul.rel_maxnorm(Y0.cpu().numpy(), ref0) < TOL
    ref1 = matmul.gemv_q4_0_f64(raws[1], x64, shapes[1], K)[0]
    assert matmul.rel_maxnorm(Y1.cpu().numpy(), ref1) < TOL
    ref2 = matmul.gemv_q4_0_f64(raws[2], x64, shapes[2], K)[0]
    y2 = Y2.to(torch.float64).cpu().numpy()
    half_ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref2), 1e-30))) - 8)
    assert float(np.maximum(np.abs(y2 - ref2) - half_ulp, 0).max() / np.abs(ref2).max()) < TOL
    refb = matmul.gemv_q4_0_f64(raw_b, Y1.to(torch.float64).cpu().numpy(), 256, 64)[0]
    assert matmul.rel_maxnorm(Yb.cpu().numpy(), refb) < TOL


def test_chain_q8_0_and_interleaved(dev):
    rng = np.random.default_rng(13)
    K, N = 5120, 2048
    raw8 = synth.q8_0_weights(rng, N, K)
    x = torch.from_numpy(synth.activations(rng, (K,))).to(torch.bfloat16).to(dev)
    Y = torch.empty(N, dtype=torch.float32, device=dev)
    ch = ops.GemvChain(ops.GGML_Q8_0, [ops.pblock(x, K, [(dev_bytes(raw8, dev), Y, N)])], dev)
    ch()
    assert ch.status() == 0
    ref = matmul.gemv_q8_0_f64(raw8, x.to(torch.float64).cpu().numpy(), N, K)[0]
    assert matmul.rel_maxnorm(Y.cpu().numpy(), ref) < TOL
    raw4 = synth.q4_0_weights(rng, 300, 1024)
    x4 = torch.from_numpy(synth.activations(rng, (1024,))).to(dev)
    Y4 = torch.empty(300, dtype=torch.float32, device=dev)
    ch4 = ops.GemvChain(ops.GGML_Q4_0, [ops.pblock(x4, 1024, [(dev_bytes(raw4, dev), Y4, 300)],
                                                   order=ops.Q4_INTERLEAVED)], dev)
    ch4()
    ref4 = matmul.gemv_q4_0_f64(raw4, x4.cpu().numpy().astype(np.float64), 300, 1024, order=1)[0]
    assert matmul.rel_maxnorm(Y4.cpu().numpy(), ref4) < TOL


def test_chain_invalid_stage_reports(dev):
    rng = np.random.default_rng(14)
    raw = synth.q4_0_weights(rng, 64, 96)           # K % 64 != 0: not a chain shape
    x = torch.zeros(96, dtype=torch.float32, device=dev)
    Y = torch.zeros(64, dtype=torch.float32, device=dev)
    pb = ops.pblock(x, 96, [(dev_bytes(raw, dev), Y, 64)])
    ch = ops.GemvChain(ops.GGML_Q4_0, [pb], dev)
    ch.max_k = 128
    ch()
    assert ch.status() == _lib.ERR_SHAPE
    assert "invalid" in _lib.last_error()


@pytest.mark.parametrize("kind", ["outlier", "fp16_limit", "tiny"])
def test_chain_activation_range(dev, kind):
    """The chain's x stage scales each block like the one-shot GEMV: f32 x of any magnitude."""
    from tests.test_gpu_kquant import _x_pattern
    N, K = 512, 2048
    rng = np.random.default_rng(len(kind))
    raw = synth.q4_0_weights(rng, N, K)
    x = torch.from_numpy(_x_pattern(kind, rng, 1, K)[0]).to(dev)
    W = torch.from_numpy(raw).to(dev)
    y = torch.empty(N, dtype=torch.float32, device=dev)
    chain = ops.GemvChain(ops.GGML_Q4_0, [ops.pblock(x, K, [(W, y, N)])], dev)
    chain()
    assert chain.status() == 0
    ref = matmul.gemv_q4_0_f64(raw, x.cpu().numpy().astype(np.float64), N, K)[0]
    assert np.all(np.isfinite(y.cpu().numpy()))
    assert matmul.rel_maxnorm(y.cpu().numpy(), ref) < matmul.TOL


@pytest.mark.parametrize("ty", [ops.GGML_Q4_K, ops.GGML_Q5_K, ops.GGML_Q6_K, ops.GGML_IQ2_S])
def test_chain_superblock_types(dev, ty):
    """Two dependent stages of a super-block type (the second reads the first's fp16 output)."""
    from tests.test_gpu_kquant import matrix_ref
    rng = np.random.default_rng(15 + ty)
    K0, N0, N1 = 2560, 1024, 768
    raw0, raw1 = synth.kquant_weights(rng, ty, N0, K0), synth.kquant_weights(rng, ty, N1, N0)
    x = torch.from_numpy(synth.activations(rng, (K0,))).to(torch.float16).to(dev)
    Y0 = torch.empty(N0, dtype=torch.float16, device=dev)
    Y1 = torch.empty(N1, dtype=torch.float32, device=dev)
    ch = ops.GemvChain(ty, [ops.pblock(x, K0, [(dev_bytes(raw0, dev), Y0, N0)]),
                            ops.pblock(Y0, N0, [(dev_bytes(raw1, dev), Y1, N1)])], dev)
    ch()
    assert ch.status() == 0, _lib.last_error()
    ref0 = matrix_ref(ty, raw0, N0, K0) @ x.to(torch.float64).cpu().numpy()
    assert gate16(Y0.to(torch.float64).cpu().numpy(), ref0) < TOL
    ref1 = matrix_ref(ty, raw1, N1, N0) @ Y0.to(torch.float64).cpu().numpy()
    assert matmul.rel_maxnorm(Y1.cpu().numpy(), ref1) < TOL


def test_chain_decode_stack_shapes(dev):
    """Two layers of the decode stack's stages (q|k|v, o, gate|up, down; fp16 x and y) as the
    benchmark runs them, each stage on its own N(0, 1) input (chained raw q4_0 GEMVs grow past the
    fp16 range: the weights' -8 d sum(x) term compounds; stage-to-stage data flow is tested above):
    lane groups of 16 (q|k|v), 32 (o, down) and 4 (gate|up, 19456 rows: 16 rows per tile)."""
    H, Q, KV, I = 2560, 4096, 1024, 9728
    rng = np.random.default_rng(16)
    f16 = torch.float16
    xin = lambda k: torch.from_numpy(synth.activations(rng, (k,))).to(f16).to(dev)
    shapes = dict(q=(Q, H), k=(KV, H), v=(KV, H), o=(H, Q), gate=(I, H), up=(I, H), down=(H, I))  # (rows, K)
    pbs, checks = [], []
    for _ in range(2):
        W = {n: synth.q4_0_weights(rng, r, k) for n, (r, k) in shapes.items()}
        Wd = {n: dev_bytes(a, dev) for n, a in W.items()}
        y = {n: torch.empty(r, dtype=f16, device=dev) for n, (r, _) in shapes.items()}
        xs = dict(attn=xin(H), o=xin(Q), mlp=xin(H), down=xin(I))
        pbs.append(ops.pblock(xs["attn"], H, [(Wd["q"], y["q"], Q), (Wd["k"], y["k"], KV), (Wd["v"], y["v"], KV)]))
        pbs.append(ops.pblock(xs["o"], Q, [(Wd["o"], y["o"], H)]))
        pbs.append(ops.pblock(xs["mlp"], H, [(Wd["gate"], y["gate"], I), (Wd["up"], y["up"], I)]))
        pbs.append(ops.pblock(xs["down"], I, [(Wd["down"], y["down"], H)]))
        checks.append((W, y, xs))
    ch = ops.GemvChain(ops.GGML_Q4_0, pbs, dev)
    ch()
    assert ch.status() == 0, _lib.last_error()
    for W, y, xs in checks:
        x64 = lambda t: t.to(torch.float64).cpu().numpy()
        for n, src in (("q", xs["attn"]), ("k", xs["attn"]), ("v", xs["attn"]), ("o", xs["o"]), ("gate", xs["mlp"]),
                       ("up", xs["mlp"]), ("down", xs["down"])):
            r, k = shapes[n]
            ref = matmul.gemv_q4_0_f64(W[n], x64(src), r, k)[0]
            assert gate16(x64(y[n]), ref) < TOL, n
    assert int(ch.ws.abs().sum()) == 0


def test_chain_stage_larger_than_the_held_registers(dev):
    """30000 rows of K = 4096: more tiles than row-owning waves (a second round of tiles) and more
    units per lane than the registers hold (the rest streamed after the wait); then a dependent
    stage reading the first 16384 of its outputs."""
    rng = np.random.default_rng(17)
    N0, K0, N1, K1 = 30000, 4096, 256, 16384
    raw0 = synth.q4_0_weights(rng, N0, K0)
    raw1 = synth.q4_0_weights(rng, N1, K1)
    x = torch.from_numpy(synth.activations(rng, (K0,))).to(dev)
    Y0 = torch.empty(N0, dtype=torch.float32, device=dev)
    Y1 = torch.empty(N1, dtype=torch.float32, device=dev)
    ch = ops.GemvChain(ops.GGML_Q4_0, [ops.pblock(x, K0, [(dev_bytes(raw0, dev), Y0, N0)]),
                                       ops.pblock(Y0, K1, [(dev_bytes(raw1, dev), Y1, N1)])], dev)
    ch()
    assert ch.status() == 0, _lib.last_error()
    ref0 = matmul.gemv_q4_0_f64(raw0, x.to(torch.float64).cpu().numpy(), N0, K0)[0]
    assert matmul.rel_maxnorm(Y0.cpu().numpy(), ref0) < TOL
    ref1 = matmul.gemv_q4_0_f64(raw1, Y0.to(torch.float64).cpu().numpy()[:K1], N1, K1)[0]
    assert matmul.rel_maxnorm(Y1.cpu().numpy(), ref1) < TOL
