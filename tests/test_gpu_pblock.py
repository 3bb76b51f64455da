"""GPU parity for vybdq_launch_pblock: the reference's own parameter blocks (little-endian int64 words
written to device memory exactly as set_gemv / set_gemm write them, native/host/ridge_decode.vyb:264-275)
launched through the C-ABI, against the float64 oracle; the words are read by the kernels when they
run (a captured graph replays with rewritten blocks); invalid blocks are reported, not computed."""

import numpy as np
import pytest
import torch

from oracle import iquants, kquants, matmul
from tests.test_gpu_gguf import gate, to_dev
from vybforge_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu

TYPES = [ops.GGML_Q4_0, ops.GGML_Q8_0, ops.GGML_Q4_K, ops.GGML_Q5_K, ops.GGML_Q6_K, ops.GGML_IQ2_S]


def weights(ty, rng, N, K):
    if ty == ops.GGML_Q4_0:
        return synth.q4_0_weights(rng, N, K)
    if ty == ops.GGML_Q8_0:
        return synth.q8_0_weights(rng, N, K)
    return synth.kquant_weights(rng, ty, N, K)


def rows(ty, raw, N, K):
    if ty == ops.GGML_Q4_0:
        return matmul.q4_0_matrix(raw, N, K)
    if ty == ops.GGML_Q8_0:
        return matmul.q8_0_matrix(raw, N, K)
    if ty == ops.GGML_IQ2_S:
        return iquants.dequant_iq2_s(raw).reshape(N, K)
    return kquants.DEQUANT[ty](raw).reshape(N, K)


def set_gemv(words, W, X, Y, N, K, YE, RS, G, segs=()):
    """The reference's set_gemv (ridge_decode.vyb:264-270), plus optional segments 2 and 3."""
    words[:] = 0
    words[0], words[1], words[2], words[3], words[4], words[5], words[6] = W, X, Y, 1, N, K, YE
    words[10], words[14] = 8, 8
    for (w, n, y, ye), (iw, ins, iy, iye) in zip(segs, [(7, 8, 9, 10), (11, 12, 13, 14)]):
        words[iw], words[ins], words[iy], words[iye] = w, n, y, ye
    words[15], words[16] = RS, G


def set_gemm(words, W, X, Y, S, N, K, LDY, RS, G, BM):
    """The reference's set_gemm (ridge_decode.vyb:272-275)."""
    words[:] = 0
    words[0:10] = [W, X, Y, S, N, K, LDY, RS, G, (S + BM - 1) // BM]


def launch(kind, pb_dev):
    _lib.call("vybdq_launch_pblock", kind, pb_dev.data_ptr(), torch.cuda.current_stream().cuda_stream)


def status():
    return _lib.lib.vybdq_pblock_status()


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("N,K,YE", [(9728, 2560, 4), (300, 5120, 8), (2560, 9728, 4), (64, 17408, 8)])
def test_pblock_gemv(dev, ty, N, K, YE):
    rng = np.random.default_rng(N + K + ty)
    raw = weights(ty, rng, N, K)
    x = synth.activations(rng, (K,))
    W, X = to_dev(raw, dev), to_dev(x, dev)
    ydt = torch.float32 if YE == 4 else torch.float64
    Y = torch.full((N,), float("nan"), dtype=ydt, device=dev)
    rs = synth.activations(rng, (N,)).astype(np.float64)
    RS = to_dev(rs, dev)
    words = np.zeros(32, np.int64)
    set_gemv(words, W.data_ptr(), X.data_ptr(), Y.data_ptr(), N, K, YE, RS.data_ptr() if YE != 4 else 0, (N + 15) // 16)
    pb = to_dev(words, dev)
    launch(_lib.PB_GEMV + ty, pb)
    assert status() == 0, _lib.last_error()
    ref = matmul.gemm_rows_f64(x.reshape(1, K), rows(ty, raw, N, K), rs.reshape(1, N) if YE != 4 else None)[0]
    assert gate(Y.cpu().numpy(), ref) < matmul.TOL


@pytest.mark.parametrize("ty", [ops.GGML_Q4_0, ops.GGML_Q4_K, ops.GGML_Q6_K])
def test_pblock_gemv_segments(dev, ty):
    """q|k|v as three segments of one block (W2/NS2/Y2/YE2 @56-80, W3/NS3/Y3/YE3 @88-112)."""
    K, shapes = 2560, [4096, 1024, 1024]
    rng = np.random.default_rng(ty)
    raws = [weights(ty, rng, n, K) for n in shapes]
    x = synth.activations(rng, (K,))
    Ws = [to_dev(r, dev) for r in raws]
    X = to_dev(x, dev)
    Ys = [torch.empty(n, dtype=torch.float32 if i != 1 else torch.float64, device=dev) for i, n in enumerate(shapes)]
    words = np.zeros(32, np.int64)
    set_gemv(words, Ws[0].data_ptr(), X.data_ptr(), Ys[0].data_ptr(), shapes[0], K, 4, 0, 0,
             segs=[(Ws[1].data_ptr(), shapes[1], Ys[1].data_ptr(), 8), (Ws[2].data_ptr(), shapes[2], Ys[2].data_ptr(), 4)])
    pb = to_dev(words, dev)
    launch(_lib.PB_GEMV + ty, pb)
    assert status() == 0, _lib.last_error()
    for r, y, n in zip(raws, Ys, shapes):
        ref = matmul.gemm_rows_f64(x.reshape(1, K), rows(ty, r, n, K))[0]
        assert gate(y.cpu().numpy(), ref) < matmul.TOL


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("S,N,K", [(300, 256, 1024), (64, 128, 2560), (512, 192, 5120), (7, 64, 256)])
@pytest.mark.parametrize("xh", [False, True])
def test_pblock_gemm(dev, ty, S, N, K, xh):
    """set_gemm blocks: LDY < 0 (f32 Y of row stride -LDY, RS ignored) and LDY > 0 (f64 Y with
    the f64 residual), X float32 (VYBDQ_PB_GEMM) or fp16 (VYBDQ_PB_GEMM_XH)."""
    if ty >= 12 and N % 64:
        pytest.skip("super-block types need N % 64 == 0")
    rng = np.random.default_rng(S + N + K + ty + xh)
    raw = weights(ty, rng, N, K)
    x = synth.activations(rng, (S, K))
    xt = torch.from_numpy(x).to(torch.float16 if xh else torch.float32)
    W, X = to_dev(raw, dev), xt.to(dev)
    x64 = xt.to(torch.float64).numpy()
    wr = rows(ty, raw, N, K)
    kind = (_lib.PB_GEMM_XH if xh else _lib.PB_GEMM) + ty
    ldy = N + 32
    # f32 output, row stride ldy: LDY = -ldy; a RS word that must be ignored
    Y32 = torch.full((S, ldy), 7.0, dtype=torch.float32, device=dev)
    junk = torch.full((S, ldy), 1e6, dtype=torch.float32, device=dev)
    words = np.zeros(32, np.int64)
    set_gemm(words, W.data_ptr(), X.data_ptr(), Y32.data_ptr(), S, N, K, -ldy, junk.data_ptr(), 0, 64)
    pb = to_dev(words, dev)
    launch(kind, pb)
    assert status() == 0, _lib.last_error()
    got = Y32.cpu().numpy()
    assert matmul.rel_maxnorm(got[:, :N], matmul.gemm_rows_f64(x64, wr)) < matmul.TOL
    assert np.all(got[:, N:] == 7.0)
    # f64 output with the f64 residual
    rs = synth.activations(rng, (S, N)).astype(np.float64)
    RS = to_dev(rs, dev)
    Y64 = torch.empty((S, N), dtype=torch.float64, device=dev)
    set_gemm(words, W.data_ptr(), X.data_ptr(), Y64.data_ptr(), S, N, K, N, RS.data_ptr(), 0, 64)
    pb2 = to_dev(words, dev)
    launch(kind, pb2)
    assert status() == 0, _lib.last_error()
    assert matmul.rel_maxnorm(Y64.cpu().numpy(), matmul.gemm_rows_f64(x64, wr, rs)) < matmul.TOL


@pytest.mark.parametrize("kind,ty", [(_lib.PB_GEMV, ops.GGML_Q4_0), (_lib.PB_GEMM, ops.GGML_Q8_0),
                                     (_lib.PB_GEMM, ops.GGML_Q4_K)])
def test_pblock_rewritten_between_graph_replays(dev, kind, ty):
    """The block is rewritten on the device between replays of a captured launch (as the reference's
    put_ia does): every replay follows the words of that moment (other weights, other output)."""
    rng = np.random.default_rng(kind + ty)
    N, K, S = 256, 1024, (1 if kind == _lib.PB_GEMV else 100)
    raws = [weights(ty, rng, N, K) for _ in range(3)]
    Ws = [to_dev(r, dev) for r in raws]
    x = synth.activations(rng, (S, K))
    X = to_dev(x, dev)
    Ys = [torch.zeros((S, N), dtype=torch.float32, device=dev) for _ in range(3)]

    def words_for(i):
        w = np.zeros(32, np.int64)
        if kind == _lib.PB_GEMV:
            set_gemv(w, Ws[i].data_ptr(), X.data_ptr(), Ys[i].data_ptr(), N, K, 4, 0, 0)
        else:
            set_gemm(w, Ws[i].data_ptr(), X.data_ptr(), Ys[i].data_ptr(), S, N, K, -N, 0, 0, 64)
        return torch.from_numpy(w)
    pb = words_for(0).to(dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        launch(kind + ty, pb)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch(kind + ty, pb)
    for i in (1, 2, 0):
        Ys[i].zero_()
        pb.copy_(words_for(i))  # the block's words change on the device, the graph does not
        g.replay()
        torch.cuda.synchronize()
        ref = matmul.gemm_rows_f64(x, rows(ty, raws[i], N, K))
        assert matmul.rel_maxnorm(Ys[i].cpu().numpy(), ref) < matmul.TOL, i
    assert status() == 0, _lib.last_error()


def test_pblock_invalid_blocks_are_reported(dev):
    """Blocks a kernel cannot run (M != 1 for a GEMV, K not a multiple of 256 or a null W for a
    GEMM) write nothing and are reported by the status call; the device keeps working."""
    rng = np.random.default_rng(5)
    N, K = 128, 512
    W = to_dev(synth.q4_0_weights(rng, N, K), dev)
    X = to_dev(synth.activations(rng, (4, K)), dev)
    Y = torch.full((4, N), 3.0, device=dev)
    assert status() == 0
    words = np.zeros(32, np.int64)
    set_gemv(words, W.data_ptr(), X.data_ptr(), Y.data_ptr(), N, K, 4, 0, 0)
    words[3] = 2  # M = 2
    launch(_lib.PB_GEMV + ops.GGML_Q4_0, to_dev(words, dev))
    assert status() == _lib.ERR_SHAPE and "GEMV" in _lib.last_error()
    assert status() == 0  # cleared
    set_gemm(words, W.data_ptr(), X.data_ptr(), Y.data_ptr(), 4, N, 320, -N, 0, 0, 64)  # K % 256 != 0
    launch(_lib.PB_GEMM + ops.GGML_Q4_0, to_dev(words, dev))
    assert status() == _lib.ERR_SHAPE and "GEMM" in _lib.last_error()
    set_gemm(words, 0, X.data_ptr(), Y.data_ptr(), 4, N, K, -N, 0, 0, 64)  # null W
    launch(_lib.PB_GEMM + ops.GGML_Q4_K, to_dev(words, dev))
    assert status() == _lib.ERR_SHAPE
    assert torch.all(Y == 3.0)
    # host-side argument errors
    assert _lib.lib.vybdq_launch_pblock(0x500 + 2, 8, 0) == _lib.ERR_ARG
    assert _lib.lib.vybdq_launch_pblock(_lib.PB_GEMV + 3, 8, 0) == _lib.ERR_ARG
    assert _lib.lib.vybdq_launch_pblock(_lib.PB_GEMV + 2, 12, 0) == _lib.ERR_ALIGN
