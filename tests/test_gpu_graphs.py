"""HIP-graph capture of the hot-path entry points: each is captured once and replayed several
times with eager work of its own between the replays; every replay equals the eager result bit
for bit (no entry point records a memset or depends on state a replay does not restore)."""

import numpy as np
import pytest
import torch

from tests.test_gpu_gemm_moe import weights
from vybforge_amd import ops, synth

pytestmark = pytest.mark.gpu


def dev_t(a, dev):
    return torch.from_numpy(np.array(a, copy=True)).to(dev)


def check_replays(fn, replays=4):
    eager = [t.clone() for t in fn()]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = fn()
    for i in range(replays):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {i}"
        fn()  # eager call between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("T", [1, 16, 80])
def test_moe_layer_graph(dev, T):
    rng = np.random.default_rng(900 + T)
    H, I, E, k = 512, 256, 8, 4
    ty = ops.GGML_Q4_0
    gate = np.concatenate([weights(ty, rng, I, H) for _ in range(E)])
    up = np.concatenate([weights(ty, rng, I, H) for _ in range(E)])
    down = np.concatenate([weights(ty, rng, H, I) for _ in range(E)])
    sh = tuple(dev_t(weights(ty, rng, n, kk), dev) for n, kk in ((I, H), (I, H), (H, I)))
    layer = ops.MoeLayer(ty, dev_t(gate, dev), dev_t(up, dev), dev_t(down, dev), H, I, E, k, shared=sh)
    x = torch.from_numpy((rng.standard_normal((T, H)) * 0.5).astype(np.float32)).to(torch.bfloat16).to(dev)
    logits = dev_t(rng.standard_normal((T, E)).astype(np.float32), dev)
    out = torch.empty((T, H), dtype=torch.float32, device=dev)
    check_replays(lambda: (layer(x, logits, out=out),))


def test_decode_gemv_graph(dev):
    rng = np.random.default_rng(910)
    K = 2560
    ws = [(dev_t(synth.q4_0_weights(rng, n, K), dev), torch.empty(n, dtype=torch.float16, device=dev), n)
          for n in (512, 128, 128)]
    x = dev_t(rng.standard_normal(K).astype(np.float16), dev)
    wo = dev_t(synth.q4_0_weights(rng, 256, K), dev)
    yo = torch.empty((1, 256), dtype=torch.float32, device=dev)

    def fn():
        ops.gemv_q4_0_seg3(x, K, ws)
        ops.gemv(ops.GGML_Q4_0, wo, x, 256, K, out=yo)
        return tuple(w[1] for w in ws) + (yo,)
    check_replays(fn)


def test_prefill_gemm_and_router_graph(dev):
    rng = np.random.default_rng(920)
    M, N, K = 128, 256, 512
    W = dev_t(weights(ops.GGML_Q8_0, rng, N, K), dev)
    X = dev_t(rng.standard_normal((M, K)).astype(np.float32), dev).to(torch.bfloat16)
    Y = torch.empty((M, N), dtype=torch.float32, device=dev)
    xr = dev_t(rng.standard_normal((4, 256)).astype(np.float32), dev)
    wr = dev_t((rng.standard_normal((16, 256)) * 0.05).astype(np.float32), dev).to(torch.bfloat16)

    def fn():
        ops.gemm(ops.GGML_Q8_0, W, X, N, K, out=Y)
        return (Y, ops.router_logits(xr, wr))
    check_replays(fn)
