"""GPU parity for the GLM-5-style MoE layer at its full workload: hidden 6144, 256 routed experts
plus 1 shared expert, top-8, expert FFN 6144 -> 2048 -> 6144, q4_0 weights (5.4 GB, generated on
the device), T in {1, 16, 256} tokens of bf16 N(0, 1), router logits N(0, 1).

Checks, per T:
- routing of every token against the oracle router: identical expert sets and |dw| < 1e-4
  (native/glm53/verify_moe_vyb.py:54-59);
- the layer output of up to 4 tokens (first, last and two between, so that at T = 256 several
  32-row m-tiles of the matrix-core path are covered) on a 256-column slice of the hidden size,
  against the float64 oracle (oracle.moe semantics, native/glm53/moe_ref.py:68-112), within the
  2e-3 gate of native/glm53/verify_layer0.py:134-139. Only the hit experts' gate/up matrices and
  the slice's down rows are copied back and decoded on the host.
"""

import numpy as np
import pytest
import torch

from oracle import matmul, moe
from vybforge_amd import ops, synth

pytestmark = pytest.mark.gpu

H, I, E, TOPK = 6144, 2048, 256, 8
RB_H = H // 32 * 18      # bytes of one q4_0 row of length H
RB_I = I // 32 * 18      # bytes of one q4_0 row of length I


@pytest.fixture(scope="module")
def glm5_layer(dev):
    gen = torch.Generator(device=dev)
    gen.manual_seed(2025)
    wg = synth.q4_0_weights_torch(gen, E * I, H, dev)
    wu = synth.q4_0_weights_torch(gen, E * I, H, dev)
    wd = synth.q4_0_weights_torch(gen, E * H, I, dev)
    sh = (synth.q4_0_weights_torch(gen, I, H, dev), synth.q4_0_weights_torch(gen, I, H, dev),
          synth.q4_0_weights_torch(gen, H, I, dev))
    layer = ops.MoeLayer(ops.GGML_Q4_0, wg, wu, wd, H, I, E, TOPK, shared=sh)
    yield layer, gen, {}
    del layer, wg, wu, wd, sh
    torch.cuda.empty_cache()


def _expert_bytes(layer, e):
    """Device bytes of expert e's (gate, up, down) q4_0 matrices (e = -1: the shared expert)."""
    if e < 0:
        return layer.shared
    return (layer.w[0][e * I * RB_H:(e + 1) * I * RB_H], layer.w[1][e * I * RB_H:(e + 1) * I * RB_H],
            layer.w[2][e * H * RB_I:(e + 1) * H * RB_I])


def _ffn_slice(layer, e, xt, cols, cache):
    """float64 FFN_e(xt) on the output columns cols: the expert's gate/up rows and the slice's
    down rows are copied back and decoded (float32, exact) on the host."""
    key = (e, int(cols[0]))
    if key not in cache:
        gb, ub, db = _expert_bytes(layer, e)
        c0, nc = int(cols[0]), len(cols)
        g = matmul.q4_0_matrix(gb.cpu().numpy(), I, H)
        u = matmul.q4_0_matrix(ub.cpu().numpy(), I, H)
        d = matmul.q4_0_matrix(db[c0 * RB_I:(c0 + nc) * RB_I].cpu().numpy(), nc, I)
        val = (g, u, d)
        if e >= 0:  # routed experts are used once or twice: decode on demand, keep only the shared
            return moe.ffn_rows(xt, *val)[0]
        cache[key] = val
    return moe.ffn_rows(xt, *cache[key])[0]


@pytest.mark.parametrize("T", [1, 16, 256])
def test_moe_glm5_full_workload(dev, glm5_layer, T):
    layer, gen, cache = glm5_layer
    x = torch.randn(T, H, generator=gen, device=dev).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=gen, device=dev)
    out, idx, w = layer(x, logits, routing=True)
    torch.cuda.synchronize()
    idx, w, out = idx.cpu().numpy(), w.cpu().numpy(), out.cpu().numpy()
    lg = logits.cpu().numpy().astype(np.float64)
    ridx, rw = moe.route_logits(lg, TOPK)
    for t in range(T):
        a = dict(zip(idx[t].tolist(), w[t].tolist()))
        b = dict(zip(ridx[t].tolist(), rw[t].tolist()))
        assert set(a) == set(b), (t, sorted(a), sorted(b))
        assert max(abs(a[k] - b[k]) for k in a) < 1e-4, t
    if T == 256:
        assert len(np.unique(idx)) > 240  # nearly every routed expert is hit: ~257 groups run

    c0 = {1: 0, 16: 2944, 256: 5888}[T]
    cols = np.arange(c0, c0 + 256)
    toks = sorted({0, T // 3, (2 * T) // 3, T - 1})
    x64 = x.to(torch.float64).cpu().numpy()
    ref = np.zeros((len(toks), len(cols)))
    for r, t in enumerate(toks):
        xt = x64[t:t + 1]
        for s in range(TOPK):
            ref[r] += rw[t, s] * _ffn_slice(layer, int(ridx[t, s]), xt, cols, cache)
        ref[r] += _ffn_slice(layer, -1, xt, cols, cache)
    got = out[toks][:, cols]
    assert matmul.rel_maxnorm(got, ref) < matmul.TOL, (T, matmul.rel_maxnorm(got, ref))
