"""The allocation-free MoE entry point (vybdq_moe_forward_noalloc) against vybdq_moe_forward with a
caller workspace: the same routing and bit-identical outputs, on two calls in a row of which the
second is smaller (the scratch keeps the first call's contents), on both grouped expert kernels
(the grouped GEMV: q4_0 at one token, Q8_0 up to 64 tokens; the matrix-core GEMM above), and the
size limit rejected before any launch."""

import numpy as np
import pytest
import torch

from oracle import matmul, moe
from vybforge_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu

H, I, E, K = 512, 256, 8, 4


def _layer(dev, ty, seed):
    rng = np.random.default_rng(seed)
    mk = synth.q4_0_weights if ty == ops.GGML_Q4_0 else synth.q8_0_weights
    t = lambda a: torch.from_numpy(a).to(dev)
    gate = np.concatenate([mk(rng, I, H) for _ in range(E)])
    up = np.concatenate([mk(rng, I, H) for _ in range(E)])
    down = np.concatenate([mk(rng, H, I) for _ in range(E)])
    sh = (mk(rng, I, H), mk(rng, I, H), mk(rng, H, I))
    layer = ops.MoeLayer(ty, t(gate), t(up), t(down), H, I, E, K, shared=tuple(t(a) for a in sh))
    return layer, (gate, up, down, sh)


def _ref(ty, host, x, logits):
    gate, up, down, sh = host
    dq = (lambda raw, n, k: matmul.q4_0_matrix(raw, n, k)) if ty == ops.GGML_Q4_0 else matmul.q8_0_matrix
    rb_h, rb_i = ops.row_bytes(ty, H), ops.row_bytes(ty, I)
    experts = lambda e: (dq(gate[e * I * rb_h:(e + 1) * I * rb_h], I, H), dq(up[e * I * rb_h:(e + 1) * I * rb_h], I, H),
                         dq(down[e * H * rb_i:(e + 1) * H * rb_i], H, I))
    shared = (dq(sh[0], I, H), dq(sh[1], I, H), dq(sh[2], H, I))
    return moe.moe_forward(x, logits, experts, shared, topk=K)


@pytest.mark.parametrize("ty", [ops.GGML_Q4_0, ops.GGML_Q8_0])
@pytest.mark.parametrize("Ts", [(16, 5), (96, 70), (80, 3), (16, 1), (4, 1)])
def test_moe_noalloc_matches_workspace_entry(dev, ty, Ts):
    layer, host = _layer(dev, ty, seed=sum(Ts) + ty)
    gen = torch.Generator(device=dev)
    gen.manual_seed(Ts[0])
    for T in Ts:  # two calls in a row, the second smaller
        x = torch.randn(T, H, generator=gen, device=dev).to(torch.bfloat16)
        logits = torch.randn(T, E, generator=gen, device=dev)
        y_na, i_na, w_na = layer(x, logits, routing=True, noalloc=True)
        y_ws, i_ws, w_ws = layer(x, logits, routing=True)
        torch.cuda.synchronize()
        assert torch.equal(i_na, i_ws) and torch.equal(w_na, w_ws), T
        assert torch.equal(y_na, y_ws), T
        ref, ridx, _ = _ref(ty, host, x.to(torch.float64).cpu().numpy(), logits.to(torch.float64).cpu().numpy())
        np.testing.assert_array_equal(i_na.cpu().numpy(), ridx)
        assert matmul.rel_maxnorm(y_na.cpu().numpy(), ref) < matmul.TOL, T


def test_moe_noalloc_size_limit():
    # GLM-5 shapes at 4096 tokens need far more than the scratch: rejected before any launch
    need = _lib.lib.vybdq_moe_workspace_size(4096, 6144, 2048, 256, 8)
    assert need > _lib.MOE_NOALLOC_MAX_BYTES
    rc = _lib.lib.vybdq_moe_forward_noalloc(2, 16, 2, 16, 0, 0, 16, 16, 16, 0, 0, 0, 16, 0, 0, 0, 4096, 6144, 2048,
                                            256, 8, 2.5, 10.0, 0)
    assert rc == _lib.ERR_WORKSPACE
    assert "scratch" in _lib.last_error()
