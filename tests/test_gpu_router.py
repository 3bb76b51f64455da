"""Router logits (vybdq_router_logits, float64 accumulation) against the oracle's ordered float64
sum, and end to end against the reference's own routing of its GLM layer-0 fixture
(native/glm53/prep: y, the bf16 gate weight, the selection bias, ref_idx / ref_w)."""

import numpy as np
import pytest
import torch

from oracle import moe
from tests.conftest import GOLDEN
from vybforge_amd import ops, synth

pytestmark = pytest.mark.gpu


def bf16_from_bits(bits):
    return torch.from_numpy(bits.astype(np.int16).view(np.int16)).view(torch.bfloat16)


@pytest.mark.parametrize("T,E,H", [(1, 256, 6144), (5, 288, 4096), (3, 7, 160), (2, 9, 2080)])
@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float16, torch.float32])
def test_router_logits_bit_exact(dev, T, E, H, wdt):
    rng = np.random.default_rng(T * E + H)
    x = torch.from_numpy(rng.standard_normal((T, H)))  # float64 activations: products round
    w = torch.from_numpy((rng.standard_normal((E, H)) * 0.02).astype(np.float32)).to(wdt)
    got = ops.router_logits(x.to(dev), w.to(dev)).cpu().numpy()
    want = moe.router_logits_f64(x.numpy(), w.to(torch.float64).numpy())
    np.testing.assert_array_equal(got, want)
    x32 = x.to(torch.float32)  # and float32 activations (every product exact)
    got = ops.router_logits(x32.to(dev), w.to(dev)).cpu().numpy()
    want = moe.router_logits_f64(x32.to(torch.float64).numpy(), w.to(torch.float64).numpy())
    np.testing.assert_array_equal(got, want)


def test_router_end_to_end_reference_routing(dev):
    d = np.load(f"{GOLDEN}/router_golden.npz")
    g = np.load(f"{GOLDEN}/moe_golden.npz")
    y = torch.from_numpy(d["y"]).to(dev)
    w = bf16_from_bits(d["gate_bf16"]).to(dev)
    logits = ops.router_logits(y, w)
    # the float64 logits agree with the plain float64 matmul to rounding
    np.testing.assert_allclose(logits.cpu().numpy(), g["logits"], rtol=0, atol=1e-12)
    idx, wts = ops.moe_route(logits, 8, torch.from_numpy(g["bias"]).to(dev), float(g["scale"]))
    np.testing.assert_array_equal(idx.cpu().numpy(), g["ref_idx"])
    assert np.abs(wts.cpu().numpy() - g["ref_w"]).max() < 1e-6


def test_layer_one_token_router_reference_routing(dev):
    """The router inside the q4_0 MoE layer at one token with a selection bias (its workgroup form:
    the sigmoids of all 288 experts over four waves, the selection on wave 0) reproduces the
    reference's routing of each golden token."""
    g = np.load(f"{GOLDEN}/moe_golden.npz")
    E, k, H, I = g["logits"].shape[1], 8, 256, 256
    rng = np.random.default_rng(3)
    w = lambda n, kk: torch.from_numpy(synth.q4_0_weights(rng, n, kk)).to(dev)
    gate = torch.cat([w(I, H) for _ in range(E)])
    up = torch.cat([w(I, H) for _ in range(E)])
    down = torch.cat([w(H, I) for _ in range(E)])
    layer = ops.MoeLayer(ops.GGML_Q4_0, gate, up, down, H, I, E, k, scale=float(g["scale"]),
                         bias=torch.from_numpy(g["bias"]).to(dev))
    x = torch.randn(1, H, device=dev).to(torch.bfloat16)
    for t in range(g["logits"].shape[0]):
        logits = torch.from_numpy(g["logits"][t:t + 1]).to(dev)
        _, idx, wts = layer(x, logits, routing=True)
        np.testing.assert_array_equal(idx.cpu().numpy()[0], g["ref_idx"][t])
        assert np.abs(wts.cpu().numpy()[0] - g["ref_w"][t]).max() < 1e-6


@pytest.mark.parametrize("E", [256, 288, 300, 512, 1024])
@pytest.mark.parametrize("ldt", [torch.float64, torch.float32, torch.float16, torch.bfloat16])
def test_layer_one_token_router_equals_wave_router(dev, E, ldt):
    """The workgroup router of the one-token route + bucket launch (sigmoids over the workgroup,
    selection on one wave) and the one-wave router of vybdq_moe_route give identical ids and
    weights for every logit type and expert count (4, 5, 8 and 16 experts per router lane)."""
    k, H, I = 8, 64, 64
    rng = np.random.default_rng(E)
    w = lambda n, kk: torch.from_numpy(synth.q4_0_weights(rng, n, kk)).to(dev)
    gate = torch.cat([w(I, H) for _ in range(E)])
    up = torch.cat([w(I, H) for _ in range(E)])
    down = torch.cat([w(H, I) for _ in range(E)])
    bias = torch.from_numpy(rng.standard_normal(E).astype(np.float32) * 0.05).to(dev)
    layer = ops.MoeLayer(ops.GGML_Q4_0, gate, up, down, H, I, E, k, bias=bias)
    x = torch.randn(1, H, device=dev).to(torch.bfloat16)
    for rep in range(4):
        logits = torch.from_numpy(rng.standard_normal((1, E))).to(ldt).to(dev)
        if rep == 3:  # ties: every logit equal, so the bias alone orders the experts
            logits = torch.zeros((1, E), dtype=ldt, device=dev)
        _, idx, wts = layer(x, logits, routing=True)
        i0, w0 = ops.moe_route(logits, k, bias)
        torch.cuda.synchronize()
        assert torch.equal(idx, i0) and torch.equal(wts, w0), rep


@pytest.mark.parametrize("ty", [ops.GGML_Q4_0, ops.GGML_Q8_0])
@pytest.mark.parametrize("E,k", [(8, 8), (64, 6), (256, 8), (256, 64)])
@pytest.mark.parametrize("shared,with_bias", [(True, True), (False, False), (True, False)])
def test_layer_one_token_routing_in_gemv_equals_routing_launch(dev, monkeypatch, ty, E, k, shared, with_bias):
    """One token on the grouped GEMV routes inside the gate|up launch (rows in slot order); with
    VYBDQ_MOE_ROUTE_GV=0 a routing + bucketing launch precedes it (rows in expert order). Ids,
    weights and outputs are bit-identical for every logit type, with and without the selection
    bias and the shared expert, topk = E included (H and I multiples of 256: the grouped kernels)."""
    H, I = 256, 512
    rng = np.random.default_rng(E * 131 + k + 2 * shared + with_bias)
    q = synth.q4_0_weights if ty == ops.GGML_Q4_0 else synth.q8_0_weights
    w = lambda n, kk: torch.from_numpy(q(rng, n, kk)).to(dev)
    gate = torch.cat([w(I, H) for _ in range(E)])
    up = torch.cat([w(I, H) for _ in range(E)])
    down = torch.cat([w(H, I) for _ in range(E)])
    sh = (w(I, H), w(I, H), w(H, I)) if shared else None
    bias = torch.from_numpy(rng.standard_normal(E).astype(np.float32) * 0.05).to(dev) if with_bias else None
    layer = ops.MoeLayer(ty, gate, up, down, H, I, E, k, shared=sh, bias=bias)
    x = torch.from_numpy(synth.activations(rng, (1, H))).to(torch.bfloat16).to(dev)
    for ldt in (torch.float64, torch.float32, torch.float16, torch.bfloat16):
        logits = torch.from_numpy(rng.standard_normal((1, E))).to(ldt).to(dev)
        got = []
        for env in ("1", "0"):
            monkeypatch.setenv("VYBDQ_MOE_ROUTE_GV", env)
            y, idx, wts = layer(x, logits, routing=True)
            torch.cuda.synchronize()
            got.append((y.cpu(), idx.cpu(), wts.cpu()))
        assert torch.equal(got[0][1], got[1][1]) and torch.equal(got[0][2], got[1][2]), ldt
        assert torch.equal(got[0][0], got[1][0]), ldt
        i0, w0 = ops.moe_route(logits, k, bias)
        assert torch.equal(got[0][1], i0.cpu()) and torch.equal(got[0][2], w0.cpu()), ldt
