"""Router logits (vybdq_router_logits, float64 accumulation) against the oracle's ordered float64
sum, and end to end against the reference's own routing of its GLM layer-0 fixture
(native/glm53/prep: y, the bf16 gate weight, the selection bias, ref_idx / ref_w)."""

import numpy as np
import pytest
import torch

from oracle import moe
from tests.conftest import GOLDEN
from vybforge_amd import ops

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
