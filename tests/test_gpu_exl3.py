"""GPU parity for EXL3: rotated-basis decode bit-exact vs the oracle (mcg codebook), full
dequant within the reference's gates (verify_exl3_vyb.py:57,66: rel 1.5e-3, |d| 3e-3), and the
fused GEMM within 2e-3 of the float64 oracle for batch 1..16."""

import numpy as np
import pytest
import torch

from oracle import exl3, matmul
from vybforge_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu


def dev_t(a, dev):
    return torch.from_numpy(np.array(a, copy=True)).to(dev)


@pytest.mark.parametrize("odt", [torch.float16, torch.float32])
def test_exl3_decode_bit_exact(dev, odt):
    rng = np.random.default_rng(31)
    K, N = 128, 256
    t, _, _ = synth.exl3_tensors(rng, K, N)
    got = ops.exl3_decode_tiles(dev_t(t, dev), K, N, odt).cpu().numpy()
    ref = exl3.decode_rotated(t)
    np.testing.assert_array_equal(got, ref.astype(got.dtype))


def test_exl3_decode_all_windows(dev):
    # every 16-bit value appears in some slot: the trellis below makes slot (r, c) of tile i
    # windows cover 0..65535 through random data at a larger size
    rng = np.random.default_rng(31)
    K, N = 1024, 2048
    t, _, _ = synth.exl3_tensors(rng, K, N)
    got = ops.exl3_decode_tiles(dev_t(t, dev), K, N, torch.float16).cpu().numpy()
    np.testing.assert_array_equal(got, exl3.decode_rotated(t))


def test_exl3_zero_trellis_kat(dev):
    t = np.zeros((8, 8, 64), np.uint16)
    got = ops.exl3_decode_tiles(dev_t(t, dev), 128, 128, torch.float32).cpu().numpy()
    assert np.all(got == 1.84375)


@pytest.mark.parametrize("odt", [torch.float32, torch.float16])
def test_exl3_dequant_full(dev, odt):
    rng = np.random.default_rng(32)
    K, N = 256, 384
    t, suh, svh = synth.exl3_tensors(rng, K, N)
    got = ops.exl3_dequant(dev_t(t, dev), dev_t(suh, dev), dev_t(svh, dev), K, N, odt).to(torch.float64).cpu().numpy()
    ref = exl3.dequant_exl3_f64(t, suh, svh)
    d = np.abs(got - ref)
    assert d.max() <= 3e-3
    assert d.max() / np.abs(ref).max() <= 1.5e-3


@pytest.mark.parametrize("B", [1, 3, 16])
def test_exl3_gemm(dev, B):
    rng = np.random.default_rng(40 + B)
    K, N = 1024, 768
    t, suh, svh = synth.exl3_tensors(rng, K, N)
    x = rng.standard_normal((B, K)).astype(np.float16)
    lin = ops.Exl3Linear(dev_t(t, dev), dev_t(suh, dev), dev_t(svh, dev), K, N)
    y = lin(dev_t(x, dev)).cpu().numpy()
    ref = x.astype(np.float64) @ exl3.dequant_exl3_f64(t, suh, svh)
    assert matmul.rel_maxnorm(y, ref) < matmul.TOL


@pytest.fixture(scope="module")
def exl3_config4(dev):
    rng = np.random.default_rng(44)
    K, N = 5120, 17408
    t, suh, svh = synth.exl3_tensors(rng, K, N)
    lin = ops.Exl3Linear(dev_t(t, dev), dev_t(suh, dev), dev_t(svh, dev), K, N)
    # float64 oracle on column slices (the full float64 dequant is 89M weights): the first 1024
    # columns and the last 1024 (the last column blocks of every k-split)
    slices = {0: exl3.dequant_exl3_f64(t[:, :64], suh, svh[:1024]),
              N - 1024: exl3.dequant_exl3_f64(t[:, -64:], suh, svh[-1024:])}
    return lin, slices, K, N


@pytest.mark.parametrize("B,xdt", [(1, torch.float32), (2, torch.float16), (4, torch.float16),
                                   (16, torch.float16), (16, torch.bfloat16)])
def test_exl3_gemm_config4_shape(dev, exl3_config4, B, xdt):
    """K = 5120, N = 17408 at every batch regime: one fused launch with 14 k-splits over 1904
    workgroups (B <= 2), and the three-launch matrix-core path with 16 k-splits over 2176
    workgroups (B = 4, 16)."""
    lin, slices, K, N = exl3_config4
    x = torch.from_numpy(np.random.default_rng(B).standard_normal((B, K)).astype(np.float32)).to(xdt)
    y = lin(x.to(dev)).cpu().numpy()
    x64 = x.to(torch.float64).numpy()
    for c0, w in slices.items():
        ref = x64 @ w
        assert matmul.rel_maxnorm(y[:, c0:c0 + 1024], ref) < matmul.TOL, (B, c0)


@pytest.mark.parametrize("K,N", [(128, 256), (1152, 256), (2048, 384)])
def test_exl3_gemm_splits_and_reuse(dev, K, N):
    """One workspace across calls of several batch sizes and dtypes (the per-block arrival
    counters must come back to zero after every call): a single k-split (K = 128), even splits
    (K = 1152: 72 k-blocks, 3 splits of 24 at batch <= 2, 9 of 8 above), a ragged last split
    (K = 2048 at batch <= 2: 128 k-blocks, 5 splits of 24 and one of 8), repeated calls
    bit-identical."""
    rng = np.random.default_rng(K + N)
    t, suh, svh = synth.exl3_tensors(rng, K, N)
    lin = ops.Exl3Linear(dev_t(t, dev), dev_t(suh, dev), dev_t(svh, dev), K, N)
    w = exl3.dequant_exl3_f64(t, suh, svh)
    first = {}
    for B, xdt, ydt in [(16, torch.bfloat16, torch.float32), (1, torch.float32, torch.float16), (5, torch.float16, torch.bfloat16),
                        (2, torch.float16, torch.float32), (16, torch.bfloat16, torch.float32), (1, torch.float32, torch.float16)]:
        x = torch.from_numpy(np.random.default_rng(B).standard_normal((B, K)).astype(np.float32)).to(xdt)
        y = lin(x.to(dev), ydt).to(torch.float64).cpu().numpy()
        ref = x.to(torch.float64).numpy() @ w
        tol = matmul.TOL if ydt == torch.float32 else 8e-3
        assert matmul.rel_maxnorm(y, ref) < tol, (B, xdt, ydt)
        key = (B, xdt, ydt)
        if key in first:
            np.testing.assert_array_equal(y, first[key])
        first[key] = y


def test_exl3_gemm_graph_replays(dev):
    """Captured once, replayed with other work between the replays: every replay matches eager."""
    rng = np.random.default_rng(7)
    K, N = 1024, 512
    t, suh, svh = synth.exl3_tensors(rng, K, N)
    lin = ops.Exl3Linear(dev_t(t, dev), dev_t(suh, dev), dev_t(svh, dev), K, N)
    x = dev_t(rng.standard_normal((3, K)).astype(np.float16), dev)
    out = torch.empty((3, N), dtype=torch.float32, device=dev)
    eager = lin(x).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        lin(x, out=out)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        lin(x, out=out)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        lin(x)  # eager call between replays on the same workspace
        torch.cuda.synchronize()


def test_exl3_workspace_errors(dev):
    assert _lib.lib.vybdq_exl3_workspace_size(17, 128, 128) == -1
    assert _lib.lib.vybdq_exl3_workspace_size(1, 100, 128) == -1
