"""GPU parity for the GLM-5.3 MoE layer with EXL3 4-bpw routed experts and a bf16 shared expert
(vybdq_moe_forward_exl3; the reference's native/glm53/glm_engine.vyb:2728-2990) against the oracle:
routing (oracle.moe.route_logits) exactly, outputs within 2e-3 of float64 (the
native/glm53/verify_layer0.py:134-139 gate).

Small shapes run the whole oracle composition (oracle.exl3.dequant_exl3_f64 per expert matrix,
oracle.moe.moe_forward). The GLM-5.3 shapes (H = 4096, I = 2048, 288 routed experts + 1 shared,
top-8, T = 1 / 16 / 256) check every token's routing and two tokens' outputs; there the routed
experts draw their trellis from a pool of four per projection (each expert keeps its own suh and
svh, so any mix-up of experts still shows), the oracle decodes each pool trellis once and applies it
in the FWHT form x W = svh * fwht(fwht(x * suh) What) that tests/test_oracle_pins.py pins to
x @ dequant_exl3_f64."""

import numpy as np
import pytest
import torch

from oracle import exl3, matmul, moe
from tests import st_writer
from vybforge_amd import ops, synth
from vybforge_amd.safetensors import Checkpoint, moe_exl3_layer

pytestmark = pytest.mark.gpu

TOL = matmul.TOL


def _bf16(rng, shape, scale=0.02):
    """bf16 weights as (torch bf16 on the host, float64 values)."""
    t = torch.from_numpy((rng.standard_normal(shape) * scale).astype(np.float32)).to(torch.bfloat16)
    return t, t.to(torch.float64).numpy()


# suh / svh of the routed experts ~ +-|N(0, SCALE)|: W = diag(suh) Hs What Hs diag(svh) then has
# entries of about N(0, 0.02) like a real checkpoint's (and like the bf16 shared expert here), so
# the routed experts weigh in the outputs as much as the shared expert does
SCALE = 0.12


def _scales(rng, K, N):
    sgn = lambda n: rng.integers(0, 2, n) * 2 - 1
    suh = (np.abs(rng.standard_normal(K) * SCALE) * sgn(K)).astype(np.float16)
    svh = (np.abs(rng.standard_normal(N) * SCALE) * sgn(N)).astype(np.float16)
    return suh, svh


def _expert_tensors(rng, H, I):
    """The 9 host arrays of one EXL3 expert in the table order of ops.EXL3_EXPERT_FIELDS."""
    out = []
    for K, N in ((H, I), (H, I), (I, H)):
        t, _, _ = synth.exl3_tensors(rng, K, N)
        out += [t, *_scales(rng, K, N)]
    return out


def _to_dev(arrs, dev):
    return [torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to(dev) for a in arrs]


def _x(rng, T, H, xdt):
    x = torch.from_numpy(synth.activations(rng, (T, H)))
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    elif xdt == "f16":
        x = x.to(torch.float16)
    return x


@pytest.mark.parametrize("T", [1, 2, 5, 16, 40])
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
@pytest.mark.parametrize("with_shared,with_bias", [(True, True), (False, False)])
def test_moe_exl3_small(dev, T, xdt, with_shared, with_bias):
    """H = I = 256, 12 experts, top-4: one-row groups (T = 1), two-row groups (T = 2, 5, 16) and
    16-row groups on the matrix cores (T = 40); the whole layer against oracle.moe.moe_forward."""
    H, I, E, k = 256, 256, 12, 4
    rng = np.random.default_rng(T * 7 + len(xdt) + with_shared)
    host = [_expert_tensors(rng, H, I) for _ in range(E)]
    experts = [_to_dev(h, dev) for h in host]
    shared = sh64 = None
    if with_shared:
        sh = [_bf16(rng, s) for s in ((I, H), (I, H), (H, I))]
        shared = tuple(t.to(dev) for t, _ in sh)
        sh64 = tuple(v for _, v in sh)
    bias = rng.standard_normal(E).astype(np.float32) * 0.1 if with_bias else None
    layer = ops.MoeExl3Layer(experts, H, I, topk=k, shared=shared,
                             bias=torch.from_numpy(bias).to(dev) if with_bias else None)
    x = _x(rng, T, H, xdt)
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32))
    y, idx, w = layer(x.to(dev), logits.to(dev), routing=True)

    def mats(e):
        h = host[e]
        return tuple(exl3.dequant_exl3_f64(h[3 * p], h[3 * p + 1], h[3 * p + 2]).T for p in range(3))
    zero = (np.zeros((I, H)), np.zeros((I, H)), np.zeros((H, I)))
    ref, ridx, rw = moe.moe_forward(x.to(torch.float64).numpy(), logits.numpy(), mats, sh64 or zero, topk=k,
                                    bias=bias)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    assert np.abs(w.cpu().numpy() - rw).max() < 1e-6
    y = y.cpu().numpy()
    assert matmul.rel_maxnorm(y, ref) < TOL
    if with_shared:  # the routed experts' part alone, so that the shared expert cannot mask it
        sh_ref = moe.ffn_rows(x.to(torch.float64).numpy(), *sh64)
        assert matmul.rel_maxnorm(y - sh_ref, ref - sh_ref) < TOL


@pytest.mark.parametrize("T", [3, 17])
def test_moe_exl3_combine_chunks(dev, monkeypatch, T):
    """Top-10 (two slot groups in the combine) at H = 640 (five 128-column chunks: a partial second
    group of four); the combine at one chunk and at four chunks per workgroup against the oracle,
    and the two bit-identical (the same additions in the same order)."""
    H, I, E, k = 640, 256, 12, 10
    rng = np.random.default_rng(31 + T)
    host = [_expert_tensors(rng, H, I) for _ in range(E)]
    sh = [_bf16(rng, s) for s in ((I, H), (I, H), (H, I))]
    bias = rng.standard_normal(E).astype(np.float32) * 0.1
    layer = ops.MoeExl3Layer([_to_dev(h, dev) for h in host], H, I, topk=k,
                             shared=tuple(t.to(dev) for t, _ in sh), bias=torch.from_numpy(bias).to(dev))
    x = _x(rng, T, H, "bf16")
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32))
    mats = lambda e: tuple(exl3.dequant_exl3_f64(host[e][3 * p], host[e][3 * p + 1], host[e][3 * p + 2]).T
                           for p in range(3))
    ref, ridx, _ = moe.moe_forward(x.to(torch.float64).numpy(), logits.numpy(), mats, tuple(v for _, v in sh),
                                   topk=k, bias=bias)
    ys = []
    for ch in ("1", "4"):
        monkeypatch.setenv("VYBDQ_MX_COMB", ch)
        y, idx, _ = layer(x.to(dev), logits.to(dev), routing=True)
        np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
        ys.append(y.cpu().numpy())
        assert matmul.rel_maxnorm(ys[-1], ref) < TOL, ch
    np.testing.assert_array_equal(ys[0], ys[1])


def test_moe_exl3_out_dtypes_and_f16_x(dev):
    """fp16 activations (two bf16 terms into the shared expert) and bf16 / fp16 outputs."""
    H, I, E, k, T = 256, 128, 6, 2, 9
    rng = np.random.default_rng(5)
    host = [_expert_tensors(rng, H, I) for _ in range(E)]
    sh = [_bf16(rng, s) for s in ((I, H), (I, H), (H, I))]
    layer = ops.MoeExl3Layer([_to_dev(h, dev) for h in host], H, I, topk=k, shared=tuple(t.to(dev) for t, _ in sh))
    x = _x(rng, T, H, "f16")
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32))
    mats = lambda e: tuple(exl3.dequant_exl3_f64(host[e][3 * p], host[e][3 * p + 1], host[e][3 * p + 2]).T
                           for p in range(3))
    ref, _, _ = moe.moe_forward(x.to(torch.float64).numpy(), logits.numpy(), mats, tuple(v for _, v in sh), topk=k)
    for odt in (torch.float16, torch.bfloat16):
        y = layer(x.to(dev), logits.to(dev), out_dtype=odt).to(torch.float64).cpu().numpy()
        assert matmul.rel_maxnorm(y, ref) < TOL + (4e-3 if odt == torch.bfloat16 else 5e-4), odt


def test_moe_exl3_from_checkpoint(dev, tmp_path):
    """The layer built from a sharded checkpoint by the reference's tensor names (experts, shared
    expert, e_score_correction_bias) equals the layer built from the same arrays directly."""
    H, I, E, k, T = 256, 128, 4, 2, 3
    rng = np.random.default_rng(17)
    host = [_expert_tensors(rng, H, I) for _ in range(E)]
    sh = [_bf16(rng, s) for s in ((I, H), (I, H), (H, I))]
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    pre = "model.language_model.layers.3."
    s1, s2 = [], []
    for e in range(E):
        for f, a in zip(ops.EXL3_EXPERT_FIELDS, host[e]):
            (s1 if f.endswith("trellis") else s2).append((f"{pre}mlp.experts.{e}.{f}", a.view(np.int16) if a.dtype == np.uint16 else a))
        for proj in ("gate_proj", "up_proj", "down_proj"):
            s2.append((f"{pre}mlp.experts.{e}.{proj}.mcg", np.array([1], np.int32)))
    for proj, (t, _) in zip(("gate_proj", "up_proj", "down_proj"), sh):
        s2.append((f"{pre}mlp.shared_experts.{proj}.weight", "BF16", list(t.shape), t.view(torch.int16).numpy().tobytes()))
    s2.append((f"{pre}mlp.gate.e_score_correction_bias", bias))
    st_writer.write(tmp_path / "model-00001-of-00002.safetensors", s1)
    st_writer.write(tmp_path / "model-00002-of-00002.safetensors", s2)
    shard_of = {n[0]: "model-00001-of-00002.safetensors" for n in s1}
    shard_of.update({n[0]: "model-00002-of-00002.safetensors" for n in s2})
    st_writer.write_index(tmp_path / "model.safetensors.index.json", shard_of)
    layer = moe_exl3_layer(Checkpoint(tmp_path), pre, dev, E, topk=k)
    direct = ops.MoeExl3Layer([_to_dev(h, dev) for h in host], H, I, topk=k, shared=tuple(t.to(dev) for t, _ in sh),
                              bias=torch.from_numpy(bias).to(dev))
    x = _x(rng, T, H, "bf16").to(dev)
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).to(dev)
    torch.testing.assert_close(layer(x, logits), direct(x, logits), rtol=0, atol=0)


def test_moe_exl3_rejects_bad_tables(dev):
    H, I = 256, 128
    rng = np.random.default_rng(3)
    ts = _to_dev(_expert_tensors(rng, H, I), dev)
    with pytest.raises(ValueError):
        ops.MoeExl3Layer([ts[:8]], H, I, topk=1)             # 8 tensors
    bad = list(ts)
    bad[4] = bad[4][:64]                                      # up suh of the wrong length
    with pytest.raises(ValueError):
        ops.MoeExl3Layer([bad], H, I, topk=1)


# ---- GLM-5.3 shapes --------------------------------------------------------------------------------

GLM = dict(H=4096, I=2048, E=288, k=8)
POOL = 4


@pytest.fixture(scope="module")
def glm_layer(dev):
    H, I, E = GLM["H"], GLM["I"], GLM["E"]
    rng = np.random.default_rng(53)
    pool_t = {p: [synth.exl3_tensors(rng, *((H, I) if p < 2 else (I, H)))[0] for _ in range(POOL)] for p in range(3)}
    pool_d = {p: [torch.from_numpy(t.view(np.int16)).to(dev) for t in pool_t[p]] for p in range(3)}
    whats = {p: [exl3.decode_rotated(t).astype(np.float64) for t in pool_t[p]] for p in range(3)}
    experts, scales = [], []
    for e in range(E):
        ts, sc = [], []
        for p, (K, N) in enumerate(((H, I), (H, I), (I, H))):
            suh, svh = _scales(rng, K, N)
            ts += [pool_d[p][e % POOL], torch.from_numpy(suh).to(dev), torch.from_numpy(svh).to(dev)]
            sc.append((suh.astype(np.float64), svh.astype(np.float64)))
        experts.append(ts)
        scales.append(sc)
    sh = [_bf16(rng, s) for s in ((I, H), (I, H), (H, I))]
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    layer = ops.MoeExl3Layer(experts, H, I, topk=GLM["k"], shared=tuple(t.to(dev) for t, _ in sh),
                             bias=torch.from_numpy(bias).to(dev))
    return layer, whats, scales, tuple(v for _, v in sh), bias


def _apply(x, what, suh, svh):
    return exl3.fwht128_rows(exl3.fwht128_rows(x * suh) @ what) * svh


@pytest.mark.parametrize("T", [1, 16, 256])
def test_moe_exl3_glm53_shapes(dev, glm_layer, T):
    layer, whats, scales, sh64, bias = glm_layer
    H, E, k = GLM["H"], GLM["E"], GLM["k"]
    rng = np.random.default_rng(1000 + T)
    x = _x(rng, T, H, "bf16")
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32))
    y, idx, w = layer(x.to(dev), logits.to(dev), routing=True)
    torch.cuda.synchronize()
    ridx, rw = moe.route_logits(logits.numpy(), k, bias)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    assert np.abs(w.cpu().numpy() - rw).max() < 1e-6
    x64 = x.to(torch.float64).numpy()
    y = y.cpu().numpy()
    for t in sorted({0, T - 1}):
        sh_ref = moe.ffn_rows(x64[t:t + 1], *sh64)[0]
        routed = np.zeros(H)
        for s in range(k):
            e = int(ridx[t, s])
            (sg, vg), (su, vu), (sd, vd) = scales[e]
            g = _apply(x64[t:t + 1], whats[0][e % POOL], sg, vg)
            u = _apply(x64[t:t + 1], whats[1][e % POOL], su, vu)
            routed += rw[t, s] * _apply(moe.swiglu(g, u), whats[2][e % POOL], sd, vd)[0]
        assert matmul.rel_maxnorm(y[t], sh_ref + routed) < TOL, (T, t)
        assert matmul.rel_maxnorm(y[t] - sh_ref, routed) < TOL, (T, t, "routed part")
