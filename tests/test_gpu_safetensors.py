"""GPU: tensors uploaded from safetensors files equal the file bytes, and an EXL3 linear layer
built from its named checkpoint tensors (<prefix>.trellis / .suh / .svh / .mcg across shards of a
sharded checkpoint) matches the float64 oracle and, bit for bit, the layer built from the same
arrays directly."""

import numpy as np
import pytest
import torch

from oracle import exl3, matmul
from tests import st_writer
from vybforge_amd import ops, synth
from vybforge_amd.safetensors import Checkpoint, SafetensorsFile, exl3_linear

pytestmark = pytest.mark.gpu


def test_upload_matches_file(dev, tmp_path):
    rng = np.random.default_rng(60)
    a = rng.standard_normal((33, 17)).astype(np.float32)
    h = rng.standard_normal(1000).astype(np.float16)
    bf = rng.integers(0, 65535, (4, 8), np.uint16)
    p = tmp_path / "u.safetensors"
    st_writer.write(p, [("a", a), ("h", h), ("bf", "BF16", [4, 8], bf.tobytes()), ("z", np.zeros(0, np.float32))])
    f = SafetensorsFile(p)
    np.testing.assert_array_equal(f.to_device("a", dev).cpu().numpy(), a)
    np.testing.assert_array_equal(f.to_device("h", dev).cpu().numpy(), h)
    got_bf = f.to_device("bf", dev)
    assert got_bf.dtype == torch.bfloat16
    np.testing.assert_array_equal(got_bf.view(torch.int16).cpu().numpy().view(np.uint16), bf)
    assert f.to_device("z", dev).numel() == 0


def test_exl3_layer_from_sharded_checkpoint(dev, tmp_path):
    rng = np.random.default_rng(62)
    cb = ops.EXL3_MCG
    K, N = 512, 384
    t, suh, svh = synth.exl3_tensors(rng, K, N)
    pre = "model.language_model.layers.3.mlp.experts.0.down_proj"
    shard1 = [(pre + ".trellis", t.view(np.int16))]
    shard2 = [(pre + ".suh", suh), (pre + ".svh", svh), (pre + ".mcg", np.array([1], np.int32))]
    st_writer.write(tmp_path / "model-00001-of-00002.safetensors", shard1)
    st_writer.write(tmp_path / "model-00002-of-00002.safetensors", shard2)
    st_writer.write_index(tmp_path / "model.safetensors.index.json",
                          {n: f"model-0000{1 if n.endswith('trellis') else 2}-of-00002.safetensors"
                           for n, _ in shard1 + shard2})
    ck = Checkpoint(tmp_path)
    lin = exl3_linear(ck, pre, dev)
    assert (lin.K, lin.N, lin.cb) == (K, N, cb)
    x = rng.standard_normal((3, K)).astype(np.float16)
    xd = torch.from_numpy(x).to(dev)
    y = lin(xd).cpu().numpy()
    ref = x.astype(np.float64) @ exl3.dequant_exl3_f64(t, suh, svh, cb)
    assert matmul.rel_maxnorm(y, ref) < matmul.TOL
    direct = ops.Exl3Linear(torch.from_numpy(t.view(np.int16)).to(dev), torch.from_numpy(suh).to(dev),
                            torch.from_numpy(svh).to(dev), K, N, cb)
    np.testing.assert_array_equal(direct(xd).cpu().numpy(), y)


def test_exl3_layer_rejects_other_codebooks_and_bad_shapes(dev, tmp_path):
    rng = np.random.default_rng(63)
    t, suh, svh = synth.exl3_tensors(rng, 128, 128)
    mcg = np.array([1], np.int32)
    st_writer.write(tmp_path / "m.safetensors", [("p.trellis", t.view(np.int16)), ("p.suh", suh), ("p.svh", svh),
                                                  ("p.mcg", mcg), ("p.mul1", np.array([1], np.int32)),
                                                  ("q.trellis", t.view(np.int16)), ("q.suh", suh[:64]),
                                                  ("q.svh", svh), ("q.mcg", mcg),
                                                  ("r.trellis", t.view(np.int16)), ("r.suh", suh), ("r.svh", svh)])
    ck = Checkpoint(tmp_path)
    with pytest.raises(NotImplementedError):
        exl3_linear(ck, "p", dev)   # mul1 codebook
    with pytest.raises(ValueError):
        exl3_linear(ck, "q", dev)   # suh of the wrong length
    with pytest.raises(NotImplementedError):
        exl3_linear(ck, "r", dev)   # no .mcg: the multiply-add codebook
