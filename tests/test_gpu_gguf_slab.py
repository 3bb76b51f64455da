"""A GGUF file resident in one device slab (vybdq_gguf_load_slab) feeds the GEMVs directly:
every tensor's slab bytes equal the file's, and GEMVs on slab views match the oracle."""

import numpy as np
import pytest
import torch

from oracle import kquants, matmul
from tests.gguf_writer import write_gguf
from vybforge_amd import ops, synth
from vybforge_amd.gguf import GgufFile

pytestmark = pytest.mark.gpu


def test_slab_gemv(dev, tmp_path):
    rng = np.random.default_rng(3)
    N, K = 192, 2560
    mats = {"blk.0.ffn_up.weight": (12, synth.kquant_weights(rng, 12, N, K)),
            "blk.0.ffn_down.weight": (14, synth.kquant_weights(rng, 14, N, K)),
            "blk.0.attn_q.weight": (8, synth.q8_0_weights(rng, N, K)),
            "blk.0.attn_k.weight": (2, synth.q4_0_weights(rng, N, K)),
            "blk.0.attn_v.weight": (13, synth.kquant_weights(rng, 13, N, K))}
    tensors = [(name, [K, N], ty, raw) for name, (ty, raw) in mats.items()]
    tensors.insert(1, ("token_embd.norm", [7], 0, rng.integers(0, 256, 28)))  # an odd-sized tensor between
    path = tmp_path / "m.gguf"
    write_gguf(path, [("general.alignment", 4, 32)], tensors, alignment=32)
    x = synth.activations(rng, (K,))
    with GgufFile(path) as g:
        slab, views = g.load_slab(dev, align=256)
        for name, dims, ty, raw in tensors:
            assert torch.equal(views[name].cpu(), torch.from_numpy(np.asarray(raw, np.uint8)))
        for name, (ty, raw) in mats.items():
            y = ops.gemv(ty, views[name], torch.from_numpy(x).to(dev), N, K).cpu().numpy()
            if ty in kquants.DEQUANT:
                w = kquants.matrix(ty, raw, N, K)
            elif ty == 8:
                w = matmul.q8_0_matrix(raw, N, K)
            else:
                w = matmul.q4_0_matrix(raw, N, K)
            assert matmul.rel_maxnorm(y, w @ x.astype(np.float64)) < matmul.TOL, name
