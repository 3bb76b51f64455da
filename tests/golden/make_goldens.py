#!/usr/bin/env python3
"""Write the committed golden fixtures from data files the reference repository holds.

Runs only where the reference checkout is present (default /root/reference; override with
VYBDQ_REFERENCE). It reads data files (raw bytes, JSON, little-endian float32 arrays); it
imports and runs no reference code. Outputs, all in this directory:

  q4_0_gguf_fixture.json          the 18-byte q4_0 block of native/legit/fixtures/gguf/
                                  test.gguf.baseline (bytes 190..207) and the values the
                                  reference's gate expects (native/gguf/dequant_gguf.vyb:118-127)
  exl3_tile_slot_composition.json native/exl3/tile_slot_composition.json, re-serialised as a
                                  sorted slot list, plus a digest of native/exl3/map.bin
                                  re-derived from it (gen_map_bin.py:1-37 layout)
  ../../vybforge_amd/data/iq2s_grid.json
                                  the IQ2_S grid (1024 x 8 bytes) and sign masks: llama.cpp's
                                  iq2s_grid / kmask_iq2xs tables (MIT) as the reference holds
                                  them in native/gguf/iq2s_tables.py, read as text (the hex
                                  literals), not imported; the library build turns it into a
                                  device table, the oracle reads it
  router_golden.npz               the router inputs of the same prep: y (4 x 4096 float32) and the
                                  gate weight (288 x 4096, exactly bf16 values, stored as bf16
                                  bits), so the router GEMM can be checked end to end against the
                                  reference's routing ids/weights in moe_golden.npz
  moe_golden.npz                  from native/glm53/prep/*.f32 (prepare_moe_fixture.py:21-70):
                                  router logits (y @ gate^T in float64), bias, the reference's
                                  routing ids/weights, the expert pre-activations g/u (float64),
                                  a 64-column slice of the down projections and of ref_out.

The reference repository is Apache-2.0 (THIRD-PARTY.md:3); these are data, copied with
attribution.
"""

import hashlib
import json
import os
import struct
import sys

import numpy as np

REF = os.environ.get("VYBDQ_REFERENCE", "/root/reference")
HERE = os.path.dirname(os.path.abspath(__file__))
SRC_NOTE = "rickenator/VybForge (Apache-2.0), data file copied with attribution"


def q4_0_fixture():
    p = os.path.join(REF, "native/legit/fixtures/gguf/test.gguf.baseline")
    raw = open(p, "rb").read()
    sha = hashlib.sha256(raw).hexdigest()
    assert sha == "f23fc38494499a0f27ec1bcb4ee162db893c22be11b33ee17e2a8779ef0a2191", sha
    blk = raw[190:208]
    out = {
        "source": SRC_NOTE + ": native/legit/fixtures/gguf/test.gguf.baseline bytes 190..207",
        "file_sha256": sha,
        "block_hex": blk.hex(),
        "expected_interleaved": [(i % 16) - 8 for i in range(32)],
        "expected_check": "native/gguf/dequant_gguf.vyb:118-127 (|out - ((i % 16) - 8)| <= 1e-6)",
    }
    json.dump(out, open(os.path.join(HERE, "q4_0_gguf_fixture.json"), "w"), indent=1)


def exl3_map():
    p = os.path.join(REF, "native/exl3/tile_slot_composition.json")
    raw = json.load(open(p))
    slots = []
    for k, v in raw.items():
        r, c = (int(t) for t in k.split(","))
        slots.append([r, c, [[int(m), int(b)] for m, b in v]])
    slots.sort(key=lambda s: (s[0], s[1]))
    # the kernel-side map.bin the reference ships: 16-B header + 256 x 16-B entries
    mb = open(os.path.join(REF, "native/exl3/map.bin"), "rb").read()
    body = b"".join(struct.pack("<4H", *(m for m, _ in s[2])) + struct.pack("<4B", *(b for _, b in s[2]))
                    + struct.pack("<HH", s[0], s[1]) for s in slots)
    assert mb[16:] == body, "map.bin body does not match tile_slot_composition.json"
    out = {
        "source": SRC_NOTE + ": native/exl3/tile_slot_composition.json",
        "format": "slots[i] = [row, col, [[nibble_index, nibble_position] x 4]]; window = "
                  "OR nibble[nibble_index] << 4*nibble_position",
        "map_bin_body_sha256": hashlib.sha256(mb[16:]).hexdigest(),
        "slots": slots,
    }
    json.dump(out, open(os.path.join(HERE, "exl3_tile_slot_composition.json"), "w"))


def moe():
    P = os.path.join(REF, "native/glm53/prep")
    f = lambda n, s: np.fromfile(os.path.join(P, n + ".f32"), dtype="<f4").reshape(s)
    H, I, E, K = 4096, 2048, 288, 8
    y = f("y", (4, H))
    gate = f("gate", (E, H))
    bias = f("bias", (E,))
    ref_idx = f("ref_idx", (4, K)).astype(np.int64)
    ref_w = f("ref_w", (4, K))
    ref_out = f("ref_out", (4, H))
    y64 = y.astype(np.float64)
    logits = y64 @ gate.astype(np.float64).T
    wg_e, wu_e, wd_e = f("wg_e", (H, I)), f("wu_e", (H, I)), f("wd_e", (I, H))
    wg_s, wu_s, wd_s = f("wg_s", (H, I)), f("wu_s", (H, I)), f("wd_s", (I, H))
    cols = np.arange(0, H, 64)
    np.savez_compressed(
        os.path.join(HERE, "moe_golden.npz"),
        logits=logits, bias=bias, ref_idx=ref_idx, ref_w=ref_w,
        g_e=y64 @ wg_e.astype(np.float64), u_e=y64 @ wu_e.astype(np.float64),
        g_s=y64 @ wg_s.astype(np.float64), u_s=y64 @ wu_s.astype(np.float64),
        cols=cols, wd_e_cols=np.ascontiguousarray(wd_e[:, cols]),
        wd_s_cols=np.ascontiguousarray(wd_s[:, cols]), ref_out_cols=np.ascontiguousarray(ref_out[:, cols]),
        scale=np.float64(2.5), limit=np.float64(10.0))


def router():
    P = os.path.join(REF, "native/glm53/prep")
    f = lambda n, shape: np.fromfile(os.path.join(P, n + ".f32"), dtype="<f4").reshape(shape)
    y, gate = f("y", (4, 4096)), f("gate", (288, 4096))
    bits = gate.view(np.uint32)
    assert (bits & 0xFFFF).max() == 0, "gate weights are not exactly bf16"
    np.savez_compressed(os.path.join(HERE, "router_golden.npz"), y=y, gate_bf16=(bits >> 16).astype(np.uint16),
                        source=np.array(SRC_NOTE))


def iq2s_grid():
    import re
    p = os.path.join(REF, "native/gguf/iq2s_tables.py")
    text = open(p).read()
    body = text[text.index("IQ2_S_GRID = ("):]
    body = body[:body.index(")")]
    grid = [int(h, 16) for h in re.findall(r"0x[0-9a-fA-F]{16}", body)]
    assert len(grid) == 1024, len(grid)
    kmask = [int(v) for v in re.search(r"IQ2_S_KMASK = \(([^)]*)\)", text).group(1).split(",")]
    assert kmask == [1, 2, 4, 8, 16, 32, 64, 128], kmask
    out = os.path.join(HERE, "..", "..", "vybforge_amd", "data", "iq2s_grid.json")
    json.dump({"source": SRC_NOTE + " (native/gguf/iq2s_tables.py, itself llama.cpp ggml-common.h, MIT)",
               "grid_u64_hex": [f"{g:016x}" for g in grid], "kmask": kmask},
              open(out, "w"), indent=0)
    print("wrote", out)


def st_header():
    """The header of the reference's safetensors fixture (the 66 MB LoRA adapter its container gate
    reads, native/torchload/st_ref.py:38): the 8-byte length, the JSON bytes (gzipped) and the data
    region size. Tests rebuild a file of the same layout with a zero data region."""
    import gzip
    src = os.path.join(REF, "artifacts", "vybos-configurator-lora", "adapter_model.safetensors")
    size = os.path.getsize(src)
    with open(src, "rb") as f:
        n = int.from_bytes(f.read(8), "little")
        hdr = f.read(n)
    out = os.path.join(HERE, "st_lora_header.json.gz")
    with gzip.GzipFile(out, "wb", mtime=0) as g:
        g.write(hdr)
    json.dump({"source": SRC_NOTE + " (artifacts/vybos-configurator-lora/adapter_model.safetensors)",
               "header_len": n, "data_size": size - 8 - n},
              open(os.path.join(HERE, "st_lora_header.meta.json"), "w"), indent=1)
    print("wrote", out)


if __name__ == "__main__":
    if not os.path.isdir(REF):
        sys.exit(f"reference checkout not found at {REF}")
    q4_0_fixture()
    exl3_map()
    moe()
    router()
    iq2s_grid()
    st_header()
    print("goldens written to", HERE)
