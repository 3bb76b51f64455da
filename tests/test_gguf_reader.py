"""The GGUF reader (vybdq_gguf_*, host code: runs without a GPU) against the reference's
frozen fixture (native/legit/fixtures/gguf/test.gguf.baseline, built by
native/gguf/mk_fixture.vyb) and against spec-layout files written by tests/gguf_writer.py."""

import numpy as np
import pytest

from oracle import formats
from tests.conftest import GOLDEN
from tests.gguf_writer import write_gguf
from vybforge_amd import _lib
from vybforge_amd.gguf import GgufFile


def test_reference_fixture():
    """mk_fixture's report: data_base=170; t0@170 t1@174 t2@190 (absolute offsets); t2 is one
    q4_0 block with scale 1 and nibble i = i in the interleaved order, so it decodes to i - 8."""
    with GgufFile(f"{GOLDEN}/gguf_fixture.gguf") as g:
        assert g.version == 3
        assert g.kv == {"general.name": ("str", "tiny")}
        t = g.tensors
        assert list(t) == ["t0", "t1", "t2"]
        assert (t["t0"]["dims"], t["t0"]["type"], t["t0"]["offset"]) == ([2, 3], 0, 170)
        assert (t["t1"]["dims"], t["t1"]["type"], t["t1"]["offset"]) == ([4], 6, 174)
        assert (t["t2"]["dims"], t["t2"]["type"], t["t2"]["offset"]) == ([32], 2, 190)
        raw = g.read_tensor("t2", absolute=True)
        assert raw.size == 18
        np.testing.assert_array_equal(formats.dequant_q4_0(raw, formats.ORDER_INTERLEAVED),
                                      np.arange(32) % 16 - 8)


def _spec_file(path, alignment=64):
    rng = np.random.default_rng(0)
    kv = [("general.architecture", 8, "qwen3"), ("general.alignment", 4, alignment),
          ("qwen3.block_count", 4, 36), ("u8", 0, 200), ("i8", 1, -5), ("u16", 2, 60000), ("i16", 3, -300),
          ("i32", 5, -70000), ("f32", 6, 0.25), ("flag", 7, True), ("u64", 10, 2 ** 40), ("i64", 11, -2 ** 40),
          ("f64", 12, 1e-300), ("tokens", 9, (8, ["a", "bc", ""])), ("ids", 9, (4, [1, 2, 3])),
          ("nested", 9, (9, [(4, [7, 8]), (8, ["x"])]))]
    tensors = [("w.f32", [3, 5], 0, rng.integers(0, 256, 60)), ("w.f16", [7], 1, rng.integers(0, 256, 14)),
               ("w.q4_0", [64, 2], 2, rng.integers(0, 256, 4 * 18)), ("w.q8_0", [32, 3], 8, rng.integers(0, 256, 3 * 34)),
               ("w.q4_k", [256, 2], 12, rng.integers(0, 256, 2 * 144)), ("w.q6_k", [512], 14, rng.integers(0, 256, 2 * 210)),
               ("w.bf16", [5], 30, rng.integers(0, 256, 10))]
    base, offsets = write_gguf(path, kv, tensors, alignment)
    return kv, tensors, base, offsets


def test_spec_layout(tmp_path):
    p = tmp_path / "m.gguf"
    kv, tensors, base, offsets = _spec_file(p)
    with GgufFile(p) as g:
        assert g.alignment == 64 and g.data_base == base
        assert g.kv["general.architecture"] == ("str", "qwen3")
        assert g.kv["qwen3.block_count"] == ("u32", 36)
        assert g.kv["i8"] == ("i8", -5) and g.kv["i16"] == ("i16", -300) and g.kv["i32"] == ("i32", -70000)
        assert g.kv["u64"] == ("u64", 2 ** 40) and g.kv["i64"] == ("i64", -2 ** 40)
        assert g.kv["f32"] == ("f32", 0.25) and g.kv["f64"] == ("f64", 1e-300) and g.kv["flag"] == ("bool", True)
        assert g.kv["tokens"] == ("array", ("str", 3)) and g.kv["nested"] == ("array", ("array", 2))
        for (name, dims, ty, data), off in zip(tensors, offsets):
            t = g.tensors[name]
            assert (t["dims"], t["type"], t["offset"], t["nbytes"]) == (dims, ty, off, len(data))
            np.testing.assert_array_equal(g.read_tensor(name), np.asarray(data, np.uint8))
        lib = _lib.lib
        prev = 0
        for name, dims, ty, data in tensors:
            o = lib.vybdq_gguf_slab_offset(g.h, g.tensors[name]["index"], 256)
            assert o % 256 == 0 and o >= prev
            prev = o + len(data)
        assert lib.vybdq_gguf_slab_bytes(g.h, 256) == (prev + 255) // 256 * 256


def test_errors(tmp_path):
    lib = _lib.lib
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + bytes(20))
    assert lib.vybdq_gguf_open(str(bad).encode()) == _lib.ERR_ARG
    p = tmp_path / "m.gguf"
    _spec_file(p)
    data = p.read_bytes()
    for cut in (10, 30, 200, len(data) - 1000):
        trunc = tmp_path / f"t{cut}.gguf"
        trunc.write_bytes(data[:cut])
        h = lib.vybdq_gguf_open(str(trunc).encode())
        if h > 0:  # the index is whole: reading past the end must fail instead
            assert lib.vybdq_gguf_read_tensor(h, 6, 0, None, 0) < 0
            lib.vybdq_gguf_close(h)
        else:
            assert h == _lib.ERR_ARG
    assert lib.vybdq_gguf_info(12345, 0) == _lib.ERR_ARG
    assert lib.vybdq_gguf_open(str(tmp_path / "missing.gguf").encode()) == _lib.ERR_ARG


def test_corrupt_counts_and_sizes_are_errors(tmp_path):
    """Counts larger than the file can hold and array sizes whose byte count overflows 64 bits are
    rejected with an error code (no allocation of the claimed size, no exception across the C ABI)."""
    import struct
    from vybforge_amd import _lib

    def write(name, body):
        p = tmp_path / name
        p.write_bytes(b"GGUF" + struct.pack("<I", 3) + body)
        return str(p).encode()

    huge = write("huge_counts.gguf", struct.pack("<QQ", 1 << 62, 1 << 62) + b"\0" * 64)
    assert _lib.lib.vybdq_gguf_open(huge) == _lib.ERR_ARG
    assert "counts" in _lib.last_error()
    key = b"a.b"
    arr = struct.pack("<QQ", 0, 1) + struct.pack("<Q", len(key)) + key + struct.pack("<I", 9)
    arr += struct.pack("<IQ", 10, (1 << 63) + 5) + b"\0" * 64  # u64 array whose byte size wraps
    wrap = write("array_wrap.gguf", arr)
    assert _lib.lib.vybdq_gguf_open(wrap) == _lib.ERR_ARG
    assert "array" in _lib.last_error()
