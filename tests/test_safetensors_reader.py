"""safetensors reader and checkpoint index (host code behind vybdq_st_*; no GPU): spec-layout files
of every sized dtype, metadata, escaped names, empty and scalar tensors, unsized dtypes, the
reference's own fixture header (the LoRA adapter its container gate reads,
native/torchload/st_ref.py:38) parsed against Python's json, sharded index resolution, and the
malformed-file errors."""

import gzip
import hashlib
import json
import os
import struct

import numpy as np
import pytest

from tests import st_writer
from vybforge_amd import _lib
from vybforge_amd.safetensors import Checkpoint, SafetensorsFile

HERE = os.path.dirname(os.path.abspath(__file__))
REF_FILE = "/root/reference/artifacts/vybos-configurator-lora/adapter_model.safetensors"


def test_every_sized_dtype_round_trip(tmp_path):
    rng = np.random.default_rng(5)
    arrs = [("f64", rng.standard_normal((3, 2))), ("f32", rng.standard_normal((4, 5)).astype(np.float32)),
            ("f16", rng.standard_normal(7).astype(np.float16)), ("i64", rng.integers(-9, 9, (2, 2), np.int64)),
            ("i32", np.array(7, np.int32)), ("i16", rng.integers(-300, 300, (2, 3, 64), np.int16)),
            ("i8", rng.integers(-100, 100, 9, np.int8)), ("u8", np.zeros(0, np.uint8)),
            ("u16", rng.integers(0, 65535, 6, np.uint16)), ("u32", rng.integers(0, 2**31, 3, np.uint32)),
            ("u64", rng.integers(0, 2**40, 2, np.uint64)), ("b", rng.integers(0, 2, 5).astype(np.bool_))]
    raw_bf16 = rng.integers(0, 65535, 8, np.uint16)
    tens = arrs + [("bf", "BF16", [2, 4], raw_bf16.tobytes()), ("e4", "F8_E4M3", [3], b"\x01\x02\x03"),
                   ("e5", "F8_E5M2", [1, 2], b"\x04\x05")]
    p = tmp_path / "a.safetensors"
    hdr = st_writer.write(p, tens, metadata={"format": "pt", "note": "x\ny"})
    f = SafetensorsFile(p)
    n = int.from_bytes(open(p, "rb").read(8), "little")
    assert f.header_len == n and f.data_base == 8 + n and f.file_size == os.path.getsize(p)
    assert list(f.tensors) == [t[0] for t in tens]  # header order
    assert f.metadata == {"format": "pt", "note": "x\ny"}
    for name, a in arrs:
        t = f.tensors[name]
        assert t["shape"] == list(np.shape(a)) and t["offset"] == 8 + n + hdr[name]["data_offsets"][0]
        np.testing.assert_array_equal(f.read(name), a)
    np.testing.assert_array_equal(f.read("bf"), raw_bf16.reshape(2, 4))
    assert f.read("e5").tobytes() == b"\x04\x05" and f.tensors["e4"]["dtype"] == "F8_E4M3"
    assert f.tensors["i32"]["shape"] == [] and f.tensors["u8"]["nbytes"] == 0
    assert _lib.lib.vybdq_st_find(f.h, b"f16") == f.tensors["f16"]["index"]
    assert _lib.lib.vybdq_st_find(f.h, b"absent") == -1
    assert f.meta("absent") is None
    f.close()


def test_escaped_names_and_unsized_dtype(tmp_path):
    names = ["a\"b\\c/d", "tab\there", "é中", "\U0001d518 non-BMP"]
    tens = [(nm, np.full(2, i, np.float32)) for i, nm in enumerate(names)]
    tens.append(("packed", "F4", [4], b"\xAB\xCD"))  # unsized: listed, bytes returned raw
    p = tmp_path / "e.safetensors"
    st_writer.write(p, tens)  # json.dumps escapes to \\uXXXX, surrogate pairs for non-BMP
    assert b"\\ud835\\udd18" in open(p, "rb").read()
    f = SafetensorsFile(p)
    assert list(f.tensors) == names + ["packed"]
    for i, nm in enumerate(names):
        np.testing.assert_array_equal(f.read(nm), np.full(2, i, np.float32))
    assert _lib.lib.vybdq_st_tensor_field(f.h, f.tensors["packed"]["index"], 0) == 0
    assert f.read("packed").tobytes() == b"\xAB\xCD"


def test_reference_fixture_header(tmp_path):
    """The reference's safetensors fixture header, rebuilt as a file with a zero data region of the
    recorded size: every tensor's dtype, shape and absolute offset equal Python's own parse."""
    meta = json.load(open(os.path.join(HERE, "golden", "st_lora_header.meta.json")))
    hdr = gzip.open(os.path.join(HERE, "golden", "st_lora_header.json.gz")).read()
    assert len(hdr) == meta["header_len"]
    ref = json.loads(hdr)
    path = tmp_path / "fixture.safetensors"
    with open(path, "wb") as g:
        g.write(struct.pack("<Q", len(hdr)))
        g.write(hdr)
        g.truncate(8 + len(hdr) + meta["data_size"])  # sparse zero data region
    f = SafetensorsFile(path)
    tensors = {k: v for k, v in ref.items() if k != "__metadata__"}
    assert len(f.tensors) == len(tensors) == 504
    assert list(f.tensors) == list(tensors)
    for k, v in tensors.items():
        t = f.tensors[k]
        assert (t["dtype"], t["shape"]) == (v["dtype"], v["shape"])
        assert t["offset"] == 8 + len(hdr) + v["data_offsets"][0]
        assert t["nbytes"] == v["data_offsets"][1] - v["data_offsets"][0]
    assert f.metadata == ref["__metadata__"]
    f.close()


@pytest.mark.skipif(not os.path.exists(REF_FILE), reason="the reference checkout is not on this machine")
def test_reference_file_bytes():
    """The reference's fixture file itself: header fields and tensor bytes (sha256) against a
    stdlib parse of the same file."""
    f = SafetensorsFile(REF_FILE)
    raw = open(REF_FILE, "rb").read()
    n = int.from_bytes(raw[:8], "little")
    hdr = json.loads(raw[8:8 + n])
    names = [k for k in hdr if k != "__metadata__"]
    for k in names[:3] + names[-3:]:
        b, e = hdr[k]["data_offsets"]
        got = f.read(k).tobytes()
        assert hashlib.sha256(got).hexdigest() == hashlib.sha256(raw[8 + n + b:8 + n + e]).hexdigest()


def test_sharded_index(tmp_path):
    a = np.arange(6, dtype=np.float32)
    b = np.arange(4, dtype=np.int16)
    st_writer.write(tmp_path / "model-00001-of-00002.safetensors", [("x.a", a)])
    st_writer.write(tmp_path / "model-00002-of-00002.safetensors", [("x.b", b), ("x.c", a)])
    st_writer.write_index(tmp_path / "model.safetensors.index.json",
                          {"x.a": "model-00001-of-00002.safetensors", "x.b": "model-00002-of-00002.safetensors",
                           "x.missing": "model-00002-of-00002.safetensors"})
    ck = Checkpoint(tmp_path)
    f, t = ck.locate("x.b")
    assert os.path.basename(f.path) == "model-00002-of-00002.safetensors" and t["dtype"] == "I16"
    np.testing.assert_array_equal(f.read("x.b"), b)
    assert "x.a" in ck and "x.c" not in ck  # the index, not a scan, decides
    with pytest.raises(KeyError):
        ck.locate("x.missing")  # listed, but absent from its shard
    # without an index: every shard is searched
    os.remove(tmp_path / "model.safetensors.index.json")
    ck2 = Checkpoint(tmp_path)
    assert "x.c" in ck2 and "x.a" in ck2


def _bad(tmp_path, text=None, raw=None, data=b""):
    p = tmp_path / "bad.safetensors"
    if raw is None:
        body = text.encode()
        raw = struct.pack("<Q", len(body)) + body + data
    open(p, "wb").write(raw)
    with pytest.raises(_lib.VybdqError):
        SafetensorsFile(p)


def test_malformed_files(tmp_path):
    ok = '{"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}'
    _bad(tmp_path, raw=b"\x01\x00")                                   # shorter than 8 bytes
    _bad(tmp_path, raw=struct.pack("<Q", 1000) + b"{}")               # header past the end
    _bad(tmp_path, ok, data=b"\0" * 4)                                # data past the end
    _bad(tmp_path, ok.replace("[2]", "[3]"), data=b"\0" * 8)          # shape x size != bytes
    _bad(tmp_path, ok.replace("[0, 8]", "[8, 0]"), data=b"\0" * 8)    # end < begin
    _bad(tmp_path, '{"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}, '
                   '"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}', data=b"\0" * 8)  # duplicate
    _bad(tmp_path, ok[:-1] + ",}", data=b"\0" * 8)                    # trailing comma
    _bad(tmp_path, '{"__metadata__": {"a": 1}}')                      # non-string metadata
    _bad(tmp_path, '{"t": {"dtype": "F32", "shape": [2]}}')           # missing data_offsets
    _bad(tmp_path, '{"t": {"dtype": "F32", "shape": [-2], "data_offsets": [0, 8]}}', data=b"\0" * 8)
    _bad(tmp_path, '[1, 2]')                                          # not an object
    _bad(tmp_path, ok + " x", data=b"\0" * 8)                         # trailing garbage
    _bad(tmp_path, '{"\\ud800": 1}')                                  # lone surrogate
    _bad(tmp_path, "[" * 100 + "]" * 100)                             # nested too deeply
    # padding spaces after the object are the container's alignment and accepted
    p = tmp_path / "pad.safetensors"
    body = (ok + "      ").encode()
    open(p, "wb").write(struct.pack("<Q", len(body)) + body + b"\0" * 8)
    assert SafetensorsFile(p).tensors["t"]["shape"] == [2]
