"""safetensors checkpoints on the device: index a file or a sharded checkpoint, upload tensors,
and build an EXL3 linear layer from its named tensors.

Host mirror of the vybdq_st_* entry points (include/vybdq.h); parsing and uploads are native code
in libvybdq. Replaces the reference's native/torchload/safetensors.vyb (the container reader) and
native/glm53/gx.vyb (tensor name -> shard through model.safetensors.index.json). The EXL3 tensors
of one linear layer are <prefix>.trellis (int16 [K/16, N/16, 64]), <prefix>.suh (f16 [K]),
<prefix>.svh (f16 [N]) and <prefix>.mcg (i32 [1], present for the mcg codebook), as listed by
native/glm53/loader.py:20-29.
"""

import ctypes
import os

import numpy as np
import torch

from . import _lib, ops
from ._lib import call

# safetensors dtype spelling -> (numpy dtype, torch dtype); BF16 reads as raw uint16 in numpy
DTYPES = {
    "F64": (np.float64, torch.float64), "F32": (np.float32, torch.float32), "F16": (np.float16, torch.float16),
    "BF16": (np.uint16, torch.bfloat16), "I64": (np.int64, torch.int64), "I32": (np.int32, torch.int32),
    "I16": (np.int16, torch.int16), "I8": (np.int8, torch.int8), "U8": (np.uint8, torch.uint8),
    "U16": (np.uint16, torch.int16), "U32": (np.uint32, torch.int32), "U64": (np.uint64, torch.int64),
    "BOOL": (np.bool_, torch.bool), "F8_E4M3": (np.uint8, torch.float8_e4m3fn),
    "F8_E5M2": (np.uint8, torch.float8_e5m2),
}


def _text(fn, *args):
    n = fn(*args, None, 0)
    if n < 0:
        raise _lib.VybdqError(n, fn.__name__, _lib.last_error())
    buf = ctypes.create_string_buffer(n + 1)
    fn(*args, buf, n + 1)
    return buf.raw[:n].decode("utf-8")


class SafetensorsFile:
    """An indexed safetensors file: ``tensors`` (name -> dict of index, dtype, shape, offset (absolute
    file offset), nbytes) in header order, and ``metadata`` (the __metadata__ strings)."""

    def __init__(self, path):
        lib = _lib.lib
        self.path = str(path)
        self.h = lib.vybdq_st_open(self.path.encode())
        if self.h < 1:
            raise _lib.VybdqError(self.h, "vybdq_st_open", _lib.last_error())
        self.header_len, self.data_base, self.file_size = (lib.vybdq_st_info(self.h, w) for w in (2, 3, 4))
        self.tensors = {}
        for i in range(lib.vybdq_st_info(self.h, 0)):
            name = _text(lib.vybdq_st_tensor_name, self.h, i)
            nd = lib.vybdq_st_tensor_field(self.h, i, 1)
            self.tensors[name] = dict(
                index=i, dtype=_text(lib.vybdq_st_tensor_dtype, self.h, i),
                shape=[lib.vybdq_st_tensor_field(self.h, i, 2 + d) for d in range(nd)],
                offset=lib.vybdq_st_tensor_field(self.h, i, -1), nbytes=lib.vybdq_st_tensor_field(self.h, i, -2))
        self.metadata = {}
        for i in range(lib.vybdq_st_info(self.h, 1)):
            key = _text(lib.vybdq_st_meta_key, self.h, i)
            self.metadata[key] = self.meta(key)

    def meta(self, key):
        """The __metadata__ value of key, or None."""
        n = _lib.lib.vybdq_st_meta(self.h, key.encode(), None, 0)
        if n < 0:
            return None
        buf = ctypes.create_string_buffer(n + 1)
        _lib.lib.vybdq_st_meta(self.h, key.encode(), buf, n + 1)
        return buf.raw[:n].decode("utf-8")

    def close(self):
        if self.h > 0:
            call("vybdq_st_close", self.h)
            self.h = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def read(self, name):
        """The tensor as a host numpy array (BF16 as raw uint16, F8 as raw uint8)."""
        t = self.tensors[name]
        raw = np.empty(max(t["nbytes"], 0), np.uint8)
        n = _lib.lib.vybdq_st_read(self.h, t["index"], raw.ctypes.data, raw.size)
        if n < 0:
            raise _lib.VybdqError(n, "vybdq_st_read", _lib.last_error())
        if t["dtype"] not in DTYPES:
            return raw
        return raw.view(DTYPES[t["dtype"]][0]).reshape(t["shape"])

    def to_device(self, name, device, dtype=None):
        """The tensor uploaded to device memory (torch dtype from the file unless given; unsigned
        16/32/64-bit tensors arrive as the signed type of the same width)."""
        t = self.tensors[name]
        if dtype is None:
            if t["dtype"] not in DTYPES:
                raise ValueError(f"{name}: dtype {t['dtype']} has no device mapping; pass dtype=")
            dtype = DTYPES[t["dtype"]][1]
        esize = torch.empty(0, dtype=dtype).element_size()
        if t["nbytes"] % esize:
            raise ValueError(f"{name}: {t['nbytes']} bytes is not a whole number of {dtype}")
        shape = t["shape"] if t["dtype"] in DTYPES and DTYPES[t["dtype"]][1].itemsize == esize else [t["nbytes"] // esize]
        out = torch.empty(shape, dtype=dtype, device=device)
        n = _lib.lib.vybdq_st_upload(self.h, t["index"], out.data_ptr(), out.numel() * esize,
                                     torch.cuda.current_stream(device).cuda_stream)
        if n < 0:
            raise _lib.VybdqError(n, "vybdq_st_upload", _lib.last_error())
        return out


class Checkpoint:
    """A checkpoint directory: model.safetensors.index.json resolves a tensor to its shard (the
    reference's index-first order, native/glm53/gx.vyb:1-16); without an index every *.safetensors
    file in the directory is searched in name order."""

    def __init__(self, directory):
        lib = _lib.lib
        self.dir = str(directory)
        self.files = {}
        self.shard_of = None
        idx = os.path.join(self.dir, "model.safetensors.index.json")
        if os.path.exists(idx):
            h = lib.vybdq_st_index_open(idx.encode())
            if h < 1:
                raise _lib.VybdqError(h, "vybdq_st_index_open", _lib.last_error())
            try:
                self.shard_of = {}
                for i in range(lib.vybdq_st_index_count(h)):
                    n = lib.vybdq_st_index_entry(h, i, None, 0, None, 0)
                    if n < 0:
                        raise _lib.VybdqError(n, "vybdq_st_index_entry", _lib.last_error())
                    buf = ctypes.create_string_buffer(n + 1)
                    lib.vybdq_st_index_entry(h, i, buf, n + 1, None, 0)
                    name = buf.raw[:n].decode("utf-8")
                    self.shard_of[name] = _text(lib.vybdq_st_index_shard, h, name.encode())
            finally:
                call("vybdq_st_index_close", h)
        else:
            for f in sorted(os.listdir(self.dir)):
                if f.endswith(".safetensors"):
                    self._file(f)

    def _file(self, fname):
        if fname not in self.files:
            self.files[fname] = SafetensorsFile(os.path.join(self.dir, fname))
        return self.files[fname]

    def locate(self, name):
        """(SafetensorsFile, tensor info) for name; KeyError if the checkpoint lacks it."""
        if self.shard_of is not None:
            if name not in self.shard_of:
                raise KeyError(name)
            f = self._file(self.shard_of[name])
            if name not in f.tensors:
                raise KeyError(f"{name}: listed in the index for {self.shard_of[name]} but absent from that shard")
            return f, f.tensors[name]
        for f in self.files.values():
            if name in f.tensors:
                return f, f.tensors[name]
        raise KeyError(name)

    def __contains__(self, name):
        try:
            self.locate(name)
            return True
        except KeyError:
            return False

    def to_device(self, name, device, dtype=None):
        f, _ = self.locate(name)
        return f.to_device(name, device, dtype)

    def close(self):
        for f in self.files.values():
            f.close()
        self.files = {}


def exl3_linear(ckpt, prefix, device, max_batch=16):
    """ops.Exl3Linear from <prefix>.trellis / .suh / .svh (+ .mcg) of a Checkpoint.

    K = 16 * trellis.shape[0], N = 16 * trellis.shape[1]. The codebook must be mcg, the only one
    the reference implements: <prefix>.mcg must be present (its value is not read: the reference
    documents it both as the id 1, native/exl3/exl3_ref.py:11, and as the multiplier 0xCBAC1FED,
    native/exl3/README.md:32). A layer without it (exllamav3's multiply-add codebook) or with
    <prefix>.mul1 is rejected."""
    _, tr = ckpt.locate(prefix + ".trellis")
    if len(tr["shape"]) != 3 or tr["shape"][2] != 64 or tr["dtype"] not in ("I16", "U16"):
        raise ValueError(f"{prefix}.trellis: expected int16 [K/16, N/16, 64], got {tr['dtype']} {tr['shape']}")
    K, N = 16 * tr["shape"][0], 16 * tr["shape"][1]
    for sfx, n in (("suh", K), ("svh", N)):
        _, ti = ckpt.locate(f"{prefix}.{sfx}")
        if ti["dtype"] != "F16" or ti["shape"] != [n]:
            raise ValueError(f"{prefix}.{sfx}: expected F16 [{n}], got {ti['dtype']} {ti['shape']}")
    if f"{prefix}.mul1" in ckpt:
        raise NotImplementedError(f"{prefix}: the mul1 codebook is not supported")
    if f"{prefix}.mcg" not in ckpt:
        raise NotImplementedError(f"{prefix}: no .mcg tensor; only the mcg codebook is supported")
    t = ckpt.to_device(prefix + ".trellis", device, torch.int16)
    suh = ckpt.to_device(prefix + ".suh", device)
    svh = ckpt.to_device(prefix + ".svh", device)
    return ops.Exl3Linear(t, suh, svh, K, N, ops.EXL3_MCG, max_batch=max_batch)


def moe_exl3_layer(ckpt, prefix, device, n_experts, topk=8, scale=2.5, limit=10.0):
    """ops.MoeExl3Layer of one GLM-5.3 MoE layer from a checkpoint, by the reference's tensor names
    (native/glm53/glm_engine.vyb:2733-2736,2845-2862,2955-2960; naming in native/glm53/loader.py:20-35):
    <prefix>mlp.experts.<e>.{gate,up,down}_proj.{trellis,suh,svh,mcg} for e < n_experts (EXL3 4-bpw,
    mcg codebook), <prefix>mlp.shared_experts.{gate,up,down}_proj.weight (bf16 [out, in]) and
    <prefix>mlp.gate.e_score_correction_bias (f32 [E], the selection bias). H and I come from the
    first expert's trellis shapes; every expert must match them."""
    experts = []
    H = I = None
    for e in range(n_experts):
        ep = f"{prefix}mlp.experts.{e}."
        ts = []
        for proj in ("gate_proj", "up_proj", "down_proj"):
            base = ep + proj
            if f"{base}.mcg" not in ckpt:
                raise NotImplementedError(f"{base}: no .mcg tensor; only the mcg codebook is supported")
            _, tr = ckpt.locate(base + ".trellis")
            if len(tr["shape"]) != 3 or tr["shape"][2] != 64 or tr["dtype"] not in ("I16", "U16"):
                raise ValueError(f"{base}.trellis: expected int16 [in/16, out/16, 64], got {tr['dtype']} {tr['shape']}")
            kin, nout = 16 * tr["shape"][0], 16 * tr["shape"][1]
            if proj == "gate_proj" and H is None:
                H, I = kin, nout
            want = (H, I) if proj != "down_proj" else (I, H)
            if (kin, nout) != want:
                raise ValueError(f"{base}.trellis: [in {kin}, out {nout}], expected {want}")
            ts.append(ckpt.to_device(base + ".trellis", device, torch.int16))
            for sfx, n in (("suh", kin), ("svh", nout)):
                _, ti = ckpt.locate(f"{base}.{sfx}")
                if ti["dtype"] != "F16" or ti["shape"] != [n]:
                    raise ValueError(f"{base}.{sfx}: expected F16 [{n}], got {ti['dtype']} {ti['shape']}")
                ts.append(ckpt.to_device(f"{base}.{sfx}", device))
        experts.append(ts)
    shared = None
    sp = f"{prefix}mlp.shared_experts."
    if sp + "gate_proj.weight" in ckpt:
        shared = []
        for proj, shp in (("gate_proj", [I, H]), ("up_proj", [I, H]), ("down_proj", [H, I])):
            _, ti = ckpt.locate(f"{sp}{proj}.weight")
            if ti["dtype"] != "BF16" or ti["shape"] != shp:
                raise ValueError(f"{sp}{proj}.weight: expected BF16 {shp}, got {ti['dtype']} {ti['shape']}")
            shared.append(ckpt.to_device(f"{sp}{proj}.weight", device))
    bias = None
    bname = f"{prefix}mlp.gate.e_score_correction_bias"
    if bname in ckpt:
        bias = ckpt.to_device(bname, device, torch.float32) if ckpt.locate(bname)[1]["dtype"] == "F32" else None
        if bias is None or bias.numel() != n_experts:
            raise ValueError(f"{bname}: expected F32 [{n_experts}]")
    return ops.MoeExl3Layer(experts, H, I, topk=topk, shared=tuple(shared) if shared else None, scale=scale,
                            limit=limit, bias=bias)
