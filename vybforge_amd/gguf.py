"""GGUF files on the device: index a GGUF file and upload every tensor into one slab.

Host mirror of the vybdq_gguf_* entry points (include/vybdq.h); the parsing and the upload are
native code in libvybdq. Replaces the reference's GGUF readers (native/gguf/parse_gguf.vyb,
read_real_meta.vyb) and its resident packed slab (native/host/ridge_decode.vyb:1-3).
"""

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import call

VALUE_TYPES = {0: "u8", 1: "i8", 2: "u16", 3: "i16", 4: "u32", 5: "i32", 6: "f32", 7: "bool", 8: "str",
               9: "array", 10: "u64", 11: "i64", 12: "f64"}


def _check(v, where):
    if v < -1 or (v == -1 and where.endswith("open")):
        raise _lib.VybdqError(v, where, _lib.last_error())
    return v


def _text(fn, *args):
    n = fn(*args, None, 0)
    if n < 0:
        raise _lib.VybdqError(n, fn.__name__, _lib.last_error())
    buf = ctypes.create_string_buffer(n + 1)
    fn(*args, buf, n + 1)
    return buf.value.decode("utf-8", "replace")


class GgufFile:
    """An indexed GGUF file: ``tensors`` (name -> dict of type, dims, offset, nbytes) and
    ``kv`` (key -> (value type name, value; arrays as (element type, length)))."""

    def __init__(self, path):
        lib = _lib.lib
        self.h = lib.vybdq_gguf_open(str(path).encode())
        if self.h < 1:
            raise _lib.VybdqError(self.h, "vybdq_gguf_open", _lib.last_error())
        info = lambda w: lib.vybdq_gguf_info(self.h, w)
        self.version, self.alignment, self.data_base = info(0), info(3), info(5)
        self.tensors = {}
        for i in range(info(1)):
            name = _text(lib.vybdq_gguf_tensor_name, self.h, i)
            nd = lib.vybdq_gguf_tensor_field(self.h, i, 1)
            self.tensors[name] = dict(
                index=i, type=lib.vybdq_gguf_tensor_field(self.h, i, 0),
                dims=[lib.vybdq_gguf_tensor_field(self.h, i, 2 + d) for d in range(nd)],
                offset=lib.vybdq_gguf_tensor_field(self.h, i, -1), nbytes=lib.vybdq_gguf_tensor_field(self.h, i, -2))
        self.kv = {}
        for i in range(info(2)):
            key = _text(lib.vybdq_gguf_kv_key, self.h, i)
            t = lib.vybdq_gguf_kv_field(self.h, i, 0)
            if t == 8:
                v = _text(lib.vybdq_gguf_kv_string, self.h, i)
            elif t == 9:
                v = (VALUE_TYPES.get(lib.vybdq_gguf_kv_field(self.h, i, 2), "?"), lib.vybdq_gguf_kv_field(self.h, i, 3))
            elif t in (6, 12):
                v = lib.vybdq_gguf_kv_float(self.h, i)
            else:
                v = lib.vybdq_gguf_kv_field(self.h, i, 1)
                v = bool(v) if t == 7 else v
            self.kv[key] = (VALUE_TYPES.get(t, "?"), v)

    def close(self):
        if self.h > 0:
            call("vybdq_gguf_close", self.h)
            self.h = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def read_tensor(self, name, absolute=False):
        """The tensor's packed bytes (numpy uint8)."""
        t = self.tensors[name]
        out = np.empty(max(t["nbytes"], 0), np.uint8)
        n = _lib.lib.vybdq_gguf_read_tensor(self.h, t["index"], int(absolute), out.ctypes.data, out.size)
        if n < 0:
            raise _lib.VybdqError(n, "vybdq_gguf_read_tensor", _lib.last_error())
        return out

    def load_slab(self, device, align=256, absolute=False):
        """Every tensor in one device buffer: (slab uint8 tensor, name -> uint8 view of the slab)."""
        lib = _lib.lib
        nbytes = lib.vybdq_gguf_slab_bytes(self.h, align)
        if nbytes < 0:
            raise _lib.VybdqError(nbytes, "vybdq_gguf_slab_bytes", _lib.last_error())
        slab = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        call("vybdq_gguf_load_slab", self.h, slab.data_ptr(), slab.numel(), align, int(absolute),
             torch.cuda.current_stream(device).cuda_stream)
        views = {}
        for name, t in self.tensors.items():
            off = lib.vybdq_gguf_slab_offset(self.h, t["index"], align)
            views[name] = slab[off:off + t["nbytes"]]
        return slab, views
