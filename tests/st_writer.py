"""A safetensors writer for tests, written from the container description (u64 LE header length,
JSON header, raw little-endian data; offsets relative to the data region), independent of the
native reader it exercises."""

import json
import struct

import numpy as np

NP_NAME = {np.dtype(np.float64): "F64", np.dtype(np.float32): "F32", np.dtype(np.float16): "F16",
           np.dtype(np.int64): "I64", np.dtype(np.int32): "I32", np.dtype(np.int16): "I16",
           np.dtype(np.int8): "I8", np.dtype(np.uint8): "U8", np.dtype(np.uint16): "U16",
           np.dtype(np.uint32): "U32", np.dtype(np.uint64): "U64", np.dtype(np.bool_): "BOOL"}


def write(path, tensors, metadata=None, align=8, header_override=None):
    """tensors: list of (name, array) or (name, dtype_str, shape, raw_bytes). Returns the header
    dict that was written."""
    hdr, blobs, off = {}, [], 0
    if metadata is not None:
        hdr["__metadata__"] = metadata
    for t in tensors:
        if len(t) == 2:
            name, a = t
            a = np.asarray(a)  # tobytes() is C order; ascontiguousarray would make a 0-d array 1-d
            dt, shape, raw = NP_NAME[a.dtype], list(a.shape), a.tobytes()
        else:
            name, dt, shape, raw = t
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    text = header_override if header_override is not None else json.dumps(hdr)
    body = text.encode("utf-8")
    body += b" " * (-(8 + len(body)) % align)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(body)))
        f.write(body)
        for b in blobs:
            f.write(b)
    return hdr


def write_index(path, weight_map, metadata=None):
    with open(path, "w") as f:
        json.dump({"metadata": metadata or {}, "weight_map": weight_map}, f)
