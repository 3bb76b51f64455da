"""A minimal GGUF v3 writer for the tests (the GGUF specification's layout, written
independently of the library's reader): metadata of every value type, tensor infos with
offsets relative to the data section, the data section aligned to general.alignment."""

import struct

import numpy as np

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == 8:
        return _str(v)
    if t == 9:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += _value(et, it)
        return out
    return struct.pack(_SCALAR[t], v)


def write_gguf(path, kv, tensors, alignment=32):
    """kv: list of (key, value type, value); tensors: list of (name, dims, ggml type, bytes).
    Returns the data section start and each tensor's relative offset."""
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv))
    meta = b"".join(_str(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in kv)
    offsets, cur = [], 0
    for _, _, _, data in tensors:
        cur = (cur + alignment - 1) // alignment * alignment
        offsets.append(cur)
        cur += len(data)
    infos = b""
    for (name, dims, ty, _), off in zip(tensors, offsets):
        infos += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", ty, off)
    body = head + meta + infos
    base = (len(body) + alignment - 1) // alignment * alignment
    out = bytearray(body + b"\0" * (base - len(body)))
    for (_, _, _, data), off in zip(tensors, offsets):
        end = base + off
        out += b"\0" * (end - len(out))
        out += bytes(np.asarray(data, np.uint8).tobytes())
    with open(path, "wb") as f:
        f.write(out)
    return base, offsets
