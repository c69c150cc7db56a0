"""Minimal GGUF (version 3) writer for the tests: metadata of every value type
and tensors with their raw bytes, each tensor's data aligned as the format
requires. Test infrastructure, written from the format description."""
from __future__ import annotations

import struct

STRING, ARRAY = 8, 9
SCALAR_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?",
              10: "<Q", 11: "<q", 12: "<d"}
GGML = {"F32": 0, "F16": 1, "Q4_0": 2, "Q5_0": 6, "Q8_0": 8, "BF16": 30, "I32": 26}


def _string(s) -> bytes:
    b = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, value, elem: int | None = None) -> bytes:
    if vtype == STRING:
        return _string(value)
    if vtype == ARRAY:
        out = struct.pack("<IQ", elem, len(value))
        for v in value:
            out += _value(elem, v)
        return out
    return struct.pack(SCALAR_FMT[vtype], value)


def gguf_bytes(kvs, tensors, alignment=32, version=3, magic=b"GGUF") -> bytes:
    """kvs: [(key, value type, value[, element type])];
    tensors: [(name, ggml type code, dims in file order, data bytes)]."""
    out = bytearray(magic + struct.pack("<IQQ", version, len(tensors), len(kvs)))
    for kv in kvs:
        key, vtype, value = kv[:3]
        out += _string(key) + struct.pack("<I", vtype) + _value(vtype, value, *kv[3:])
    offsets, pos = [], 0
    for name, gtype, dims, data in tensors:
        pos = (pos + alignment - 1) // alignment * alignment
        offsets.append(pos)
        pos += len(data)
    for (name, gtype, dims, data), off in zip(tensors, offsets):
        out += _string(name) + struct.pack("<I", len(dims))
        out += b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", gtype, off)
    start = (len(out) + alignment - 1) // alignment * alignment
    out += bytes(start - len(out))
    for (name, gtype, dims, data), off in zip(tensors, offsets):
        out += bytes(start + off - len(out)) + data
    return bytes(out)
