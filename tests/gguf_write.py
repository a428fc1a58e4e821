"""A small GGUF writer for the tests, written from the format's description (magic, version,
counts, metadata key/value pairs, tensor directory with dims innermost first, tensor data at
offsets aligned to general.alignment, default 32). Test helper only."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q", I64: "<q",
        F64: "<d"}


def _len(n, version):
    return struct.pack("<I" if version == 1 else "<Q", n)


def _str(s, version):
    b = s.encode()
    return _len(len(b), version) + b


def _value(vt, v, version):
    if vt == STRING:
        return _str(v, version)
    if vt == ARRAY:
        et, items = v
        return struct.pack("<I", et) + _len(len(items), version) + b"".join(_value(et, x, version) for x in items)
    return struct.pack(_FMT[vt], v)


def gguf_bytes(meta, tensors, version=3, alignment=32):
    """meta: [(key, type, value)]; tensors: [(name, ggml type id, dims outermost first, raw bytes)].
    Returns (file bytes, offset of the tensor data, [offset of each tensor within the data])."""
    head = b"GGUF" + struct.pack("<I", version) + _len(len(tensors), version) + _len(len(meta), version)
    for key, vt, v in meta:
        head += _str(key, version) + struct.pack("<I", vt) + _value(vt, v, version)
    offs, pos = [], 0
    for _, _, _, raw in tensors:
        pos = (pos + alignment - 1) // alignment * alignment
        offs.append(pos)
        pos += len(raw)
    for (name, gt, dims, _), off in zip(tensors, offs):
        head += _str(name, version) + struct.pack("<I", len(dims))
        for d in reversed(dims):
            head += struct.pack("<I" if version == 1 else "<Q", d)
        head += struct.pack("<I", gt) + struct.pack("<Q", off)
    data_off = (len(head) + alignment - 1) // alignment * alignment
    body = bytearray(head + b"\0" * (data_off - len(head)))
    for (_, _, _, raw), off in zip(tensors, offs):
        body += b"\0" * (data_off + off - len(body))
        body += bytes(np.asarray(raw, dtype=np.uint8).tobytes())
    return bytes(body), data_off, offs


def write_gguf(path, meta, tensors, version=3, alignment=32):
    data, data_off, offs = gguf_bytes(meta, tensors, version, alignment)
    with open(path, "wb") as f:
        f.write(data)
    return data_off, offs
