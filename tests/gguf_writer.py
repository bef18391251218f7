"""Minimal GGUF v3 writer for tests: the public file layout (magic "GGUF",
version 3, u64 tensor and metadata counts, typed key/values, tensor infos of
name / dims / ggml type / offset, data aligned to general.alignment), as the
reference's reader (src/loader/gguf.rs:297-397) and test builders
(tests/gguf_loader.rs:8-104) use it."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v):
    if vtype == STR:
        return _str(v)
    if vtype == ARR:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        for it in items:
            out += _value(etype, it)
        return out
    return struct.pack(_FMT[vtype], v)


def write_gguf(path, metadata, tensors, alignment=32):
    """metadata: list of (key, vtype, value); tensors: list of (name, shape (GGUF
    order), ggml type id, raw bytes as a uint8 array)."""
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(metadata))
    for key, vtype, val in metadata:
        head += _str(key) + struct.pack("<I", vtype) + _value(vtype, val)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        offsets.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, shape, gtype, _), o in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        head += struct.pack("<IQ", gtype, o)
    pad = (-len(head)) % alignment
    blob = bytearray(head + b"\0" * pad)
    for (_, _, _, data), o in zip(tensors, offsets):
        start = len(head) + pad + o
        if len(blob) < start:
            blob += b"\0" * (start - len(blob))
        blob += np.asarray(data, dtype=np.uint8).tobytes()
    with open(path, "wb") as f:
        f.write(bytes(blob))
