"""A GGUF v3 writer for the tests, written from the published format description (magic
"GGUF", version, tensor and metadata counts, typed key/value pairs, tensor records
name / n_dims / ne[] / ggml type / data offset, data section aligned to general.alignment,
default 32), with struct.pack for every field so that it shares nothing with the reader."""
import struct

import numpy as np

# metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vt, v) -> bytes:
    if vt == STR:
        return _str(v)
    if vt == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[vt], v)


def write_gguf(path, tensors, kv=(), alignment=None, version=3):
    """tensors: (name, ggml_type, ne list, payload bytes); kv: (key, value type, value)."""
    kv = list(kv)
    if alignment is not None:
        kv.append(("general.alignment", U32, alignment))
    align = alignment or 32
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, vt, v in kv:
        head += _str(key) + struct.pack("<I", vt) + _value(vt, v)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        offsets.append(off)
        off = (off + len(data) + align - 1) // align * align
    for (name, t, ne, _), o in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", t, o)
    start = (len(head) + align - 1) // align * align
    blob = bytearray(head + b"\0" * (start - len(head)))
    for (_, _, _, data), o in zip(tensors, offsets):
        blob += b"\0" * (start + o - len(blob))
        blob += bytes(np.asarray(data, np.uint8))
    with open(path, "wb") as f:
        f.write(blob)
    return start, [start + o for o in offsets]
