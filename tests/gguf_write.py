"""A GGUF writer for tests, from ggml's published file-format description
(docs/gguf.md in the ggml / llama.cpp repositories): independent of the
reference's reader (gguf.mojo) and of libllmq's, so that both can be
checked against files whose layout is known.

    GGUF   magic "GGUF", u32 version, u64 tensor count, u64 metadata count
    kv     gguf_string key, u32 value type, value
    info   gguf_string name, u32 n_dims, u64 dims[n_dims] (dims[0] the
           contiguous one), u32 ggml type, u64 offset into the data section
    data   starts at the next multiple of general.alignment (default 32);
           each tensor's offset is a multiple of the alignment

gguf_string = u64 length + UTF-8 bytes; all little-endian.
"""
import struct

import numpy as np

# metadata value types (gguf.md "gguf_metadata_value_type")
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64: "<d"}


def _gstr(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STRING:
        return _gstr(v)
    if t == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_SCALAR[t], v)


def write(path, tensors, metadata=(), version=3, alignment=None):
    """tensors: [(name, ggml_type, dims, data bytes)]; metadata: [(key,
    type, value)] (arrays as (element type, [values])).  A general.alignment
    entry is added when alignment is given.  Returns the data section's
    start and each tensor's offset."""
    meta = list(metadata)
    align = 32
    if alignment is not None:
        meta.append(("general.alignment", U32, alignment))
        align = alignment
    out = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta)))
    for key, t, v in meta:
        out += _gstr(key) + struct.pack("<I", t) + _value(t, v)
    offsets, off = [], 0
    for name, gt, dims, data in tensors:
        offsets.append(off)
        out += _gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", gt, off)
        off += (len(data) + align - 1) // align * align
    start = (len(out) + align - 1) // align * align
    out += bytes(start - len(out))
    for (name, gt, dims, data), o in zip(tensors, offsets):
        assert len(out) == start + o
        out += data + bytes((len(data) + align - 1) // align * align - len(data))
    with open(path, "wb") as f:
        f.write(bytes(out))
    return start, offsets


def f32_bytes(a):
    return np.ascontiguousarray(a, np.float32).tobytes()


def f16_bytes(a):
    return np.ascontiguousarray(a, np.float16).tobytes()
