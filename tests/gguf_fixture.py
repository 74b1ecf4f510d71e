"""GGUF v3 files for the loader tests, written from the published container
layout (ggml's docs/gguf.md, the format gguf-py writes for SAM.cpp's
converter, tools/convert/sam3_gguf.py:392-445):

    "GGUF" | u32 version=3 | u64 tensor_count | u64 kv_count
    kv:     string key | u32 value type | value
    tensor: string name | u32 n_dims | u64 ne[n_dims] | u32 ggml type | u64 offset
    zero padding to general.alignment (32), then the tensor blob, each tensor
    at its 32-aligned offset and zero-padded to the next multiple of 32.

Strings are u64 length + bytes (no NUL); arrays are u32 element type + u64
count + elements; all integers little-endian.  This writer is independent of
the C++ reader it checks.

`probe_fixture` is the small container of the reference's loader contract
test (tests/api/test_contracts.cpp:84-110) and `text_at` / `integer_at` its
byte-mutation helpers (:149-165).
"""

import struct

import numpy as np

# gguf value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64: "<d"}

# ggml tensor types: (block elements, block bytes)
GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K = 0, 1, 8, 12, 13, 14
GGML_BLOCK = {0: (1, 4), 1: (1, 2), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}
ALIGNMENT = 32


def _string(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vtype, value):
    if vtype == STRING:
        return _string(value)
    if vtype == ARRAY:
        etype, items = value
        out = struct.pack("<IQ", etype, len(items))
        for item in items:
            out += _string(item) if etype == STRING else struct.pack(_SCALAR[etype], item)
        return out
    return struct.pack(_SCALAR[vtype], value)


def tensor_nbytes(ggml_type, ne):
    be, bb = GGML_BLOCK[ggml_type]
    n = int(np.prod(ne, dtype=np.int64))
    assert ne[0] % be == 0
    return n // be * bb


def gguf_bytes(kv, tensors):
    """kv: [(key, vtype, value)], value of an ARRAY = (element type, items).
    tensors: [(name, ne, ggml_type, payload bytes)], ne innermost first."""
    meta = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv))
    for key, vtype, value in kv:
        meta += _string(key) + struct.pack("<I", vtype) + _value(vtype, value)
    offset = 0
    blob = b""
    for name, ne, ggml_type, payload in tensors:
        assert len(payload) == tensor_nbytes(ggml_type, ne), name
        dims = list(ne)
        while len(dims) > 1 and dims[-1] == 1:    # ggml_n_dims: trailing 1s are not written
            dims.pop()
        meta += _string(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        meta += struct.pack("<IQ", ggml_type, offset)
        pad = (-len(payload)) % ALIGNMENT
        blob += payload + b"\0" * pad
        offset += len(payload) + pad
    meta += b"\0" * ((-len(meta)) % ALIGNMENT)
    return meta + blob


def write_gguf(path, kv, tensors):
    data = gguf_bytes(kv, tensors)
    with open(path, "wb") as f:
        f.write(data)
    return data


PROBE_VALUES = np.array([-2, -1, 0, 1, 2, 3], dtype=np.float32)


def probe_fixture(extra_kv=(), second_tensor=False):
    """The reference's write_fixture: one F32 tensor probe.weight with
    ne = (1, 3, 2) holding -2..3, typed probe metadata, optionally a second
    tensor other.weight with the same contents."""
    kv = [("general.architecture", STRING, "sam3"),
          ("sam.schema_version", U32, 1),
          ("sam.task", STRING, "text_image"),
          ("probe.scalar", U32, 17),
          ("probe.label", STRING, "labelx"),
          ("probe.indices", ARRAY, (U32, [3, 5])),
          ("probe.labels", ARRAY, (STRING, ["first", "second"]))]
    kv += list(extra_kv)
    tensors = [("probe.weight", (1, 3, 2), GGML_F32, PROBE_VALUES.tobytes())]
    if second_tensor:
        tensors.append(("other.weight", (1, 3, 2), GGML_F32, PROBE_VALUES.tobytes()))
    return gguf_bytes(kv, tensors)


def text_at(data, text):
    """Offset of the first occurrence of `text` (the test's text_at)."""
    i = bytes(data).find(text.encode())
    assert i >= 0, text
    return i


def integer_at(data, offset, value, width=8):
    """Overwrite `width` little-endian bytes at `offset` (the test's integer_at)."""
    assert offset + width <= len(data)
    data[offset:offset + width] = (value & ((1 << (8 * width)) - 1)).to_bytes(width, "little")
