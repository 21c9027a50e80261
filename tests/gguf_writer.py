"""Minimal GGUF v3 writer for tests, from the published GGUF layout:

  "GGUF", u32 version, u64 tensor count, u64 metadata count,
  metadata (gguf string key, u32 value type, value),
  tensor infos (gguf string name, u32 n_dims, u64 ne[n_dims] fastest axis
  first, u32 ggml type, u64 offset from the data section), zero padding to
  general.alignment, then the tensor payloads at their aligned offsets.

A gguf string is a u64 byte length followed by the UTF-8 bytes.  Only F32
(ggml type 0), F16 (1) and BF16 (30) payloads are written.  Metadata values:
str -> string, bool -> bool, int -> u32, float -> f32, and lists of str,
float or int (or tuples ("i32", [...]) / ("f32", [...])) -> arrays.
"""
import struct

import numpy as np

GGML_F32, GGML_F16, GGML_BF16 = 0, 1, 30
_U32, _I32, _F32, _BOOL, _STRING, _ARRAY = 4, 5, 6, 7, 8, 9


def _string(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(v):
    if isinstance(v, str):
        return struct.pack("<I", _STRING) + _string(v)
    if isinstance(v, bool):
        return struct.pack("<IB", _BOOL, int(v))
    if isinstance(v, float):
        return struct.pack("<If", _F32, v)
    if isinstance(v, int):
        return struct.pack("<II", _U32, v)
    kind, items = v if isinstance(v, tuple) else (None, v)
    if kind is None:
        kind = "str" if items and isinstance(items[0], str) else ("f32" if items and isinstance(items[0], float) else "i32")
    if kind == "str":
        return struct.pack("<IIQ", _ARRAY, _STRING, len(items)) + b"".join(_string(x) for x in items)
    if kind == "f32":
        return struct.pack("<IIQ", _ARRAY, _F32, len(items)) + struct.pack(f"<{len(items)}f", *items)
    return struct.pack("<IIQ", _ARRAY, _I32, len(items)) + struct.pack(f"<{len(items)}i", *items)


def write_gguf(path, tensors, alignment=32, ggml_type=GGML_F32, metadata=None):
    """tensors: dict name -> numpy array in PyTorch order."""
    meta = {"general.architecture": "sana", "general.alignment": alignment}
    meta.update(metadata or {})
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta)))
    for k, v in meta.items():
        head += _string(k) + _value(v)
    payloads, offset = [], 0
    for name, arr in tensors.items():
        arr = np.ascontiguousarray(arr, dtype=np.float32)
        if ggml_type == GGML_F32:
            data = arr.tobytes()
        elif ggml_type == GGML_F16:
            data = arr.astype(np.float16).tobytes()
        else:
            data = (arr.view(np.uint32) >> 16).astype(np.uint16).tobytes()  # truncating bf16
        ne = list(reversed(arr.shape)) or [1]
        head += _string(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne)
        head += struct.pack("<IQ", ggml_type, offset)
        payloads.append((offset, data))
        offset += (len(data) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * ((-len(head)) % alignment))
        base = f.tell()
        for off, data in payloads:
            f.seek(base + off)
            f.write(data)
        f.truncate(base + offset)
    return path
