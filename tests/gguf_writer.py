"""A small GGUF (v3) writer for the tests: synthetic model files with chosen metadata and
tensors, written from the GGUF format description (little-endian; magic, version, tensor
and metadata counts; typed key/value pairs; tensor infos with fastest-first dims, ggml
type and data offset; tensor data from the next multiple of ``general.alignment``, each
tensor starting on such a multiple)."""
from __future__ import annotations

import struct

import numpy as np

# metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}

# ggml tensor types used here: name -> (id, values per block, bytes per block)
TYPES = {"F32": (0, 1, 4), "F16": (1, 1, 2), "Q4_0": (2, 32, 18), "Q4_1": (3, 32, 20),
         "Q8_0": (8, 32, 34), "Q4_K": (12, 256, 144), "BF16": (30, 1, 2)}


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(vt: int, v) -> bytes:
    if vt == STR:
        return _str(v)
    if vt == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[vt], v)


def write_gguf(path, tensors, metadata=(), alignment: int | None = None, version: int = 3) -> None:
    """``tensors``: [(name, type_name, shape slowest-first, payload bytes / uint8 array)].
    ``metadata``: [(key, value_type, value)], an array value being (element_type, items).
    ``alignment`` adds ``general.alignment`` (u32) and aligns to it; default 32."""
    meta = list(metadata)
    align = 32
    if alignment is not None:
        meta.append(("general.alignment", U32, alignment))
        align = alignment
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    for key, vt, v in meta:
        head += _str(key) + struct.pack("<I", vt) + _value(vt, v)
    blobs, off = [], 0
    for name, tname, shape, payload in tensors:
        tid, per_block, block_bytes = TYPES[tname]
        data = np.ascontiguousarray(payload).view(np.uint8).reshape(-1).tobytes()
        count = int(np.prod(shape))
        if count // per_block * block_bytes != len(data):
            raise ValueError(f"{name}: {len(data)} bytes do not hold {shape} of {tname}")
        dims = list(reversed(shape))
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", tid, off)
        blobs.append((off, data))
        off = (off + len(data) + align - 1) // align * align
    start = (len(head) + align - 1) // align * align
    out = bytearray(head + b"\0" * (start - len(head)))
    for o, data in blobs:
        out += b"\0" * (start + o - len(out))
        out += data
    with open(path, "wb") as f:
        f.write(bytes(out))
