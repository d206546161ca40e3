"""A small .q4nx (safetensors) writer for the tests: an 8-byte little-endian header
length, the JSON header of name -> {dtype, shape, data_offsets} plus "__metadata__",
then the tensors' bytes back to back."""
from __future__ import annotations

import json
import struct

import numpy as np


def write_q4nx(path, tensors, metadata=None, pad_header_to: int = 8) -> dict:
    """``tensors``: [(name, dtype string, shape, bytes / array)]. Returns the header written."""
    header, blobs, off = {}, [], 0
    for name, dtype, shape, payload in tensors:
        data = np.ascontiguousarray(payload).view(np.uint8).reshape(-1).tobytes()
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(data)]}
        blobs.append(data)
        off += len(data)
    if metadata:
        header["__metadata__"] = dict(metadata)
    text = json.dumps(header).encode()
    text += b" " * (-len(text) % pad_header_to)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)))
        f.write(text)
        for b in blobs:
            f.write(b)
    return header
