"""GGUF files in: the tensors of a llama.cpp GGUF model, zero-copy, and their
Q4 weights packed for the kernels.

The counterpart of the reference's GGUF readers (open_kernels/model/gguf_ref.py:
the header walk and the ggml block laws; gguf_pool/gguf_pool.py: the direct-GGUF
pool). Here a weight goes from the file's own block bytes straight to the mx
layout on the GPU:

  * Q4_1 / Q4_0 blocks -> ``q4_repack`` (bit-exact codes, d and m narrowed to
    bf16 as the reference pool does);
  * Q4_K super-blocks -> ``q4_repack_q4k`` (each 32-value sub-block is a Q4_1
    block with d*sc and -dmin*min, exact products narrowed to bf16).

Layout facts used (the GGUF v2/v3 format): little-endian; magic ``GGUF``; version;
tensor and metadata counts (uint64); metadata key/value pairs; tensor infos (name,
dims fastest-first, ggml type, data offset); the data section starts at the next
multiple of ``general.alignment`` (default 32) after the header.
"""
from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

# ggml tensor types this reader knows: id -> (name, values per block, bytes per block)
GGML_TYPES = {
    0: ("F32", 1, 4),
    1: ("F16", 1, 2),
    2: ("Q4_0", 32, 18),
    3: ("Q4_1", 32, 20),
    8: ("Q8_0", 32, 34),
    12: ("Q4_K", 256, 144),
    30: ("BF16", 1, 2),
}
Q4_TYPES = {"Q4_0", "Q4_1", "Q4_K"}

# metadata value types: id -> struct format (8 string, 9 array handled apart)
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


class GGUFError(ValueError):
    """A file that is not a GGUF this reader can use (the message says why)."""


@dataclass(frozen=True)
class GGUFTensor:
    name: str
    type_id: int
    shape: tuple               # slowest-first: (rows, cols) for a weight [out, in]
    offset: int                # absolute byte offset in the file
    nbytes: int

    @property
    def type_name(self) -> str:
        return GGML_TYPES[self.type_id][0]


class GGUFFile:
    """A GGUF file, memory-mapped; tensors are read on demand without copies."""

    def __init__(self, path):
        self.path = Path(path)
        self._fh = open(self.path, "rb")
        try:
            self._mm = mmap.mmap(self._fh.fileno(), 0, access=mmap.ACCESS_READ)
        except ValueError as e:                      # empty file
            self._fh.close()
            raise GGUFError(f"{self.path.name}: not a GGUF ({e})") from None
        self._pos = 0
        try:
            self._parse()
        except (struct.error, UnicodeDecodeError, IndexError) as e:
            self.close()
            raise GGUFError(f"{self.path.name}: truncated or corrupt header ({e})") from None
        except GGUFError:
            self.close()
            raise

    # ---- header -------------------------------------------------------
    def _take(self, fmt: str):
        v = struct.unpack_from(fmt, self._mm, self._pos)[0]
        self._pos += struct.calcsize(fmt)
        return v

    def _string(self) -> str:
        n = self._take("<Q")
        if n > len(self._mm) - self._pos:
            raise GGUFError(f"{self.path.name}: string of {n} bytes runs past the file")
        s = bytes(self._mm[self._pos:self._pos + n]).decode("utf-8")
        self._pos += n
        return s

    def _value(self, vt: int):
        if vt in _SCALAR:
            return self._take(_SCALAR[vt])
        if vt == 8:
            return self._string()
        if vt == 9:
            et, n = self._take("<I"), self._take("<Q")
            if et == 9:
                raise GGUFError(f"{self.path.name}: nested metadata arrays are not supported")
            return [self._value(et) for _ in range(n)]
        raise GGUFError(f"{self.path.name}: unknown metadata value type {vt}")

    def _parse(self):
        if bytes(self._mm[0:4]) != b"GGUF":
            raise GGUFError(f"{self.path.name}: not a GGUF (bad magic)")
        self._pos = 4
        self.version = self._take("<I")
        if self.version not in (2, 3):
            raise GGUFError(f"{self.path.name}: GGUF version {self.version} is not supported (2, 3 are)")
        n_tensors, n_kv = self._take("<Q"), self._take("<Q")
        self.metadata: dict = {}
        for _ in range(n_kv):
            key = self._string()
            self.metadata[key] = self._value(self._take("<I"))
        infos = []
        for _ in range(n_tensors):
            name = self._string()
            nd = self._take("<I")
            dims = [self._take("<Q") for _ in range(nd)]
            infos.append((name, dims, self._take("<I"), self._take("<Q")))
        align = int(self.metadata.get("general.alignment", 32))
        if align <= 0 or align & (align - 1):
            raise GGUFError(f"{self.path.name}: alignment {align} is not a power of two")
        self.data_start = (self._pos + align - 1) // align * align
        self.tensors: dict[str, GGUFTensor] = {}
        for name, dims, ty, off in infos:
            if ty not in GGML_TYPES:
                raise GGUFError(f"{self.path.name}: tensor {name!r} has ggml type {ty}; this reader knows "
                                f"{sorted(v[0] for v in GGML_TYPES.values())}")
            _, per_block, block_bytes = GGML_TYPES[ty]
            if not dims or dims[0] % per_block:
                raise GGUFError(f"{self.path.name}: tensor {name!r} row of {dims[:1]} is not whole blocks")
            count = int(np.prod(dims, dtype=np.int64))
            nbytes = count // per_block * block_bytes
            start = self.data_start + off
            if off % align or start + nbytes > len(self._mm):
                raise GGUFError(f"{self.path.name}: tensor {name!r} data is misaligned or runs past the file")
            self.tensors[name] = GGUFTensor(name, ty, tuple(int(d) for d in reversed(dims)), start, nbytes)

    # ---- tensors ------------------------------------------------------
    def tensor(self, name: str) -> GGUFTensor:
        try:
            return self.tensors[name]
        except KeyError:
            raise GGUFError(f"{self.path.name}: no tensor {name!r}") from None

    def raw(self, name: str) -> np.ndarray:
        """The tensor's bytes as uint8, a view of the mapped file."""
        t = self.tensor(name)
        return np.frombuffer(self._mm, dtype=np.uint8, count=t.nbytes, offset=t.offset)

    def blocks(self, name: str) -> np.ndarray:
        """A quantized matrix [rows, cols] as its blocks uint8[rows, cols / per_block, block_bytes]."""
        t = self.tensor(name)
        _, per_block, block_bytes = GGML_TYPES[t.type_id]
        if per_block == 1:
            raise GGUFError(f"{name!r} is {t.type_name}, not a block-quantized type")
        cols = t.shape[-1]
        rows = t.nbytes // (cols // per_block * block_bytes)
        return self.raw(name).reshape(rows, cols // per_block, block_bytes)

    def array(self, name: str) -> np.ndarray:
        """An F32 / F16 / BF16 tensor as float32 (a copy), in its slowest-first shape."""
        t = self.tensor(name)
        raw = self.raw(name)
        if t.type_name == "F32":
            a = raw.view(np.float32).copy()
        elif t.type_name == "F16":
            a = raw.view(np.float16).astype(np.float32)
        elif t.type_name == "BF16":
            a = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        else:
            raise GGUFError(f"{name!r} is {t.type_name}; use blocks() or packed()")
        return a.reshape(t.shape)

    def packed(self, name: str, device=None, q4k: str = "mx"):
        """A Q4_0 / Q4_1 / Q4_K weight [N, K] (N % 64 == 0) packed for the kernels on the GPU
        (a PackedQ4), or a Q8_0 one as the exact q8 pair (a PackedQ8, for gemm_q8). A Q4_K
        weight goes to the mx layout (``q4k="mx"``: d sc and m mn rounded to bf16, for every
        kernel) or stays Q4_K (``q4k="native"``: a PackedQ4K for gemm_q4k, exact)."""
        from . import q4                                  # needs the HIP library: imported on use
        t = self.tensor(name)
        if t.type_name not in Q4_TYPES | {"Q8_0"}:
            raise GGUFError(f"{name!r} is {t.type_name}; the kernels take {sorted(Q4_TYPES | {'Q8_0'})}")
        if len(t.shape) != 2:
            raise GGUFError(f"{name!r} has shape {t.shape}, not a matrix")
        b = self.blocks(name)
        if t.type_name == "Q8_0":
            return q4.pack_q8(b, t.shape[0], t.shape[1], fmt="q8_0", device=device)
        if t.type_name == "Q4_K":
            if q4k not in ("mx", "native"):
                raise ValueError(f"q4k must be 'mx' or 'native', got {q4k!r}")
            return q4.pack_q4_k_native(b, device) if q4k == "native" else q4.pack_q4_k(b, device)
        return q4.pack_q4_1(b, device)

    # ---- lifetime -----------------------------------------------------
    def close(self):
        mm, self._mm = getattr(self, "_mm", None), None
        if mm is not None:
            try:
                mm.close()
            except BufferError:                      # a returned view is still alive: let GC close it
                pass
        if getattr(self, "_fh", None) is not None:
            self._fh.close()
            self._fh = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
