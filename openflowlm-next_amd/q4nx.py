"""`.q4nx` containers in: OFLM's converted models, zero-copy, their matrices packed for
the kernels on the device.

The counterpart of the reference's container readers (open_kernels/model/q4nx.py:178-274,
Q4NX; src/open_qwen36/q4nx_file.cpp/.hpp). The container is a safetensors file -- an
8-byte little-endian header length, a JSON header of tensor name -> {dtype, shape,
data_offsets} (plus an optional "__metadata__" map of strings), then the data. BF16 / F32
tensors are plain row-major. A quantised matrix is an I8 tensor [chunks, chunk_bytes] of
32-row x 256-K chunks in the file's raster order (chunk f covers rows 32 (f // ncol) and
columns 256 (f % ncol), ncol = in / 256), and the chunk format is per tensor:

  5120 B  q4_1 (bf16 d, bf16 m per 32-block)         -> q4_repack_pool, rs = 1 (exact)
  5120 B  the signed quantiser (every min 0)         -> q4_repack_pool_signed (exact)
  8704 B  q8 (bf16 scale per 32-block, int8 codes)   -> q4_repack_q8_chunks (requant_q4_1)
  4736 B  Q4_K (uint8 scales/mins, bf16 S/M per row) -> q4_repack_q4k_chunks

A 5120-byte tensor is the signed form when its first chunk's 256 mins are all exactly
zero (recipes/pack.py:583-603's rule; a container's own "quant_format" metadata for the
tensor, when present, wins). The logical [out, in] shape is not in the container; the
caller gives it, as the reference's dq_tile(raw, out_dim, in_dim) is given it.
"""
from __future__ import annotations

import json
import mmap
import struct
from pathlib import Path

import numpy as np

CHUNK_Q4 = 5120
CHUNK_Q8 = 8704
CHUNK_Q4K = 4736
CHUNK_FORMATS = {CHUNK_Q4: "q4_1", CHUNK_Q8: "q8", CHUNK_Q4K: "q4_k"}
_DTYPES = {"BF16": np.uint16, "F32": np.float32, "F16": np.float16, "I8": np.int8, "U8": np.uint8,
           "I32": np.int32, "I64": np.int64}


class Q4NXError(ValueError):
    """A container this reader cannot use (the message names the file and tensor)."""


class Q4NXFile:
    def __init__(self, path):
        self.path = Path(path)
        self._fh = open(self.path, "rb")
        try:
            self._mm = mmap.mmap(self._fh.fileno(), 0, access=mmap.ACCESS_READ)
        except ValueError:
            self._fh.close()
            raise Q4NXError(f"{self.path.name}: empty file, not a .q4nx") from None
        try:
            self._parse()
        except Exception:
            self.close()
            raise

    def _parse(self):
        size = len(self._mm)
        if size < 8:
            raise Q4NXError(f"{self.path.name}: {size} bytes, too short for a header")
        n = struct.unpack_from("<Q", self._mm, 0)[0]
        if n > size - 8:
            raise Q4NXError(f"{self.path.name}: header of {n} bytes runs past the file")
        try:
            header = json.loads(bytes(self._mm[8:8 + n]))
        except (UnicodeDecodeError, json.JSONDecodeError) as e:
            raise Q4NXError(f"{self.path.name}: header is not JSON ({e})") from None
        self.data_base = 8 + n
        meta = header.pop("__metadata__", None) or {}
        self.metadata = {k: v for k, v in meta.items() if isinstance(v, str)}
        self.tensors = {}
        for name, t in header.items():
            try:
                o0, o1 = (int(v) for v in t["data_offsets"])
                shape = tuple(int(d) for d in t["shape"])
                dtype = str(t["dtype"])
            except (KeyError, TypeError, ValueError):
                raise Q4NXError(f"{self.path.name}: tensor {name!r} has a malformed entry") from None
            if not 0 <= o0 <= o1 or self.data_base + o1 > size:
                raise Q4NXError(f"{self.path.name}: tensor {name!r} data [{o0}, {o1}) runs past the file")
            self.tensors[name] = {"dtype": dtype, "shape": shape, "start": o0, "end": o1}

    # ---- tensors ------------------------------------------------------
    def _t(self, name: str) -> dict:
        try:
            return self.tensors[name]
        except KeyError:
            raise Q4NXError(f"{self.path.name}: no tensor {name!r}") from None

    def raw(self, name: str) -> np.ndarray:
        """The tensor's bytes as uint8, a view of the mapped file."""
        t = self._t(name)
        return np.frombuffer(self._mm, dtype=np.uint8, count=t["end"] - t["start"], offset=self.data_base + t["start"])

    def chunk_bytes_of(self, name: str) -> int:
        """The chunk size a quantised (I8) tensor is stored in, 0 for any other tensor
        (q4nx.py's chunk_bytes_of, q4nx_file.cpp's chunk_bytes)."""
        t = self._t(name)
        return t["shape"][-1] if t["dtype"] == "I8" and t["shape"] else 0

    def quant_format_of(self, name: str) -> str:
        """'q4_1', 'q4_0' (the signed quantiser), 'q8' or 'q4_k'; '' when not quantised."""
        cb = self.chunk_bytes_of(name)
        if cb == 0:
            return ""
        declared = self.metadata.get(f"quant_format.{name}")
        if declared:
            return declared
        if cb == CHUNK_Q4:
            first = self.raw(name)[:CHUNK_Q4]
            return "q4_0" if first.size == CHUNK_Q4 and not first[512:1024].any() else "q4_1"
        if cb in CHUNK_FORMATS:
            return CHUNK_FORMATS[cb]
        guess = (f"a smaller chunk geometry ({cb * 8192 // CHUNK_Q4} values per chunk)" if cb in (1280, 2560)
                 else "not a chunk format this reader knows")
        raise Q4NXError(f"{self.path.name}: {name} has {cb}-byte quant chunks; this reader takes {CHUNK_Q4} (q4_1), "
                        f"{CHUNK_Q8} (q8) and {CHUNK_Q4K} (Q4_K) -- {cb} is {guess}")

    def array(self, name: str) -> np.ndarray:
        """A BF16 / F32 / F16 tensor as float32 in its stored shape (a copy)."""
        t = self._t(name)
        raw = self.raw(name)
        if t["dtype"] == "BF16":
            a = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        elif t["dtype"] == "F32":
            a = raw.view(np.float32).copy()
        elif t["dtype"] == "F16":
            a = raw.view(np.float16).astype(np.float32)
        else:
            raise Q4NXError(f"{name!r} is {t['dtype']}; use packed() for quantised matrices")
        return a.reshape(t["shape"])

    def packed(self, name: str, out_dim: int, in_dim: int, device=None, q8: str = "requant", q4k: str = "mx"):
        """A quantised matrix [out_dim, in_dim] (out_dim % 64 == 0, in_dim % 256 == 0)
        transcoded into the mx layout on the GPU, from its chunks as they lie in the file.
        A q8 tensor is re-quantised to q4_1 (``q8="requant"``, the reference packer's
        default) or kept exact as the hi/lo pair (``q8="exact"``, a PackedQ8 for gemm_q8).
        A Q4_K tensor is collapsed to q4_1 (``q4k="mx"``, recipes/pack.py:266-310) or kept
        as Q4_K (``q4k="native"``, a PackedQ4K for gemm_q4k, the chunk's exact value)."""
        from . import q4                                 # needs the HIP library: imported on use
        fmt = self.quant_format_of(name)
        if not fmt:
            raise Q4NXError(f"{name!r} is {self._t(name)['dtype']}, not a quantised matrix")
        cb = self.chunk_bytes_of(name)
        if out_dim % 64 or in_dim % 256:
            raise Q4NXError(f"{name!r}: [{out_dim}, {in_dim}] is not whole 64-row groups of 256-K chunks")
        want = (out_dim // 32) * (in_dim // 256) * cb
        raw = self.raw(name)
        if raw.size != want:
            raise Q4NXError(f"{name!r} holds {raw.size} bytes; [{out_dim}, {in_dim}] in {cb}-byte chunks is {want}")
        if fmt == "q8" and q8 == "exact":
            return q4.pack_q8(raw, out_dim, in_dim, fmt="chunks", rs=1, device=device)
        if q8 not in ("requant", "exact"):
            raise ValueError(f"q8 must be 'requant' or 'exact', got {q8!r}")
        if q4k not in ("mx", "native"):
            raise ValueError(f"q4k must be 'mx' or 'native', got {q4k!r}")
        if fmt == "q4_k" and q4k == "native":
            return q4.pack_q4_k_chunks_native(raw, out_dim, in_dim, rs=1, device=device)
        return q4.pack_chunks(raw, fmt, out_dim, in_dim, rs=1, device=device)

    # ---- lifetime -----------------------------------------------------
    def close(self):
        mm, self._mm = getattr(self, "_mm", None), None
        if mm is not None:
            try:
                mm.close()
            except BufferError:                 # a returned view is still alive: let GC close it
                pass
        if getattr(self, "_fh", None) is not None:
            self._fh.close()
            self._fh = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
