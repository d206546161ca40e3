"""Python operator surface of the MI355X Q4_1 kernels (ctypes over libq4mi.so).

Same semantics as the reference's operators for this path -- packed Q4_1
weights in, bf16 or fp32 activations in, fp32 out:

* ``pack_q4_1`` / ``pack_q4_1_pool``   weight packing (open_kernels/q4_1_pack.py:124-142)
* ``dequant``                          dequant_pool / dq_chunks_q4_1 (q4_1_pack.py:173-180,
                                       model/q4nx.py:105-126), bit-exact
* ``gemv_q4``                          designs/gemv_q4 (gemv_q4.py:118-123): y[N] = W x
* ``gemm_q4``                          designs/gemm_q4 (gemm_q4.py:164-197): Y[M,N], M <= 24
* ``gemm_q4_prefill``                  designs/gemm_q4_prefill (gemm_q4_prefill.py:171-177)
* ``moe_batch``                        designs/moe_batch + Core::moe_block's gather/scatter
                                       (moe_batch.py:145-281, core.cpp:5150-5245)

Every call goes to a HIP kernel; nothing here computes on the CPU. Tensors
may be torch (on the GPU) or numpy (copied to the GPU). Work is enqueued on
torch's current stream of the tensors' device.
"""
from __future__ import annotations

import ctypes as C
import warnings
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from ._lib import Q4MI_BF16, Q4MI_F32, Q4GemvDesc, check

__all__ = [
    "PackedQ4", "PackedExperts", "packed_bytes", "pack_q4_1", "pack_q4_1_pool", "pack_q4_k", "pack_q4_k_chunks", "dequant",
    "gemv_q4", "gemm_q4", "gemm_q4_prefill", "moe_batch", "pack_moe_experts", "GemvGroup",
    "gemv_workspace_bytes", "prefill_workspace_bytes", "moe_workspace_bytes", "logits_topk", "lm_head_topk",
    "swiglu_q4", "rmsnorm_add", "pack_chunks", "PackedQ8", "pack_q8", "gemm_q8", "prefill_scales",
    "decode_segment", "decode_segment_splits", "decode_segment_workspace",
]

ROWS = 64          # rows per mx tile / row group
BLK = 32           # K per tile (one GGUF block)


def _lib_handle():
    return _lib.load()


def _device(dev=None) -> torch.device:
    if dev is None:
        return torch.device("cuda", torch.cuda.current_device())
    d = torch.device(dev)
    if d.type != "cuda":
        raise ValueError(f"device must be a GPU, got {d}")
    return d if d.index is not None else torch.device("cuda", torch.cuda.current_device())


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _to_dev(a, dev: torch.device, dtype=None) -> torch.Tensor:
    if isinstance(a, np.ndarray):
        a = np.ascontiguousarray(a)
        with warnings.catch_warnings():
            # a read-only view (a memory-mapped file's tensor) is only read, to copy it over
            warnings.filterwarnings("ignore", message="The given NumPy array is not writable")
            t = torch.from_numpy(a)
    elif isinstance(a, torch.Tensor):
        t = a
    else:
        raise TypeError(f"expected a numpy array or torch tensor, got {type(a)}")
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.to(dev, non_blocking=False).contiguous()


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def _buf(t, name: str, dtype, shape, dev: torch.device) -> torch.Tensor:
    """A caller's output / in-place buffer, or a new one of ``shape``. The kernels write
    through raw device pointers with no byte count, so a buffer of the wrong dtype, element
    count, layout or device would be written (or read) out of bounds: refuse it here."""
    numel = 1
    for v in shape:
        numel *= int(v)
    if t is None:
        return torch.empty(shape, dtype=dtype, device=dev)
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch tensor, got {type(t)}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.numel() != numel:
        raise ValueError(f"{name} must hold {numel} elements {tuple(shape)}, got {t.numel()} {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.device != dev:
        raise ValueError(f"{name} must be on {dev}, got {t.device}")
    return t


def packed_bytes(n: int, k: int) -> int:
    """Bytes of the mx layout for an [n, k] matrix (n % 64 == 0, k % 32 == 0)."""
    b = _lib_handle().q4_packed_bytes(n, k)
    if b < 0:
        raise ValueError(f"[{n}, {k}] does not fit the mx layout (n % 64 == 0, k % 32 == 0)")
    return int(b)


@dataclass
class PackedQ4:
    """One [n, k] Q4_1 weight matrix in the mx layout, resident on a GPU. ``prefill_scales``
    caches the matrix's fp16 prefill scales (q4_prefill_scales) once a prefill GEMM has
    needed them; the weights are static, so they are computed once."""
    data: torch.Tensor        # uint8, packed_bytes(n, k)
    n: int
    k: int
    prefill_scales: torch.Tensor | None = field(default=None, repr=False, compare=False)
    # "bf16": d and m narrowed to bf16 (the reference pool's scales); "fp16": GGUF's fp16 d
    # and m kept exactly (pack_q4_1(..., scales="fp16")), read by dequant, gemm_q4 (M <= 16),
    # gemv_q4 and GemvGroup only
    scales: str = "bf16"

    @property
    def shape(self):
        return (self.n, self.k)

    @property
    def device(self):
        return self.data.device

    @property
    def nbytes(self) -> int:
        return self.data.numel()


@dataclass
class PackedExperts:
    """E experts' matrices of one shape [n, k], back to back in the mx layout (one [E n, k]
    mx matrix). ``prefill_scales`` caches that matrix's fp16 prefill scales once the
    prefill-scale MoE path has needed them."""
    data: torch.Tensor
    experts: int
    n: int
    k: int
    prefill_scales: torch.Tensor | None = field(default=None, repr=False, compare=False)

    @property
    def expert_bytes(self) -> int:
        return packed_bytes(self.n, self.k)


# --------------------------------------------------------------------------
# packing and dequant
# --------------------------------------------------------------------------

def pack_q4_1(blocks, device=None, out: torch.Tensor | None = None, scales: str = "bf16") -> PackedQ4:
    """GGUF Q4_1 (20 B) or Q4_0 (18 B) blocks uint8[N, K/32, w] -> mx layout on the GPU.

    ``scales="bf16"``: d and m are narrowed fp16 -> bf16 (RNE), exactly the reference
    pool's semantics (q4_1_pack.py:104-109, :129-130); the block width says which format
    it is, as in q4_1_pack.py:8-9. ``scales="fp16"`` (Q4_1 only): GGUF's fp16 d and m kept
    exactly, as the reference's GGUF-direct pool keeps them (gguf_pool.py:1-17); such a
    matrix goes to dequant, gemm_q4 / gemv_q4 (M <= 16) and GemvGroup."""
    if scales not in ("bf16", "fp16"):
        raise ValueError(f"scales must be 'bf16' or 'fp16', got {scales!r}")
    dev = _device(device if device is not None else (blocks.device if isinstance(blocks, torch.Tensor)
                                                     and blocks.is_cuda else None))
    src = _to_dev(blocks, dev, torch.uint8)
    if src.dim() != 3 or src.shape[2] not in (18, 20):
        raise ValueError(f"blocks must be uint8[N, K/32, 20|18], got {tuple(src.shape)}")
    n, nb, w = src.shape
    k = nb * BLK
    nbytes = packed_bytes(n, k)
    out = _buf(out, "out", torch.uint8, (nbytes,), dev)
    if scales == "fp16" and w != 20:
        raise ValueError("fp16 scales are a Q4_1 mode (Q4_0 has the exact mx0 layout: pack_q4_0_native)")
    with torch.cuda.device(dev):
        check("q4_repack", _lib_handle().q4_repack(_ptr(src), w, _ptr(out), n, k, int(scales == "fp16"),
                                                   _stream(dev)))
    return PackedQ4(out[:nbytes], n, k, scales=scales)


def pack_q4_1_pool(pool, n: int, k: int, rs: int, device=None) -> PackedQ4:
    """The reference's pool chunk bytes (5120 B chunks, band row split rs;
    q4_1_pack.py:16-34) -> mx layout on the GPU. Bytes carry over exactly."""
    dev = _device(device)
    src = _to_dev(pool, dev, torch.uint8).reshape(-1)
    if src.numel() != n * k * 5 // 8:
        raise ValueError(f"pool holds {src.numel()} bytes, [{n}, {k}] needs {n * k * 5 // 8}")
    nbytes = packed_bytes(n, k)
    out = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        check("q4_repack_pool", _lib_handle().q4_repack_pool(_ptr(src), rs, _ptr(out), n, k, _stream(dev)))
    return PackedQ4(out, n, k)


def pack_q4_k(blocks, device=None) -> PackedQ4:
    """GGUF Q4_K super-blocks uint8[N, K/256, 144] -> mx layout on the GPU.

    Every 32-value sub-block becomes a Q4_1 block with d = bf16(d*sc) and
    m = bf16(-dmin*min): the products are exact, the bf16 rounding is the
    reference's own Q4_K transcode (recipes/pack.py:266-310)."""
    dev = _device(device if device is not None else (blocks.device if isinstance(blocks, torch.Tensor)
                                                     and blocks.is_cuda else None))
    src = _to_dev(blocks, dev, torch.uint8)
    if src.dim() != 3 or src.shape[2] != 144:
        raise ValueError(f"blocks must be uint8[N, K/256, 144], got {tuple(src.shape)}")
    n, nsb, _ = src.shape
    k = nsb * 256
    out = torch.empty(packed_bytes(n, k), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        check("q4_repack_q4k", _lib_handle().q4_repack_q4k(_ptr(src), _ptr(out), n, k, _stream(dev)))
    return PackedQ4(out, n, k)


def pack_q4_k_chunks(chunks, n: int, k: int, rs: int = 1, device=None) -> PackedQ4:
    """The reference container's Q4_K chunks (4736 B per 32 rows x 256 K, band order
    with row split rs; rs = 1 is the file raster) -> mx layout on the GPU, with
    d = bf16(S*scale) and m = bf16(M*min) (recipes/pack.py:266-310)."""
    dev = _device(device)
    src = _to_dev(chunks, dev, torch.uint8).reshape(-1)
    want = (n // 32) * (k // 256) * 4736 if n % 32 == 0 and k % 256 == 0 else -1
    if src.numel() != want:
        raise ValueError(f"Q4_K chunks hold {src.numel()} bytes, [{n}, {k}] needs {want} (4736 B per 32 x 256)")
    out = torch.empty(packed_bytes(n, k), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        check("q4_repack_q4k_chunks",
              _lib_handle().q4_repack_q4k_chunks(_ptr(src), rs, _ptr(out), n, k, _stream(dev)))
    return PackedQ4(out, n, k)


# --------------------------------------------------------------------------
# native Q4_K (the "mxk" layout: the super-block's own integers, no bf16 collapse)
# --------------------------------------------------------------------------

def q4k_packed_bytes(n: int, k: int) -> int:
    """Bytes of the native Q4_K layout for an [n, k] matrix (n % 64 == 0, k % 256 == 0)."""
    b = _lib_handle().q4_q4k_packed_bytes(n, k)
    if b < 0:
        raise ValueError(f"[{n}, {k}] does not fit the Q4_K layout (n % 64 == 0, k % 256 == 0)")
    return int(b)


@dataclass
class PackedQ4K:
    """One [n, k] Q4_K matrix in the native layout: weight fl32(d sc q + m mn) with d sc
    and m mn exact, as the reference's Q4_K GEMM reads it (gemm_q4.h:456-507); 0.594 B
    per weight."""
    data: torch.Tensor
    n: int
    k: int

    @property
    def shape(self):
        return (self.n, self.k)

    @property
    def device(self):
        return self.data.device

    @property
    def nbytes(self) -> int:
        return self.data.numel()


def pack_q4_k_native(blocks, device=None) -> PackedQ4K:
    """GGUF Q4_K super-blocks uint8[N, K/256, 144] -> the native Q4_K layout on the GPU:
    weight d sc q - dmin min, exactly the GGUF reader's value (gguf_file.cpp:611-635)."""
    dev = _device(device if device is not None else (blocks.device if isinstance(blocks, torch.Tensor)
                                                     and blocks.is_cuda else None))
    src = _to_dev(blocks, dev, torch.uint8)
    if src.dim() != 3 or src.shape[2] != 144:
        raise ValueError(f"blocks must be uint8[N, K/256, 144], got {tuple(src.shape)}")
    n, nsb, _ = src.shape
    k = nsb * 256
    out = torch.empty(q4k_packed_bytes(n, k), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        check("q4_repack_q4k_native", _lib_handle().q4_repack_q4k_native(_ptr(src), _ptr(out), n, k, _stream(dev)))
    return PackedQ4K(out, n, k)


def pack_q4_k_chunks_native(chunks, n: int, k: int, rs: int = 1, device=None) -> PackedQ4K:
    """The reference container's Q4_K chunks (4736 B per 32 rows x 256 K, band order with
    row split rs) -> the native Q4_K layout: weight S sc nib + M mn, the chunk's own value
    (gemm_q4.h:456-507), with no bf16 collapse."""
    dev = _device(device)
    src = _to_dev(chunks, dev, torch.uint8).reshape(-1)
    want = (n // 32) * (k // 256) * 4736 if n % 32 == 0 and k % 256 == 0 else -1
    if src.numel() != want:
        raise ValueError(f"Q4_K chunks hold {src.numel()} bytes, [{n}, {k}] needs {want} (4736 B per 32 x 256)")
    out = torch.empty(q4k_packed_bytes(n, k), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        check("q4_repack_q4k_chunks_native",
              _lib_handle().q4_repack_q4k_chunks_native(_ptr(src), rs, _ptr(out), n, k, _stream(dev)))
    return PackedQ4K(out, n, k)


def dequant_q4k(w: PackedQ4K, out: torch.Tensor | None = None) -> torch.Tensor:
    """Native Q4_K layout -> f32[n, k], w = fl32(q (d sc) + m mn), bit-exact."""
    dev = w.device
    out = _buf(out, "out", torch.float32, (w.n, w.k), dev)
    with torch.cuda.device(dev):
        check("q4_dequant_q4k", _lib_handle().q4_dequant_q4k(_ptr(w.data), _ptr(out), w.n, w.k, _stream(dev)))
    return out


def gemm_q4k(w: PackedQ4K, x, y: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
             residual: torch.Tensor | None = None) -> torch.Tensor:
    """Y[M, N] = X[M, K] @ W^T over a native Q4_K matrix, 1 <= M <= 16, fp32 out (the
    reference's gemm_q4k_tile4 operator, gemm_q4.h:555); ``residual`` as in gemm_q4."""
    dev = w.device
    xt = _acts(x, dev)
    if xt.dim() == 1:
        xt = xt.unsqueeze(0)
    M, K = xt.shape
    if K != w.k:
        raise ValueError(f"x has K={K}, W is [{w.n}, {w.k}]")
    if not 1 <= M <= 16:
        raise ValueError(f"gemm_q4k takes 1..16 tokens, got {M}")
    y = _buf(y, "y", torch.float32, (M, w.n), dev)
    if residual is not None and (residual.dtype != torch.float32 or not residual.is_contiguous()
                                 or residual.numel() != M * w.n or residual.device != dev):
        raise ValueError(f"residual must be a contiguous float32 [{M}, {w.n}] tensor on {dev}")
    lib = _lib_handle()
    with torch.cuda.device(dev):
        wp, wn = _ws_arg(dev, lib.q4_gemv_q4k_workspace_bytes(M, w.n, w.k), "gemv", workspace)
        check("q4_gemv_q4k", lib.q4_gemv_q4k(_ptr(w.data), _ptr(xt), _x_dtype(xt),
                                             None if residual is None else _ptr(residual), _ptr(y), M, w.n, w.k,
                                             wp, wn, _stream(dev)))
    return y


@dataclass
class PackedQ8:
    """A q8 matrix [n, k] held exactly as two mx q4_1 planes, hi + lo = s q
    (split_q8_q4_1, recipes/pack.py:94-117); 1.25 B per weight."""
    hi: PackedQ4
    lo: PackedQ4

    @property
    def n(self) -> int:
        return self.hi.n

    @property
    def k(self) -> int:
        return self.hi.k

    @property
    def shape(self):
        return (self.n, self.k)

    @property
    def device(self):
        return self.hi.device

    @property
    def nbytes(self) -> int:
        return self.hi.nbytes + self.lo.nbytes


def pack_q8(src, n: int, k: int, fmt: str = "chunks", rs: int = 1, device=None) -> PackedQ8:
    """q8 weights -> the exact hi/lo mx pair on the GPU. ``fmt`` "chunks": 8704 B q8
    chunks in band order with row split rs (rs = 1: a .q4nx raster); "q8_0": GGUF Q8_0
    blocks uint8[n, k/32, 34] (fp16 d narrowed to bf16 by RNE); "chunks_f32": the
    GGUF-direct pool's 9216 B q8 chunks (f32 scales narrowed to bf16 by RNE)."""
    if fmt not in ("chunks", "q8_0", "chunks_f32"):
        raise ValueError(f"fmt must be 'chunks', 'q8_0' or 'chunks_f32', got {fmt!r}")
    dev = _device(device if device is not None else (src.device if isinstance(src, torch.Tensor)
                                                     and src.is_cuda else None))
    t = _to_dev(src, dev, torch.uint8).reshape(-1)
    cb = {"chunks": 8704, "chunks_f32": 9216}.get(fmt)
    want = ((n // 32) * (k // 256) * cb if n % 32 == 0 and k % 256 == 0 else -1) if cb \
        else (n * (k // 32) * 34 if k % 32 == 0 else -1)
    if t.numel() != want:
        raise ValueError(f"{fmt} source holds {t.numel()} bytes, [{n}, {k}] needs {want}")
    planes = []
    with torch.cuda.device(dev):
        for part in (0, 1):
            out = torch.empty(packed_bytes(n, k), dtype=torch.uint8, device=dev)
            check("q4_repack_q8_split", _lib_handle().q4_repack_q8_split(_ptr(t), {"chunks": 0, "q8_0": 1,
                                                                                   "chunks_f32": 2}[fmt], rs,
                                                                         part, _ptr(out), n, k, _stream(dev)))
            planes.append(PackedQ4(out, n, k))
    return PackedQ8(*planes)


@dataclass
class PackedQ8N:
    """A q8 matrix [n, k] in the native mx8 layout: 8-bit codes + a bf16 scale per row
    and 32-K block, weight s * q exactly (1.0625 B per weight)."""
    data: torch.Tensor
    n: int
    k: int

    @property
    def shape(self):
        return (self.n, self.k)

    @property
    def device(self):
        return self.data.device

    @property
    def nbytes(self) -> int:
        return self.data.numel()


def pack_q8_native(src, n: int, k: int, fmt: str = "chunks", rs: int = 1, device=None) -> PackedQ8N:
    """q8 weights (``fmt`` and ``rs`` as pack_q8) -> the native mx8 layout on the GPU: the
    same values s * q as the exact hi/lo pair, at 1.0625 B per weight instead of 1.25."""
    if fmt not in ("chunks", "q8_0", "chunks_f32"):
        raise ValueError(f"fmt must be 'chunks', 'q8_0' or 'chunks_f32', got {fmt!r}")
    dev = _device(device if device is not None else (src.device if isinstance(src, torch.Tensor)
                                                     and src.is_cuda else None))
    t = _to_dev(src, dev, torch.uint8).reshape(-1)
    cb = {"chunks": 8704, "chunks_f32": 9216}.get(fmt)
    want = ((n // 32) * (k // 256) * cb if n % 32 == 0 and k % 256 == 0 else -1) if cb \
        else (n * (k // 32) * 34 if k % 32 == 0 else -1)
    if t.numel() != want:
        raise ValueError(f"{fmt} source holds {t.numel()} bytes, [{n}, {k}] needs {want}")
    lib = _lib_handle()
    nbytes = lib.q4_q8_native_packed_bytes(n, k)
    if nbytes < 0:
        raise ValueError(f"[{n}, {k}] does not fit the mx8 layout (n % 64 == 0, k % 32 == 0)")
    out = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        check("q4_repack_q8_native", lib.q4_repack_q8_native(_ptr(t), {"chunks": 0, "q8_0": 1, "chunks_f32": 2}[fmt],
                                                             rs, _ptr(out), n, k, _stream(dev)))
    return PackedQ8N(out, n, k)


def dequant_q8_native(w: PackedQ8N, out: torch.Tensor | None = None) -> torch.Tensor:
    """mx8 -> f32[n, k], w = s * q (exact)."""
    dev = w.device
    out = _buf(out, "out", torch.float32, (w.n, w.k), dev)
    with torch.cuda.device(dev):
        check("q4_dequant_q8_native", _lib_handle().q4_dequant_q8_native(_ptr(w.data), _ptr(out), w.n, w.k,
                                                                         _stream(dev)))
    return out


def gemm_q8_native(w: PackedQ8N, x, y: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                   residual: torch.Tensor | None = None) -> torch.Tensor:
    """Y[M, N] = X[M, K] @ W^T over a native q8 matrix, 1 <= M <= 16 (the gemv_q8 sibling of
    gemm_q4 on the mx8 layout); ``residual`` as in gemm_q4."""
    dev = w.device
    xt = _acts(x, dev)
    if xt.dim() == 1:
        xt = xt.unsqueeze(0)
    M, K = xt.shape
    if K != w.k:
        raise ValueError(f"x has K={K}, W is [{w.n}, {w.k}]")
    if not 1 <= M <= 16:
        raise ValueError(f"gemm_q8_native takes 1..16 tokens, got {M}")
    y = _buf(y, "y", torch.float32, (M, w.n), dev)
    if residual is not None and (residual.dtype != torch.float32 or not residual.is_contiguous()
                                 or residual.numel() != M * w.n or residual.device != dev):
        raise ValueError(f"residual must be a contiguous float32 [{M}, {w.n}] tensor on {dev}")
    lib = _lib_handle()
    with torch.cuda.device(dev):
        wp, wn = _ws_arg(dev, lib.q4_gemv_q8_native_workspace_bytes(M, w.n, w.k), "gemv", workspace)
        check("q4_gemv_q8_native", lib.q4_gemv_q8_native(_ptr(w.data), _ptr(xt), _x_dtype(xt),
                                                         None if residual is None else _ptr(residual), _ptr(y),
                                                         M, w.n, w.k, wp, wn, _stream(dev)))
    return y


@dataclass
class PackedQ40:
    """A Q4_0 matrix [n, k] in the Q4_0-native mx0 layout: the mx codes plus one bf16 d per
    row and 32-K block, weight q d - 8 d (0.5625 B per weight; the reference's 4608 B
    Q4_0-native chunk, q4_1_pack.py:145-152)."""
    data: torch.Tensor
    n: int
    k: int

    @property
    def shape(self):
        return (self.n, self.k)

    @property
    def device(self):
        return self.data.device

    @property
    def nbytes(self) -> int:
        return self.data.numel()


def pack_q4_0_native(src, n: int, k: int, fmt: str = "q4_0", rs: int = 1, device=None) -> PackedQ40:
    """Q4_0 weights -> the mx0 layout on the GPU. ``fmt`` "q4_0": GGUF Q4_0 blocks (18 B,
    [n, k/32, 18] or flat); "chunks": the reference's 4608 B Q4_0-native chunks in pool
    order with row split ``rs`` (pack_q4_0_native_pool, q4_1_pack.py:148-152)."""
    if fmt not in ("q4_0", "chunks"):
        raise ValueError(f"fmt must be 'q4_0' or 'chunks', got {fmt!r}")
    dev = _device(device if device is not None else (src.device if isinstance(src, torch.Tensor)
                                                     and src.is_cuda else None))
    t = _to_dev(src, dev, torch.uint8).reshape(-1)
    if fmt == "chunks":
        want = (n // 32) * (k // 256) * 4608 if n % 32 == 0 and k % 256 == 0 else -1
    else:
        want = n * (k // 32) * 18 if k % 32 == 0 else -1
    if t.numel() != want:
        raise ValueError(f"{fmt} source holds {t.numel()} bytes, [{n}, {k}] needs {want}")
    lib = _lib_handle()
    nbytes = lib.q4_q40_packed_bytes(n, k)
    if nbytes < 0:
        raise ValueError(f"[{n}, {k}] does not fit the mx0 layout (n % 64 == 0, k % 32 == 0)")
    out = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        check("q4_repack_q40", lib.q4_repack_q40(_ptr(t), 0 if fmt == "q4_0" else 1, rs, _ptr(out), n, k,
                                                 _stream(dev)))
    return PackedQ40(out, n, k)


def dequant_q4_0_native(w: PackedQ40, out: torch.Tensor | None = None) -> torch.Tensor:
    """mx0 -> f32[n, k], w = fl32(q d - 8 d), bit-exact."""
    dev = w.device
    out = _buf(out, "out", torch.float32, (w.n, w.k), dev)
    with torch.cuda.device(dev):
        check("q4_dequant_q40", _lib_handle().q4_dequant_q40(_ptr(w.data), _ptr(out), w.n, w.k, _stream(dev)))
    return out


def gemm_q4_0_native(w: PackedQ40, x, y: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                     residual: torch.Tensor | None = None) -> torch.Tensor:
    """Y[M, N] = X[M, K] @ W^T over a Q4_0-native matrix, 1 <= M <= 16: gemm_q4 on the mx0
    layout (gemv_q4.h:66-82's GEMV_Q4_0_NATIVE build), bit-identical to gemm_q4 over
    pack_q4_1 of the same Q4_0 blocks; ``residual`` as in gemm_q4."""
    dev = w.device
    xt = _acts(x, dev)
    if xt.dim() == 1:
        xt = xt.unsqueeze(0)
    M, K = xt.shape
    if K != w.k:
        raise ValueError(f"x has K={K}, W is [{w.n}, {w.k}]")
    if not 1 <= M <= 16:
        raise ValueError(f"gemm_q4_0_native takes 1..16 tokens, got {M}")
    y = _buf(y, "y", torch.float32, (M, w.n), dev)
    if residual is not None and (residual.dtype != torch.float32 or not residual.is_contiguous()
                                 or residual.numel() != M * w.n or residual.device != dev):
        raise ValueError(f"residual must be a contiguous float32 [{M}, {w.n}] tensor on {dev}")
    lib = _lib_handle()
    with torch.cuda.device(dev):
        wp, wn = _ws_arg(dev, lib.q4_gemv_workspace_bytes(M, w.n, w.k), "gemv", workspace)
        check("q4_gemv_q40", lib.q4_gemv_q40(_ptr(w.data), _ptr(xt), _x_dtype(xt),
                                             None if residual is None else _ptr(residual), _ptr(y),
                                             M, w.n, w.k, wp, wn, _stream(dev)))
    return y


_CHUNK_ENTRY = {   # chunk format -> (chunk bytes, C entry point)
    "q4_1": (5120, "q4_repack_pool"),
    "q4_f32": (6144, "q4_repack_pool_f32"),
    "q4_0": (5120, "q4_repack_pool_signed"),
    "q8": (8704, "q4_repack_q8_chunks"),
    "q4_k": (4736, "q4_repack_q4k_chunks"),
}


def pack_chunks(chunks, fmt: str, n: int, k: int, rs: int = 1, device=None) -> PackedQ4:
    """32-row x 256-K chunks of one matrix [n, k] (band order with row split rs; rs = 1
    is a .q4nx file's raster) -> mx layout on the GPU. ``fmt``: "q4_1" (bytes carry over),
    "q4_f32" (the GGUF-direct pool's 6144 B chunks, f32 scales narrowed to bf16),
    "q4_0" (the signed quantiser, read exactly as q4_1), "q8" (re-quantised to q4_1 as
    recipes/pack.py:224-263 does) or "q4_k" (recipes/pack.py:266-310)."""
    if fmt not in _CHUNK_ENTRY:
        raise ValueError(f"chunk format must be one of {sorted(_CHUNK_ENTRY)}, got {fmt!r}")
    cb, entry = _CHUNK_ENTRY[fmt]
    dev = _device(device)
    src = _to_dev(chunks, dev, torch.uint8).reshape(-1)
    want = (n // 32) * (k // 256) * cb if n % 32 == 0 and k % 256 == 0 else -1
    if src.numel() != want:
        raise ValueError(f"{fmt} chunks hold {src.numel()} bytes, [{n}, {k}] needs {want} ({cb} B per 32 x 256)")
    out = torch.empty(packed_bytes(n, k), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        check(entry, getattr(_lib_handle(), entry)(_ptr(src), rs, _ptr(out), n, k, _stream(dev)))
    return PackedQ4(out, n, k)


def dequant(w: PackedQ4, out: torch.Tensor | None = None) -> torch.Tensor:
    """mx layout -> f32[n, k], w = fl32(q*d + m), bit-exact with dequant_pool."""
    dev = w.device
    out = _buf(out, "out", torch.float32, (w.n, w.k), dev)
    fn = "q4_dequant_fp16s" if w.scales == "fp16" else "q4_dequant"
    with torch.cuda.device(dev):
        check(fn, getattr(_lib_handle(), fn)(_ptr(w.data), _ptr(out), w.n, w.k, _stream(dev)))
    return out


def _bf16_scales(op: str, *ws) -> None:
    """Refuse matrices packed with fp16 scale words where only the bf16 form is built."""
    for w in ws:
        if getattr(w, "scales", "bf16") != "bf16":
            raise ValueError(f"{op} takes matrices with bf16 scales (pack_q4_1(..., scales='bf16'))")


# --------------------------------------------------------------------------
# workspaces (zero-filled once; the kernels leave their counters at zero)
# --------------------------------------------------------------------------

_WS: dict = {}


def _workspace(dev: torch.device, nbytes: int, op: str) -> torch.Tensor | None:
    """A cached scratch buffer per (operator, device, stream), grown on demand
    (never allocated by the C library itself)."""
    if nbytes == 0:
        return None
    key = (op, dev.index, torch.cuda.current_stream(dev).cuda_stream)
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        _WS[key] = ws
    return ws


def _ws_arg(dev, nbytes: int, op: str, workspace):
    """(pointer, size) of the caller's workspace, else of the cached one."""
    if workspace is None:
        ws = _workspace(dev, nbytes, op)
        return (_ptr(ws), ws.numel()) if ws is not None else (None, 0)
    if not isinstance(workspace, torch.Tensor):
        raise TypeError(f"workspace must be a torch tensor, got {type(workspace)}")
    if workspace.device != dev or not workspace.is_contiguous():
        raise ValueError(f"workspace must be a contiguous tensor on {dev}, got {workspace.device}")
    if workspace.numel() * workspace.element_size() < nbytes:
        raise ValueError(f"workspace holds {workspace.numel() * workspace.element_size()} bytes, {nbytes} needed")
    return _ptr(workspace), workspace.numel() * workspace.element_size()


def gemv_workspace_bytes(m: int, n: int, k: int) -> int:
    """Bytes of workspace gemm_q4 / gemv_q4 needs for this shape (0: none)."""
    return int(_lib_handle().q4_gemv_workspace_bytes(m, n, k))


def prefill_workspace_bytes(t: int, n: int, k: int) -> int:
    return int(_lib_handle().q4_gemm_prefill_workspace_bytes(t, n, k))


def moe_prefill_workspace_bytes(t: int, e: int, topk: int, h: int, f: int) -> int:
    return int(_lib_handle().q4_moe_prefill_workspace_bytes(t, e, topk, h, f))


def moe_shared_workspace_bytes(t: int, e: int, topk: int, h: int, f: int, fs: int) -> int:
    """Bytes q4_moe_gemv_shared needs: q4_moe_gemv's, then the shared expert's h and y."""
    return int(_lib_handle().q4_moe_shared_workspace_bytes(t, e, topk, h, f, fs))


def moe_workspace_bytes(t: int, e: int, topk: int, h: int, f: int) -> int:
    return int(_lib_handle().q4_moe_workspace_bytes(t, e, topk, h, f))


def _x_dtype(x: torch.Tensor) -> int:
    if x.dtype == torch.bfloat16:
        return Q4MI_BF16
    if x.dtype == torch.float32:
        return Q4MI_F32
    raise TypeError(f"activations must be bf16 or fp32, got {x.dtype}")


def _acts(x, dev: torch.device) -> torch.Tensor:
    if isinstance(x, np.ndarray):
        x = torch.from_numpy(np.ascontiguousarray(x))
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.to(torch.float32)
    return x.to(dev).contiguous()


# --------------------------------------------------------------------------
# decode GEMV / skinny GEMM
# --------------------------------------------------------------------------

def gemm_q4(w: PackedQ4, x, y: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
            residual: torch.Tensor | None = None) -> torch.Tensor:
    """Y[M, N] = X[M, K] @ W^T for 1 <= M <= 24 decode tokens, fp32 out
    (gemm_q4.py:164-197's operator, logical [M, N] order; the reference's blocked dataflow
    covers M = 1..24, gemm_q4.py:9-13). ``workspace``
    (>= gemv_workspace_bytes) avoids the cached one, e.g. under graph capture.
    ``residual`` (f32 [M, N]) is added in the epilogue -- the x_res + W h of
    model/replica.py:81 -- and may be ``y`` itself to accumulate in place."""
    dev = w.device
    xt = _acts(x, dev)
    if xt.dim() == 1:
        xt = xt.unsqueeze(0)
    M, K = xt.shape
    if K != w.k:
        raise ValueError(f"x has K={K}, W is [{w.n}, {w.k}]")
    if not 1 <= M <= 24:
        raise ValueError(f"gemm_q4 takes 1..24 tokens, got {M} (use gemm_q4_prefill)")
    y = _buf(y, "y", torch.float32, (M, w.n), dev)
    lib = _lib_handle()
    if w.scales == "fp16":
        if M > 16:
            raise ValueError(f"a matrix with fp16 scales takes 1..16 tokens, got {M}")
        if residual is not None and (residual.dtype != torch.float32 or not residual.is_contiguous()
                                     or residual.numel() != M * w.n or residual.device != dev):
            raise ValueError(f"residual must be a contiguous float32 [{M}, {w.n}] tensor on {dev}")
        with torch.cuda.device(dev):
            wp, wn = _ws_arg(dev, lib.q4_gemv_workspace_bytes(M, w.n, w.k), "gemv", workspace)
            check("q4_gemv_fp16s", lib.q4_gemv_fp16s(_ptr(w.data), _ptr(xt), _x_dtype(xt),
                                                     None if residual is None else _ptr(residual), _ptr(y), M, w.n,
                                                     w.k, wp, wn, _stream(dev)))
        return y
    with torch.cuda.device(dev):
        wp, wn = _ws_arg(dev, lib.q4_gemv_workspace_bytes(M, w.n, w.k), "gemv", workspace)
        if residual is None:
            check("q4_gemv", lib.q4_gemv(_ptr(w.data), _ptr(xt), _x_dtype(xt), _ptr(y), M, w.n, w.k, wp, wn,
                                         _stream(dev)))
        else:
            if residual.dtype != torch.float32 or not residual.is_contiguous() or residual.numel() != M * w.n \
                    or residual.device != dev:
                raise ValueError(f"residual must be a contiguous float32 [{M}, {w.n}] tensor on {dev}")
            check("q4_gemv_residual", lib.q4_gemv_residual(_ptr(w.data), _ptr(xt), _x_dtype(xt), _ptr(residual),
                                                           _ptr(y), M, w.n, w.k, wp, wn, _stream(dev)))
    return y


def gemm_q8(w: PackedQ8, x, y: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
            residual: torch.Tensor | None = None) -> torch.Tensor:
    """Y[M, N] = X[M, K] @ W^T for a q8 matrix (the exact hi/lo pair), 1 <= M <= 16, in
    one launch (the gemv_q8 sibling of gemm_q4); ``residual`` as in gemm_q4."""
    dev = w.device
    xt = _acts(x, dev)
    if xt.dim() == 1:
        xt = xt.unsqueeze(0)
    M, K = xt.shape
    if K != w.k:
        raise ValueError(f"x has K={K}, W is [{w.n}, {w.k}]")
    if not 1 <= M <= 16:
        raise ValueError(f"gemm_q8 takes 1..16 tokens, got {M}")
    y = _buf(y, "y", torch.float32, (M, w.n), dev)
    if residual is not None and (residual.dtype != torch.float32 or not residual.is_contiguous()
                                 or residual.numel() != M * w.n or residual.device != dev):
        raise ValueError(f"residual must be a contiguous float32 [{M}, {w.n}] tensor on {dev}")
    lib = _lib_handle()
    with torch.cuda.device(dev):
        wp, wn = _ws_arg(dev, lib.q4_gemv_workspace_bytes(M, w.n, w.k), "gemv", workspace)
        check("q4_gemv_q8", lib.q4_gemv_q8(_ptr(w.hi.data), _ptr(w.lo.data), _ptr(xt), _x_dtype(xt),
                                           None if residual is None else _ptr(residual), _ptr(y), M, w.n, w.k,
                                           wp, wn, _stream(dev)))
    return y


def _norm_w(norm_w, K: int, dev) -> tuple[torch.Tensor, int]:
    if not isinstance(norm_w, torch.Tensor) or norm_w.numel() != K or norm_w.dtype not in (torch.float32,
                                                                                            torch.bfloat16):
        raise ValueError(f"norm_w must be a float32 or bfloat16 tensor of {K} values")
    wt = norm_w.to(dev).contiguous()
    return wt, Q4MI_BF16 if wt.dtype == torch.bfloat16 else Q4MI_F32


def _norm_x(x, K: int, dev) -> torch.Tensor:
    if not isinstance(x, torch.Tensor) or x.dtype != torch.float32 or x.device != dev or not x.is_contiguous():
        raise TypeError(f"x must be the contiguous float32 residual stream on {dev}")
    xt = x.view(-1, x.shape[-1])
    if xt.shape[1] != K:
        raise ValueError(f"x has K={xt.shape[1]}, W has K={K}")
    return xt


def _norm_ws_bytes(lib, M: int, w: PackedQ4, workspace) -> int:
    """A norm GEMV's workspace: the cached one is sized for the normalise-once form of
    vocabulary-sized matrices; a caller's needs only what gemm_q4 needs (the library picks
    the form its size allows)."""
    if workspace is None:
        return int(lib.q4_gemv_rmsnorm_workspace_bytes(M, w.n, w.k))
    return int(lib.q4_gemv_workspace_bytes(M, w.n, w.k))


def gemm_q4_rmsnorm(w: PackedQ4, x: torch.Tensor, norm_w: torch.Tensor, eps: float = 1e-6,
                    y: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Y = bf16(RMSNorm(x) * norm_w) @ W^T with the norm formed inside the GEMV from the f32
    residual stream x [M, K] (1 <= M <= 16, K <= 16384): the bits of rmsnorm_add (bf16 out)
    followed by gemm_q4, with no launch and no copy for the norm. Vocabulary-sized matrices
    (an lm_head: >= 1024 row groups) normalise the rows once into the workspace first (one
    more launch, the same bits); a caller's ``workspace`` needs gemv_workspace_bytes, and
    takes that form from q4_gemv_rmsnorm_workspace_bytes on."""
    _bf16_scales("gemm_q4_rmsnorm", w)
    dev = w.device
    xt = _norm_x(x, w.k, dev)
    M = xt.shape[0]
    if not 1 <= M <= 16:
        raise ValueError(f"gemm_q4_rmsnorm takes 1..16 tokens, got {M}")
    wt, wd = _norm_w(norm_w, w.k, dev)
    y = _buf(y, "y", torch.float32, (M, w.n), dev)
    lib = _lib_handle()
    with torch.cuda.device(dev):
        wp, wn = _ws_arg(dev, _norm_ws_bytes(lib, M, w, workspace), "gemv", workspace)
        check("q4_gemv_rmsnorm", lib.q4_gemv_rmsnorm(_ptr(w.data), _ptr(xt), _ptr(wt), wd, float(eps), _ptr(y),
                                                     M, w.n, w.k, wp, wn, _stream(dev)))
    return y


def gemv_split_count(w: PackedQ4) -> int:
    """The K-split count gemm_q4 plans for ``w`` at decode sizes (1: unsplit)."""
    _bf16_scales("gemv_split_count", w)
    return int(_lib_handle().q4_gemv_split_count(w.n, w.k))


def gemm_q4_partials(w: PackedQ4, x, splits: int | None = None, part: torch.Tensor | None = None) -> torch.Tensor:
    """The partial sums of a K-split gemm_q4, unreduced: part[s] = X @ W[:, K_s]^T over the
    s-th of ``splits`` contiguous K ranges (f32 [splits, M, N]; 1 <= M <= 16). With the
    default ``splits`` (gemv_split_count) they add up, in split order, to gemm_q4's Y bit
    for bit. The planes go to gemm_q4_rmsnorm_acc / swiglu_q4_acc, which add them to the
    residual stream in place of gemm_q4(residual=...)'s reduce launch."""
    _bf16_scales("gemm_q4_partials", w)
    dev = w.device
    xt = _acts(x, dev)
    if xt.dim() == 1:
        xt = xt.unsqueeze(0)
    M, K = xt.shape
    if K != w.k:
        raise ValueError(f"x has K={K}, W is [{w.n}, {w.k}]")
    if not 1 <= M <= 16:
        raise ValueError(f"gemm_q4_partials takes 1..16 tokens, got {M}")
    S = gemv_split_count(w) if splits is None else int(splits)
    if not 1 <= S <= min(16, w.k // 32):
        raise ValueError(f"splits must be 1..{min(16, w.k // 32)}, got {S}")
    part = _buf(part, "part", torch.float32, (S, M, w.n), dev)
    lib = _lib_handle()
    with torch.cuda.device(dev):
        check("q4_gemv_partials", lib.q4_gemv_partials(_ptr(w.data), _ptr(xt), _x_dtype(xt), _ptr(part), S, M, w.n,
                                                       w.k, _stream(dev)))
    return part


def _acc_args(res: torch.Tensor, partials, x_out, K: int, dev):
    xt = _norm_x(res, K, dev)
    M = xt.shape[0]
    if partials is None:
        S, pp = 0, None
    else:
        if not isinstance(partials, torch.Tensor) or partials.dtype != torch.float32 or partials.device != dev \
                or not partials.is_contiguous() or partials.dim() != 3 or tuple(partials.shape[1:]) != (M, K):
            raise ValueError(f"partials must be a contiguous float32 [S, {M}, {K}] tensor on {dev}")
        S, pp = partials.shape[0], _ptr(partials)
        if not 1 <= S <= 16:
            raise ValueError(f"partials hold 1..16 planes, got {S}")
    x_out = _buf(x_out, "x_out", torch.float32, (M, K), dev)
    lo, hi = x_out.data_ptr(), x_out.data_ptr() + x_out.numel() * 4
    for t in (res, partials):
        if t is not None and t.data_ptr() < hi and lo < t.data_ptr() + t.numel() * 4:
            raise ValueError("x_out must not overlap res or partials")
    return xt, M, S, pp, x_out


def gemm_q4_rmsnorm_acc(w: PackedQ4, res: torch.Tensor, partials: torch.Tensor | None, norm_w: torch.Tensor,
                        eps: float = 1e-6, x_out: torch.Tensor | None = None, y: torch.Tensor | None = None,
                        workspace: torch.Tensor | None = None):
    """(y, x_out): x_out = res + the partial planes added in split order (gemm_q4(...,
    residual=res)'s bits for the GEMV that made them), then y = gemm_q4_rmsnorm(w, x_out,
    norm_w) -- with the reduction inside the norm GEMV's workgroups at M = 1 (K <= 4096)
    instead of a launch of its own. ``x_out`` must not share memory with ``res``."""
    _bf16_scales("gemm_q4_rmsnorm_acc", w)
    dev = w.device
    xt, M, S, pp, x_out = _acc_args(res, partials, x_out, w.k, dev)
    if not 1 <= M <= 16:
        raise ValueError(f"gemm_q4_rmsnorm_acc takes 1..16 tokens, got {M}")
    wt, wd = _norm_w(norm_w, w.k, dev)
    y = _buf(y, "y", torch.float32, (M, w.n), dev)
    lib = _lib_handle()
    with torch.cuda.device(dev):
        wp, wn = _ws_arg(dev, _norm_ws_bytes(lib, M, w, workspace), "gemv", workspace)
        check("q4_gemv_rmsnorm_acc", lib.q4_gemv_rmsnorm_acc(_ptr(w.data), _ptr(xt), pp, S, _ptr(wt), wd, float(eps),
                                                             _ptr(x_out), _ptr(y), M, w.n, w.k, wp, wn,
                                                             _stream(dev)))
    return y, x_out


def swiglu_q4_acc(gate: PackedQ4, up: PackedQ4, res: torch.Tensor, partials: torch.Tensor | None,
                  norm_w: torch.Tensor, eps: float = 1e-6, out_dtype=torch.float32, x_out: torch.Tensor | None = None,
                  h: torch.Tensor | None = None, workspace: torch.Tensor | None = None):
    """(h, x_out): x_out = res + partials as in gemm_q4_rmsnorm_acc, then h =
    swiglu_q4(gate, up, x_out, norm_w=norm_w)."""
    _bf16_scales("swiglu_q4_acc", gate, up)
    if gate.n != up.n or gate.k != up.k or gate.device != up.device:
        raise ValueError(f"gate {gate.shape} and up {up.shape} must match")
    dev = gate.device
    xt, M, S, pp, x_out = _acc_args(res, partials, x_out, gate.k, dev)
    if not 1 <= M <= 16:
        raise ValueError(f"swiglu_q4_acc takes 1..16 tokens, got {M}")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("out_dtype must be float32 or bfloat16")
    wt, wd = _norm_w(norm_w, gate.k, dev)
    h = _buf(h, "h", out_dtype, (M, gate.n), dev)
    lib = _lib_handle()
    with torch.cuda.device(dev):
        wp, wn = _ws_arg(dev, lib.q4_gemv_swiglu_workspace_bytes(M, gate.n, gate.k), "swiglu", workspace)
        check("q4_gemv_swiglu_rmsnorm_acc", lib.q4_gemv_swiglu_rmsnorm_acc(
            _ptr(gate.data), _ptr(up.data), _ptr(xt), pp, S, _ptr(wt), wd, float(eps), _ptr(x_out), _ptr(h),
            Q4MI_BF16 if out_dtype == torch.bfloat16 else Q4MI_F32, M, gate.n, gate.k, wp, wn, _stream(dev)))
    return h, x_out


def swiglu_q4(gate: PackedQ4, up: PackedQ4, x, out_dtype=torch.float32, h: torch.Tensor | None = None,
              workspace: torch.Tensor | None = None, norm_w: torch.Tensor | None = None,
              eps: float = 1e-6) -> torch.Tensor:
    """h[M, F] = silu(X @ G^T) * (X @ U^T) for 1 <= M <= 16 tokens in one launch (two
    when K is split): the gate/up GEMVs with the silu_mul design fused as their
    epilogue (designs/silu_mul/silu_mul.cc). ``out_dtype`` float32 or bfloat16 (RNE),
    the down projection's input. With ``norm_w``, x is the f32 residual stream and
    X = bf16(RMSNorm(x) * norm_w) is formed inside the kernel (rmsnorm_add's bits)."""
    _bf16_scales("swiglu_q4", gate, up)
    if gate.n != up.n or gate.k != up.k or gate.device != up.device:
        raise ValueError(f"gate {gate.shape} and up {up.shape} must match")
    dev = gate.device
    if norm_w is not None:
        xt = _norm_x(x, gate.k, dev)
        M = xt.shape[0]
        if not 1 <= M <= 16:
            raise ValueError(f"swiglu_q4 with a norm takes 1..16 tokens, got {M}")
        wt, wd = _norm_w(norm_w, gate.k, dev)
        if out_dtype not in (torch.float32, torch.bfloat16):
            raise TypeError("out_dtype must be float32 or bfloat16")
        h = _buf(h, "h", out_dtype, (M, gate.n), dev)
        lib = _lib_handle()
        with torch.cuda.device(dev):
            wp, wn = _ws_arg(dev, lib.q4_gemv_swiglu_workspace_bytes(M, gate.n, gate.k), "swiglu", workspace)
            check("q4_gemv_swiglu_rmsnorm", lib.q4_gemv_swiglu_rmsnorm(
                _ptr(gate.data), _ptr(up.data), _ptr(xt), _ptr(wt), wd, float(eps), _ptr(h),
                Q4MI_BF16 if out_dtype == torch.bfloat16 else Q4MI_F32, M, gate.n, gate.k, wp, wn, _stream(dev)))
        return h
    xt = _acts(x, dev)
    if xt.dim() == 1:
        xt = xt.unsqueeze(0)
    M, K = xt.shape
    if K != gate.k:
        raise ValueError(f"x has K={K}, gate/up are [{gate.n}, {gate.k}]")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("out_dtype must be float32 or bfloat16")
    h = _buf(h, "h", out_dtype, (M, gate.n), dev)
    lib = _lib_handle()
    with torch.cuda.device(dev):
        wp, wn = _ws_arg(dev, lib.q4_gemv_swiglu_workspace_bytes(M, gate.n, gate.k), "swiglu", workspace)
        check("q4_gemv_swiglu", lib.q4_gemv_swiglu(_ptr(gate.data), _ptr(up.data), _ptr(xt), _x_dtype(xt), _ptr(h),
                                                   Q4MI_BF16 if out_dtype == torch.bfloat16 else Q4MI_F32, M,
                                                   gate.n, gate.k, wp, wn, _stream(dev)))
    return h


def decode_segment_splits(h: int, f: int, nq: int) -> tuple[int, int, int]:
    """(So, Sd, Sq): the K splits of o, down and qkv in decode_segment for hidden size h,
    FFN size f and nq qkv rows (nq = 0: no qkv; Sq 0)."""
    out = (C.c_int * 3)()
    check("q4_decode_segment_splits", _lib_handle().q4_decode_segment_splits(h, f, nq, out))
    return int(out[0]), int(out[1]), int(out[2])


def decode_segment_workspace(h: int, f: int, nq: int, device=None) -> torch.Tensor:
    """A zero-filled workspace for decode_segment at these sizes (its counters must start at
    zero; every call leaves them at zero, so one workspace serves all calls of a stream)."""
    n = int(_lib_handle().q4_decode_segment_workspace_bytes(h, f, nq))
    if n == 0:
        raise ValueError(f"decode_segment does not take h={h}, f={f}, nq={nq}")
    return torch.zeros(n, dtype=torch.uint8, device=_device(device))


def decode_segment(o: PackedQ4, gate: PackedQ4, up: PackedQ4, down: PackedQ4, qkv: PackedQ4 | None,
                   attn: torch.Tensor, x: torch.Tensor, nw_post: torch.Tensor, nw_next: torch.Tensor | None = None,
                   eps: float = 1e-6, x_mid: torch.Tensor | None = None, x_next: torch.Tensor | None = None,
                   down_planes: torch.Tensor | None = None, qkv_planes: torch.Tensor | None = None,
                   workspace: torch.Tensor | None = None):
    """The decoder layer's GEMVs between two attentions at M = 1, in one launch (the
    reference's whole-layer dispatch, designs/dense/dx.py:1-5, attention left out):

        x_mid  = x + o @ attn
        h      = bf16(silu(gate @ n1) * (up @ n1)),   n1 = bf16(RMSNorm(x_mid) * nw_post)
        x_next = x_mid + down @ h                     (down_planes: its K splits, f32 [Sd, H])
        qkv    = sum over s of qkv_planes[s]          (f32 [Sq, NQ]; qkv @ n2,
                                                       n2 = bf16(RMSNorm(x_next) * nw_next))

    attn bf16 [H]; x the f32 residual stream [H] (``x_next`` may be ``x``); norm weights f32
    or bf16 [H]. ``qkv`` None (the last layer) stops after down: x_next and qkv_planes are
    not formed, and gemm_q4_rmsnorm_acc(lm_head, x_mid, down_planes, ...) goes on from
    there. Returns (x_mid, x_next, down_planes, qkv_planes). ``workspace`` from
    decode_segment_workspace (else a zero-filled one per call)."""
    mats = [o, gate, up, down] + ([qkv] if qkv is not None else [])
    _bf16_scales("decode_segment", *mats)
    dev = o.device
    H, F = o.k, gate.n
    NQ = qkv.n if qkv is not None else 0
    if o.n != H or gate.shape != (F, H) or up.shape != (F, H) or down.shape != (H, F) \
            or (qkv is not None and qkv.k != H) or any(m.device != dev for m in mats):
        raise ValueError(f"decode_segment needs o [H, H], gate/up [F, H], down [H, F], qkv [NQ, H] on one device; "
                         f"got {[m.shape for m in mats]}")
    So, Sd, Sq = decode_segment_splits(H, F, NQ)
    if not isinstance(attn, torch.Tensor) or attn.dtype != torch.bfloat16 or attn.numel() != H \
            or attn.device != dev or not attn.is_contiguous():
        raise ValueError(f"attn must be a contiguous bfloat16 tensor of {H} values on {dev}")
    xt = _norm_x(x, H, dev)
    if xt.shape[0] != 1:
        raise ValueError("decode_segment takes one token")
    wpost, wd = _norm_w(nw_post, H, dev)
    wnext = None
    if qkv is not None:
        if nw_next is None:
            raise ValueError("nw_next is needed with qkv")
        wnext, wd2 = _norm_w(nw_next, H, dev)
        if wd2 != wd:
            raise TypeError("nw_post and nw_next must share a dtype")
    x_mid = _buf(x_mid, "x_mid", torch.float32, (1, H), dev)
    down_planes = _buf(down_planes, "down_planes", torch.float32, (Sd, 1, H), dev)
    if qkv is not None:
        x_next = _buf(x_next, "x_next", torch.float32, (1, H), dev)
        qkv_planes = _buf(qkv_planes, "qkv_planes", torch.float32, (Sq, 1, NQ), dev)
    else:
        x_next = qkv_planes = None
    if workspace is None:
        workspace = decode_segment_workspace(H, F, NQ, dev)
    lib = _lib_handle()
    with torch.cuda.device(dev):
        wp, wn = _ws_arg(dev, lib.q4_decode_segment_workspace_bytes(H, F, NQ), "decode_segment", workspace)
        opt = lambda t: None if t is None else _ptr(t)
        check("q4_decode_segment", lib.q4_decode_segment(
            _ptr(o.data), _ptr(gate.data), _ptr(up.data), _ptr(down.data), opt(qkv.data if qkv is not None else None),
            _ptr(attn), _ptr(xt), _ptr(wpost), opt(wnext), wd, float(eps), _ptr(x_mid), opt(x_next),
            _ptr(down_planes), opt(qkv_planes), H, F, NQ, wp, wn, _stream(dev)))
    return x_mid, x_next, down_planes, qkv_planes


def rmsnorm_add(x: torch.Tensor, w: torch.Tensor, add: torch.Tensor | None = None, eps: float = 1e-6,
                out_dtype=torch.bfloat16, y: torch.Tensor | None = None, xn: torch.Tensor | None = None):
    """(y, xn): y = x + add (f32; x itself when add is None and y is not given) and
    xn = (y * rsqrt(mean(y^2) + eps)) * w stored as ``out_dtype`` -- the ln design
    (designs/ln/ln.py:1-6). ``w`` float32 or bfloat16 [N]; ``y`` may be ``x``."""
    if x.dtype != torch.float32 or not x.is_cuda or not x.is_contiguous():
        raise TypeError("x must be a contiguous float32 GPU tensor")
    x2 = x.view(-1, x.shape[-1])
    M, N = x2.shape
    dev = x.device
    if w.numel() != N or w.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"w must be float32 or bfloat16 with {N} values")
    wt = w.to(dev).contiguous()
    if add is not None:
        add = _buf(add, "add", torch.float32, tuple(x.shape), dev)
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("out_dtype must be float32 or bfloat16")
    if y is not None or add is not None:
        y = _buf(y, "y", torch.float32, tuple(x.shape), dev)
    if y is not None and N > 16384 and y.data_ptr() == x.data_ptr():
        raise ValueError("y may alias x only for rows of <= 16384 values")
    xn = _buf(xn, "xn", out_dtype if xn is None else xn.dtype, tuple(x.shape), dev)
    if xn.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"xn must be float32 or bfloat16, got {xn.dtype}")
    with torch.cuda.device(dev):
        check("q4_rmsnorm_add", _lib_handle().q4_rmsnorm_add(
            _ptr(x), None if add is None else _ptr(add), _ptr(wt), Q4MI_BF16 if wt.dtype == torch.bfloat16 else Q4MI_F32,
            None if y is None else _ptr(y), _ptr(xn), Q4MI_BF16 if xn.dtype == torch.bfloat16 else Q4MI_F32, M, N,
            float(eps), _stream(dev)))
    return (x if y is None else y), xn


def gemv_q4(w: PackedQ4, x, y: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """y[N] = W[N, K] @ x[K], fp32 out (gemv_q4.py:118-123: pool in, bf16 x in, f32 y out)."""
    xt = _acts(x, w.device)
    if xt.dim() != 1:
        raise ValueError("gemv_q4 takes one activation vector x[K]")
    if y is not None:
        y = _buf(y, "y", torch.float32, (w.n,), w.device).view(1, -1)
    out = gemm_q4(w, xt.unsqueeze(0), y, workspace)
    return out.view(-1)


# --------------------------------------------------------------------------
# lm_head and its sampling epilogue
# --------------------------------------------------------------------------

_TOPK_MODES = {"f32": 0, "sampler": 1}


def _topk_mode(mode) -> int:
    if mode not in _TOPK_MODES:
        raise ValueError(f"mode must be one of {sorted(_TOPK_MODES)}, got {mode!r}")
    return _TOPK_MODES[mode]


def _topk_outputs(M: int, k: int, dev, ids, vals):
    if not 1 <= k <= 64:
        raise ValueError(f"k must be in 1..64, got {k}")
    return _buf(ids, "ids", torch.int32, (M, k), dev), _buf(vals, "vals", torch.float32, (M, k), dev)


def logits_topk(logits: torch.Tensor, k: int = 1, mode: str = "sampler", n_valid: int | None = None,
                workspace: torch.Tensor | None = None, ids: torch.Tensor | None = None,
                vals: torch.Tensor | None = None):
    """The k largest logits of each row (value descending, lower id first on a tie),
    as (ids int32[M, k], vals f32[M, k]); k = 1 is the greedy argmax.

    mode "sampler" ranks what the reference's sampler sees -- each logit rounded to
    bf16, an f32 subnormal read as 0 (Sampler::sample_greedy / sampler_topk_apply,
    src/common/modules/sampler.cpp:222-245, :355-430); "f32" ranks the logits as they
    are. Rows past ``n_valid`` (padding beyond the tokenizer's vocabulary) are skipped."""
    if logits.dtype != torch.float32 or not logits.is_cuda:
        raise TypeError("logits must be a float32 GPU tensor")
    lg = logits if logits.dim() == 2 else logits.view(1, -1)
    if lg.stride(1) != 1:
        raise ValueError("logits rows must be contiguous")
    M, N = lg.shape
    n = N if n_valid is None else int(n_valid)
    if not 0 <= n <= N:
        raise ValueError(f"n_valid must be in 0..{N}, got {n}")
    dev = lg.device
    ids, vals = _topk_outputs(M, k, dev, ids, vals)
    lib = _lib_handle()
    with torch.cuda.device(dev):
        wp, wn = _ws_arg(dev, lib.q4_topk_workspace_bytes(M, n, k), "topk", workspace)
        check("q4_logits_topk", lib.q4_logits_topk(_ptr(lg), lg.stride(0), M, n, k, _topk_mode(mode),
                                                   _ptr(ids), _ptr(vals), wp, wn, _stream(dev)))
    return ids, vals


def lm_head_topk(w: PackedQ4, x, k: int = 1, mode: str = "sampler", n_valid: int | None = None,
                 logits: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                 ids: torch.Tensor | None = None, vals: torch.Tensor | None = None):
    """lm_head over 1..16 tokens and its sampling epilogue in one call:
    (ids int32[M, k], vals f32[M, k], logits f32[M, N]) (designs/lm_head_q4 plus the
    host's greedy / top-k pass; see logits_topk for ``mode`` and ``n_valid``)."""
    _bf16_scales("lm_head_topk", w)
    dev = w.device
    xt = _acts(x, dev)
    if xt.dim() == 1:
        xt = xt.unsqueeze(0)
    M, K = xt.shape
    if K != w.k:
        raise ValueError(f"x has K={K}, W is [{w.n}, {w.k}]")
    n = w.n if n_valid is None else int(n_valid)
    if not 0 <= n <= w.n:
        raise ValueError(f"n_valid must be in 0..{w.n}, got {n}")
    logits = _buf(logits, "logits", torch.float32, (M, w.n), dev)
    ids, vals = _topk_outputs(M, k, dev, ids, vals)
    lib = _lib_handle()
    with torch.cuda.device(dev):
        wp, wn = _ws_arg(dev, lib.q4_lm_head_workspace_bytes(M, w.n, w.k, k), "lm_head", workspace)
        check("q4_lm_head_topk", lib.q4_lm_head_topk(_ptr(w.data), _ptr(xt), _x_dtype(xt), _ptr(logits), M, w.n,
                                                     w.k, n, k, _topk_mode(mode), _ptr(ids), _ptr(vals), wp, wn,
                                                     _stream(dev)))
    return ids, vals, logits


class GemvGroup:
    """Many independent GEMVs (same M, same activation dtype) as ONE launch.

    ``items`` is a list of (PackedQ4, x[M, K], y[M, N]) on one device; the
    descriptor table is built and uploaded once, so ``run()`` is a single
    kernel launch -- the counterpart of the reference's fused dispatches that
    run several projections' bands in one xclbin (gemv_q4.py:46-53)."""

    def __init__(self, items):
        if not items:
            raise ValueError("empty group")
        dev = items[0][0].device
        descs = (Q4GemvDesc * len(items))()
        begin = 0
        m0 = dt = None
        self._keep = []
        self.scales = items[0][0].scales
        for i, (w, x, y) in enumerate(items):
            if w.scales != self.scales:
                raise ValueError("all group members need the same scale form (bf16 or fp16)")
            if x.device != dev or y.device != dev or w.device != dev:
                raise ValueError("all group members must be on one device")
            xx = x if x.dim() == 2 else x.view(1, -1)
            M, K = xx.shape
            if K != w.k or tuple(y.reshape(M, -1).shape) != (M, w.n) or y.dtype != torch.float32:
                raise ValueError(f"item {i}: x {tuple(xx.shape)} / y {tuple(y.shape)} do not fit W {w.shape}")
            if not (xx.is_contiguous() and y.is_contiguous()):
                raise ValueError(f"item {i}: x and y must be contiguous")
            m0 = M if m0 is None else m0
            d = _x_dtype(xx)
            dt = d if dt is None else dt
            if M != m0 or d != dt:
                raise ValueError("all group members need the same M and activation dtype")
            packed_bytes(w.n, w.k)
            descs[i] = Q4GemvDesc(_ptr(w.data), _ptr(xx), _ptr(y), w.n, w.k, begin)
            begin += w.n // ROWS
            self._keep.append((w, xx, y))
        if not 1 <= m0 <= 16:
            raise ValueError("GemvGroup takes 1..16 tokens")
        raw = np.frombuffer(bytes(descs), dtype=np.uint8)
        self.table = torch.from_numpy(raw.copy()).to(dev)
        self.count = len(items)
        self.total_items = begin
        self.M = m0
        self.x_dtype = dt
        self.device = dev
        self.weight_bytes = sum(w.nbytes for w, _, _ in self._keep)

    def run(self) -> None:
        fn = "q4_gemv_grouped_fp16s" if self.scales == "fp16" else "q4_gemv_grouped"
        with torch.cuda.device(self.device):
            check(fn, getattr(_lib_handle(), fn)(
                _ptr(self.table), self.count, self.total_items, self.M, self.x_dtype, _stream(self.device)))

    __call__ = run


# --------------------------------------------------------------------------
# prefill GEMM
# --------------------------------------------------------------------------

_PRECISION = {"fp16": 0, "bf16": 1}


def prefill_scales(w) -> torch.Tensor:
    """The matrix's fp16 prefill scales (per-row power-of-two exponents and the scale words
    in fp16, q4_prefill_scales), computed on first use and kept on ``w`` (a PackedQ4, or a
    PackedExperts as its stacked [E n, k] matrix)."""
    _bf16_scales("prefill_scales", w)
    if w.prefill_scales is None:
        dev = w.data.device
        n = w.n * w.experts if isinstance(w, PackedExperts) else w.n
        lib = _lib_handle()
        t = torch.empty(int(lib.q4_prefill_scales_bytes(n, w.k)), dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            check("q4_prefill_scales", lib.q4_prefill_scales(_ptr(w.data), n, w.k, _ptr(t), t.numel(), _stream(dev)))
        w.prefill_scales = t
    return w.prefill_scales


@dataclass
class PreparedActs:
    """Activations [t, k] converted once for the prefill GEMM (q4_prefill_prepare): the
    GEMM's 16-bit tiled image (fp16 scaled per token row by a power of two, or bf16), so
    several projections of the same input (gate and up, Q / K / V) read it without
    converting it again."""
    data: torch.Tensor
    t: int
    k: int
    x_dtype: int
    precision: str


def prefill_prepare(x, precision: str = "fp16", out: torch.Tensor | None = None) -> PreparedActs:
    """Convert X [T, K] (bf16 or f32) for gemm_q4_prefill once (its activation pre-pass)."""
    if precision not in _PRECISION:
        raise ValueError(f"precision must be one of {sorted(_PRECISION)}, got {precision!r}")
    dev = _device(x.device if isinstance(x, torch.Tensor) and x.is_cuda else None)
    xt = _acts(x, dev)
    if xt.dim() != 2:
        raise ValueError(f"x must be [T, K], got {tuple(xt.shape)}")
    T, K = xt.shape
    lib = _lib_handle()
    nbytes = int(lib.q4_prefill_prepared_bytes(T, K, _x_dtype(xt), _PRECISION[precision])) if T else 0
    if T and nbytes == 0:
        raise ValueError(f"[{T}, {K}] cannot be prepared (K % 32 == 0)")
    data = _buf(out, "out", torch.uint8, (nbytes,), dev)
    if T:
        with torch.cuda.device(dev):
            check("q4_prefill_prepare", lib.q4_prefill_prepare(_ptr(xt), _x_dtype(xt), T, K, _PRECISION[precision],
                                                               _ptr(data), nbytes, _stream(dev)))
    return PreparedActs(data, T, K, _x_dtype(xt), precision)


def rmsnorm_prepare(x: torch.Tensor, w: torch.Tensor, add: torch.Tensor | None = None, eps: float = 1e-6,
                    precision: str = "fp16", y: torch.Tensor | None = None,
                    out: torch.Tensor | None = None) -> tuple[torch.Tensor, PreparedActs]:
    """(y, prepared): the RMSNorm producer writing the prefill GEMM's prepared activations in
    one launch -- y = x + add (f32 [T, K]; x itself when add is None and y is not given) and
    prefill_prepare(bf16((y * rsqrt(mean(y^2) + eps)) * w)), bit for bit what rmsnorm_add
    (bf16 out) followed by prefill_prepare gives (designs/ln/ln.py:1-6 in front of the
    host's X tiling, block_host.cpp:228-244). ``add`` [T, K], or [S, T, K] partial planes
    (gemm_q4_prefill_partials) summed in the split reduce's order, so no reduce launch runs.
    ``w`` float32 or bfloat16 [K]; ``y`` may be ``x``; K % 32 == 0, K <= 16384."""
    if precision not in _PRECISION:
        raise ValueError(f"precision must be one of {sorted(_PRECISION)}, got {precision!r}")
    if not isinstance(x, torch.Tensor) or x.dtype != torch.float32 or not x.is_cuda or not x.is_contiguous() \
            or x.dim() != 2:
        raise TypeError("x must be a contiguous float32 [T, K] GPU tensor")
    T, K = x.shape
    dev = x.device
    if K % 32 or K > 16384:
        raise ValueError(f"K must be a multiple of 32 up to 16384, got {K}")
    if w.numel() != K or w.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"w must be float32 or bfloat16 with {K} values")
    wt = w.to(dev).contiguous()
    planes = 0
    if add is not None:
        planes = add.shape[0] if isinstance(add, torch.Tensor) and add.dim() == 3 else 1
        if not 1 <= planes <= 64:
            raise ValueError(f"add holds 1..64 planes, got {planes}")
        add = _buf(add, "add", torch.float32, (planes, T, K) if add.dim() == 3 else (T, K), dev)
    if y is not None or add is not None:
        y = _buf(y, "y", torch.float32, (T, K), dev)
    lib = _lib_handle()
    nbytes = int(lib.q4_prefill_prepared_bytes(T, K, Q4MI_BF16, _PRECISION[precision])) if T else 0
    data = _buf(out, "out", torch.uint8, (nbytes,), dev)
    if T:
        with torch.cuda.device(dev):
            check("q4_rmsnorm_prepare", lib.q4_rmsnorm_prepare(
                _ptr(x), None if add is None else _ptr(add), planes, _ptr(wt),
                Q4MI_BF16 if wt.dtype == torch.bfloat16 else Q4MI_F32, None if y is None else _ptr(y), T, K,
                float(eps), _PRECISION[precision], _ptr(data), nbytes, _stream(dev)))
    return (x if y is None else y), PreparedActs(data, T, K, Q4MI_BF16, precision)


def swiglu_prepare(g: torch.Tensor, u: torch.Tensor | None = None, precision: str = "fp16",
                   out: torch.Tensor | None = None, h: torch.Tensor | None = None) -> PreparedActs:
    """The SwiGLU producer writing the down projection's prepared activations in one launch:
    h = bf16(silu(g) * u) per token row (moe_batch.h:181-202's h) and prefill_prepare(h),
    bit for bit. ``g``, ``u`` float32 [T, F] row views (any row stride, unit column stride);
    with ``u`` None, ``g`` is the fused [T, 2F] gate/up output and its halves are taken.
    ``h`` (bf16 [T, F]) also receives h when given."""
    if precision not in _PRECISION:
        raise ValueError(f"precision must be one of {sorted(_PRECISION)}, got {precision!r}")
    if not isinstance(g, torch.Tensor) or g.dtype != torch.float32 or not g.is_cuda or g.dim() != 2:
        raise TypeError("g must be a float32 [T, F] GPU tensor")
    if u is None:
        if g.shape[1] % 2:
            raise ValueError("a fused gate/up output has an even number of columns")
        F = g.shape[1] // 2
        g, u = g[:, :F], g[:, F:]
    if u.dtype != torch.float32 or u.device != g.device or u.shape != g.shape:
        raise ValueError(f"u must be float32 {tuple(g.shape)} on {g.device}")
    for name, t_ in (("g", g), ("u", u)):
        if t_.stride(1) != 1 or t_.stride(0) % 4 or t_.data_ptr() % 16:
            raise ValueError(f"{name} needs unit column stride, a row stride of 4k and 16-byte alignment")
    T, F = g.shape
    dev = g.device
    if F % 32 or F > 16384:
        raise ValueError(f"F must be a multiple of 32 up to 16384, got {F}")
    if h is not None:
        h = _buf(h, "h", torch.bfloat16, (T, F), dev)
    lib = _lib_handle()
    nbytes = int(lib.q4_prefill_prepared_bytes(T, F, Q4MI_BF16, _PRECISION[precision])) if T else 0
    data = _buf(out, "out", torch.uint8, (nbytes,), dev)
    if T:
        with torch.cuda.device(dev):
            check("q4_swiglu_prepare", lib.q4_swiglu_prepare(
                _ptr(g), _ptr(u), g.stride(0), u.stride(0), T, F, _PRECISION[precision],
                None if h is None else _ptr(h), _ptr(data), nbytes, _stream(dev)))
    return PreparedActs(data, T, F, Q4MI_BF16, precision)


def interleave_gate_up(gate: PackedQ4, up: PackedQ4) -> PackedQ4:
    """One mx matrix [2F, K] whose 64-row groups alternate gate / up (a device copy of the two
    matrices' row groups): the layout gemm_q4_prefill_swiglu and the MoE experts take."""
    _bf16_scales("interleave_gate_up", gate, up)
    if gate.n != up.n or gate.k != up.k or gate.device != up.device:
        raise ValueError("gate and up must have the same shape and device")
    rg = gate.nbytes // (gate.n // 64)
    g = gate.data[:gate.nbytes].view(gate.n // 64, rg)
    u = up.data[:up.nbytes].view(up.n // 64, rg)
    return PackedQ4(torch.stack((g, u), 1).reshape(-1), 2 * gate.n, gate.k)


def gemm_q4_prefill_swiglu(gate_up: PackedQ4, x, h: torch.Tensor | None = None,
                           precision: str = "fp16") -> torch.Tensor:
    """h [T, F] bf16 = bf16(silu(X G^T) * (X U^T)): the FFN's gate/up prefill GEMM with the
    SwiGLU in its epilogue (moe_batch.h:181-202's bf16 h), over an interleaved gate/up matrix
    (interleave_gate_up) and bf16 or prepared activations; the same h swiglu_prepare forms
    from the plain GEMM's f32 outputs, with no f32 output in memory. F % 128 == 0, K % 64 == 0."""
    _bf16_scales("gemm_q4_prefill_swiglu", gate_up)
    dev = gate_up.device
    if isinstance(x, PreparedActs):
        if x.data.device != dev:
            raise ValueError(f"prepared activations are on {x.data.device}, W on {dev}")
        precision = x.precision
        prep = x
    else:
        xt = _acts(x, dev)
        if xt.dtype != torch.bfloat16 and precision == "fp16":
            raise ValueError("the SwiGLU epilogue takes one activation pass: bf16 x, or precision 'bf16'")
        prep = prefill_prepare(xt, precision)
    if precision not in _PRECISION:
        raise ValueError(f"precision must be one of {sorted(_PRECISION)}, got {precision!r}")
    if prep.k != gate_up.k:
        raise ValueError(f"x has K={prep.k}, W is [{gate_up.n}, {gate_up.k}]")
    T, F = prep.t, gate_up.n // 2
    if F % 128 or gate_up.k % 64:
        raise ValueError(f"the SwiGLU epilogue needs F % 128 == 0 and K % 64 == 0, got F={F}, K={gate_up.k}")
    h = _buf(h, "h", torch.bfloat16, (T, F), dev)
    sc = prefill_scales(gate_up) if precision == "fp16" else None
    if T:
        with torch.cuda.device(dev):
            check("q4_gemm_prefill_swiglu", _lib_handle().q4_gemm_prefill_swiglu(
                _ptr(gate_up.data), None if sc is None else _ptr(sc), _ptr(prep.data), prep.x_dtype, _ptr(h), T, F,
                gate_up.k, _PRECISION[precision], _stream(dev)))
    return h


def gemm_q4_prefill_partials(w: PackedQ4, x: PreparedActs, part: torch.Tensor | None = None) -> torch.Tensor:
    """The prepared prefill GEMM without its K-split reduce: f32 [S, T, N] planes whose ordered
    sum is gemm_q4_prefill's Y bit for bit (S = the plan's split count, 1 when unsplit). They go
    to rmsnorm_prepare(add=...), which sums them in the residual add of the next norm
    (the reference sums its down K-pieces on the host, ironutil.py:98-115)."""
    _bf16_scales("gemm_q4_prefill_partials", w)
    if not isinstance(x, PreparedActs):
        raise TypeError("gemm_q4_prefill_partials takes prepared activations (prefill_prepare / rmsnorm_prepare)")
    if x.k != w.k:
        raise ValueError(f"x has K={x.k}, W is [{w.n}, {w.k}]")
    dev = w.device
    if x.data.device != dev:
        raise ValueError(f"prepared activations are on {x.data.device}, W on {dev}")
    lib = _lib_handle()
    S = max(1, int(lib.q4_prefill_split_count(max(x.t, 1), w.n, w.k)))
    part = _buf(part, "part", torch.float32, (S, x.t, w.n), dev)
    sc = prefill_scales(w) if x.precision == "fp16" else None
    if x.t:
        with torch.cuda.device(dev):
            check("q4_gemm_prefill_prepared_partials", lib.q4_gemm_prefill_prepared_partials(
                _ptr(w.data), None if sc is None else _ptr(sc), _ptr(x.data), x.x_dtype, _ptr(part),
                part.numel() * 4, x.t, w.n, w.k, _PRECISION[x.precision], _stream(dev)))
    return part


def gemm_q4_prefill(w: PackedQ4, x, y: torch.Tensor | None = None, precision: str = "fp16",
                    workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Y[T, N] = X[T, K] @ W^T for a prefill block of T tokens, fp32 out.

    precision "fp16": each weight rounded once to fp16 in LDS (fp16 MFMA), weight and token
    rows scaled into fp16's range by powers of two (the matrix's prefill scales, computed
    once and kept on ``w``); "bf16": the reference tile RNE_bf16(fl32(q*d+m))
    (gemm_q4_dequant.h:283-286). ``x`` may be a PreparedActs (its own precision is used)."""
    _bf16_scales("gemm_q4_prefill", w)
    dev = w.device
    if isinstance(x, PreparedActs):
        if x.k != w.k:
            raise ValueError(f"prepared activations have K={x.k}, W is [{w.n}, {w.k}]")
        if x.data.device != dev:
            raise ValueError(f"prepared activations are on {x.data.device}, W on {dev}")
        T, prec = x.t, _PRECISION[x.precision]
        y = _buf(y, "y", torch.float32, (T, w.n), dev)
        if T == 0 or w.n == 0:
            return y
        lib = _lib_handle()
        sc = prefill_scales(w) if x.precision == "fp16" else None
        with torch.cuda.device(dev):
            wp, wn = _ws_arg(dev, lib.q4_gemm_prefill_prepared_workspace_bytes(T, w.n, w.k), "prefill", workspace)
            check("q4_gemm_prefill_prepared", lib.q4_gemm_prefill_prepared(
                _ptr(w.data), None if sc is None else _ptr(sc), _ptr(x.data), x.x_dtype, _ptr(y), T, w.n, w.k, prec,
                wp, wn, _stream(dev)))
        return y
    xt = _acts(x, dev)
    if xt.dim() != 2 or xt.shape[1] != w.k:
        raise ValueError(f"x must be [T, {w.k}], got {tuple(xt.shape)}")
    T = xt.shape[0]
    if precision not in _PRECISION:
        raise ValueError(f"precision must be one of {sorted(_PRECISION)}, got {precision!r}")
    y = _buf(y, "y", torch.float32, (T, w.n), dev)
    lib = _lib_handle()
    if precision == "fp16" and T > 0 and w.n > 0:
        sc = prefill_scales(w)
        with torch.cuda.device(dev):
            wp, wn = _ws_arg(dev, lib.q4_gemm_prefill_scaled_workspace_bytes(T, w.n, w.k), "prefill", workspace)
            check("q4_gemm_prefill_scaled", lib.q4_gemm_prefill_scaled(
                _ptr(w.data), _ptr(sc), _ptr(xt), _x_dtype(xt), _ptr(y), T, w.n, w.k, wp, wn, _stream(dev)))
        return y
    with torch.cuda.device(dev):
        wp, wn = _ws_arg(dev, lib.q4_gemm_prefill_workspace_bytes(T, w.n, w.k), "prefill", workspace)
        check("q4_gemm_prefill", lib.q4_gemm_prefill(
            _ptr(w.data), _ptr(xt), _x_dtype(xt), _ptr(y), T, w.n, w.k, _PRECISION[precision], wp, wn,
            _stream(dev)))
    return y


# --------------------------------------------------------------------------
# routed MoE
# --------------------------------------------------------------------------

def pack_moe_experts(gate_blocks, up_blocks, down_blocks, device=None):
    """Per-expert GGUF blocks -> (gate_up, down) PackedExperts.

    gate_up expert e is one [2F, H] mx matrix whose 64-row groups alternate
    gate rows and the same up rows (the counterpart of the reference pool's
    interleaved up/gate stripes, moe_batch/make_test.py:35-59); down expert e
    is [H, F]."""
    dev = _device(device)
    E = len(gate_blocks)
    F, nbh, bw = np.asarray(gate_blocks[0]).shape
    H = nbh * BLK
    Hd, nbf, _ = np.asarray(down_blocks[0]).shape
    if Hd != H or nbf * BLK != F:
        raise ValueError("down must be [H, F] for gate/up [F, H]")
    gu_bytes = packed_bytes(2 * F, H)
    dn_bytes = packed_bytes(H, F)
    gu = torch.empty(E * gu_bytes, dtype=torch.uint8, device=dev)
    dn = torch.empty(E * dn_bytes, dtype=torch.uint8, device=dev)
    for e in range(E):
        g = np.asarray(gate_blocks[e]).reshape(F // ROWS, ROWS, nbh, bw)
        u = np.asarray(up_blocks[e]).reshape(F // ROWS, ROWS, nbh, bw)
        inter = np.stack([g, u], axis=1).reshape(2 * F, nbh, bw)
        pack_q4_1(inter, dev, out=gu[e * gu_bytes:(e + 1) * gu_bytes])
        pack_q4_1(np.asarray(down_blocks[e]), dev, out=dn[e * dn_bytes:(e + 1) * dn_bytes])
    return PackedExperts(gu, E, 2 * F, H), PackedExperts(dn, E, H, F)


MOE_DECODE_MAX_PAIRS = 4096        # T * topk the decode kernels take (q4_moe_gemv)


def moe_batch(gate_up: PackedExperts, down: PackedExperts, x, topk_ids, topk_w,
              out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
              residual: torch.Tensor | None = None, shared: torch.Tensor | None = None,
              shared_gate_w=None, path: str = "auto", precision: str = "fp16",
              h_bf16: bool | None = None, shared_expert: tuple | None = None) -> torch.Tensor:
    """out[t] = sum_j w[t,j] * down_e(silu(gate_e x_t) * (up_e x_t)), e = ids[t,j]; fp32 h,
    fp32 out [T, H] (moe_batch.py's per-slot product plus core.cpp:5150-5245's
    gather/scatter, done on the device).

    With ``residual`` (f32 [T, H], may be ``out``) and/or ``shared`` (the shared expert's
    f32 [T, H] output) with ``shared_gate_w`` (sgw, [H], rounded to bf16 if given wider),
    the block's finish is folded into the combine, as moe_fin does
    (designs/moe_combine/moe_fin.py:1-4): out = (residual + routed sum) + sigmoid(x . sgw) * shared.

    ``path``: "decode" (q4_moe_gemv: routed-expert GEMVs, T * topk <= 4096), "prefill"
    (q4_moe_prefill: the experts' tokens batched into 256-token tiles of the prefill GEMM,
    any T; ``precision`` "fp16" or "bf16" as gemm_q4_prefill, h rounded to bf16 in "bf16" as
    the reference's moe_batch does, and in "fp16" too unless ``h_bf16=False``), or "auto"
    (decode up to 4096 pairs, then prefill). The prefill path takes no residual / shared
    expert.

    ``shared_expert`` = (gate_up_s, down_s): the block's shared expert as weights, run inside
    the same expert launches (decode path, q4_moe_gemv_shared): gate_up_s the interleaved
    [2 Fs, H] matrix (interleave_gate_up of its gate and up), down_s [H, Fs]; with
    ``shared_gate_w`` it adds sigmoid(x . sgw) * down_s(silu(gate_s x) * (up_s x)) (fp32 h),
    the replica's moe_decode (replica.py:131-144) and the reference's one-dispatch block
    (designs/moe_experts/moe_experts.py:1-13). Takes the place of ``shared``.

    ``h_bf16`` (prefill path): None, the default, rounds h to bf16, the reference kernel's
    own h (moe_batch.h:181-202): down then takes one pass over h, and the gate/up GEMM forms h
    in its epilogue (T = 2048 at config 4's experts: 422 us against 690 us for f32 h). False
    keeps h in fp32 (value and fp16 remainder, two down passes), the decode kernels' h and
    the model replica's (replica.py:139-144), for a caller that wants the same h on both sides
    of the 4096-pair switch."""
    dev = gate_up.data.device
    xt = _acts(x, dev)
    if xt.dim() == 1:
        xt = xt.unsqueeze(0)
    T, H = xt.shape
    F = gate_up.n // 2
    E = gate_up.experts
    if H != gate_up.k or down.n != H or down.k != F or down.experts != E:
        raise ValueError("expert shapes do not match x")
    ids = _to_dev(topk_ids, dev, torch.int32)
    wts = _to_dev(topk_w, dev, torch.float32)
    if ids.dim() == 1:
        ids, wts = ids.unsqueeze(0), wts.unsqueeze(0)
    if ids.shape[0] != T or ids.shape != wts.shape:
        raise ValueError("topk_ids / topk_w must be [T, topk]")
    topk = ids.shape[1]
    out = _buf(out, "out", torch.float32, (T, H), dev)
    if shared_expert is not None:
        if shared is not None:
            raise ValueError("give the shared expert as its output (shared) or as weights (shared_expert), not both")
        if shared_gate_w is None:
            raise ValueError("shared_expert needs shared_gate_w")
        sgu, sdn = shared_expert
        if not isinstance(sgu, PackedQ4) or not isinstance(sdn, PackedQ4):
            raise TypeError("shared_expert must be (PackedQ4 gate_up [2 Fs, H], PackedQ4 down [H, Fs])")
        if sgu.k != H or sgu.n % 128 or sdn.n != H or sdn.k != sgu.n // 2:
            raise ValueError(f"shared expert shapes {sgu.shape}, {sdn.shape} do not fit H={H}")
        if sgu.device != dev or sdn.device != dev:
            raise ValueError(f"the shared expert's weights must be on {dev}")
    elif (shared is None) != (shared_gate_w is None):
        raise ValueError("shared and shared_gate_w go together")
    for name, t_ in (("residual", residual), ("shared", shared)):
        if t_ is not None and (t_.dtype != torch.float32 or not t_.is_contiguous() or t_.numel() != T * H
                               or t_.device != dev):
            raise ValueError(f"{name} must be a contiguous float32 [{T}, {H}] tensor on {dev}")
    sgw = None
    if shared_gate_w is not None:
        sgw = _to_dev(shared_gate_w, dev)
        if sgw.dtype != torch.bfloat16:
            sgw = sgw.to(torch.float32).to(torch.bfloat16)
        sgw = sgw.contiguous().reshape(-1)
        if sgw.numel() != H:
            raise ValueError(f"shared_gate_w must have {H} values, got {sgw.numel()}")
    if path not in ("auto", "decode", "prefill"):
        raise ValueError(f"path must be 'auto', 'decode' or 'prefill', got {path!r}")
    if path == "auto":
        path = "decode" if T * topk <= MOE_DECODE_MAX_PAIRS else "prefill"
    lib = _lib_handle()
    if path == "prefill":
        if residual is not None or shared is not None or shared_expert is not None:
            raise ValueError("the prefill MoE path takes no residual or shared expert")
        if precision not in _PRECISION:
            raise ValueError(f"precision must be one of {sorted(_PRECISION)}, got {precision!r}")
        if T == 0:
            return out
        sc = (prefill_scales(gate_up), prefill_scales(down)) if precision == "fp16" else (None, None)
        with torch.cuda.device(dev):
            wp, wn = _ws_arg(dev, lib.q4_moe_prefill_workspace_bytes(T, E, topk, H, F), "moe_prefill", workspace)
            check("q4_moe_prefill", lib.q4_moe_prefill(
                _ptr(gate_up.data), _ptr(down.data), None if sc[0] is None else _ptr(sc[0]),
                None if sc[1] is None else _ptr(sc[1]), _ptr(xt), _x_dtype(xt), _ptr(ids), _ptr(wts), _ptr(out),
                T, E, topk, H, F, 2 if (precision == "fp16" and h_bf16 is not False) else _PRECISION[precision], wp, wn,
                _stream(dev)))
        return out
    if shared_expert is not None:
        sgu, sdn = shared_expert
        Fs = sgu.n // 2
        with torch.cuda.device(dev):
            wp, wn = _ws_arg(dev, lib.q4_moe_shared_workspace_bytes(T, E, topk, H, F, Fs), "moe", workspace)
            check("q4_moe_gemv_shared", lib.q4_moe_gemv_shared(
                _ptr(gate_up.data), _ptr(down.data), _ptr(sgu.data), _ptr(sdn.data), Fs, _ptr(sgw), _ptr(xt),
                _x_dtype(xt), _ptr(ids), _ptr(wts), None if residual is None else _ptr(residual), _ptr(out),
                T, E, topk, H, F, wp, wn, _stream(dev)))
        return out
    with torch.cuda.device(dev):
        wp, wn = _ws_arg(dev, lib.q4_moe_workspace_bytes(T, E, topk, H, F), "moe", workspace)
        if residual is None and shared is None:
            check("q4_moe_gemv", lib.q4_moe_gemv(
                _ptr(gate_up.data), _ptr(down.data), _ptr(xt), _x_dtype(xt), _ptr(ids), _ptr(wts), _ptr(out),
                T, E, topk, H, F, wp, wn, _stream(dev)))
        else:
            check("q4_moe_gemv_fin", lib.q4_moe_gemv_fin(
                _ptr(gate_up.data), _ptr(down.data), _ptr(xt), _x_dtype(xt), _ptr(ids), _ptr(wts),
                None if residual is None else _ptr(residual), None if shared is None else _ptr(shared),
                None if sgw is None else _ptr(sgw), _ptr(out), T, E, topk, H, F, wp, wn, _stream(dev)))
    return out
