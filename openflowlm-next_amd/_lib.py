"""ctypes binding of libq4mi.so (the C ABI declared in include/q4mi.h).

The library is built in-tree by ``build.py``; loading fails loudly when it is
missing -- there is no CPU fallback for any operator.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("Q4MI_LIB", HERE / "libq4mi.so"))

Q4MI_OK = 0
Q4MI_F32 = 0
Q4MI_BF16 = 1

_vp, _i32, _i64, _sz = C.c_void_p, C.c_int, C.c_int64, C.c_size_t


class Q4GemvDesc(C.Structure):
    """Mirror of struct q4_gemv_desc (include/q4mi.h)."""
    _fields_ = [("packed", _vp), ("x", _vp), ("y", _vp),
                ("N", _i64), ("K", _i64), ("item_begin", _i64)]


# name -> (restype, argtypes); every function declared in include/q4mi.h
SIGNATURES = {
    "q4mi_version": (_i32, []),
    "q4_decode_segment_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "q4_decode_segment_splits": (_i32, [_i64, _i64, _i64, _vp]),
    "q4_decode_segment": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, C.c_float, _vp, _vp, _vp, _vp,
                                 _i64, _i64, _i64, _vp, _sz, _vp]),
    "q4_dequant_fp16s": (_i32, [_vp, _vp, _i64, _i64, _vp]),
    "q4_gemv_fp16s": (_i32, [_vp, _vp, _i32, _vp, _vp, _i32, _i64, _i64, _vp, _sz, _vp]),
    "q4_gemv_grouped_fp16s": (_i32, [_vp, _i32, _i64, _i32, _i32, _vp]),
    "q4_moe_shared_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "q4_moe_gemv_shared": (_i32, [_vp, _vp, _vp, _vp, _i64, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _i32, _i32, _i32,
                                  _i64, _i64, _vp, _sz, _vp]),
    "q4_probe_stream_read_out_bytes": (_sz, [_i32]),
    "q4_probe_stream_read": (_i32, [_vp, _sz, _i32, _vp, _vp]),
    "q4_probe_mfma": (_i32, [_i32, _i32, _vp, _vp, _vp]),
    "q4mi_strerror": (C.c_char_p, [_i32]),
    "q4_packed_bytes": (_i64, [_i64, _i64]),
    "q4_repack": (_i32, [_vp, _i32, _vp, _i64, _i64, _i32, _vp]),
    "q4_repack_pool": (_i32, [_vp, _i32, _vp, _i64, _i64, _vp]),
    "q4_repack_pool_f32": (_i32, [_vp, _i32, _vp, _i64, _i64, _vp]),
    "q4_repack_q4k": (_i32, [_vp, _vp, _i64, _i64, _vp]),
    "q4_repack_q4k_chunks": (_i32, [_vp, _i32, _vp, _i64, _i64, _vp]),
    "q4_q4k_packed_bytes": (_i64, [_i64, _i64]),
    "q4_repack_q4k_native": (_i32, [_vp, _vp, _i64, _i64, _vp]),
    "q4_repack_q4k_chunks_native": (_i32, [_vp, _i32, _vp, _i64, _i64, _vp]),
    "q4_dequant_q4k": (_i32, [_vp, _vp, _i64, _i64, _vp]),
    "q4_gemv_q4k_workspace_bytes": (_sz, [_i32, _i64, _i64]),
    "q4_gemv_q4k": (_i32, [_vp, _vp, _i32, _vp, _vp, _i32, _i64, _i64, _vp, _sz, _vp]),
    "q4_q8_native_packed_bytes": (_i64, [_i64, _i64]),
    "q4_repack_q8_native": (_i32, [_vp, _i32, _i32, _vp, _i64, _i64, _vp]),
    "q4_dequant_q8_native": (_i32, [_vp, _vp, _i64, _i64, _vp]),
    "q4_q40_packed_bytes": (_i64, [_i64, _i64]),
    "q4_repack_q40": (_i32, [_vp, _i32, _i32, _vp, _i64, _i64, _vp]),
    "q4_dequant_q40": (_i32, [_vp, _vp, _i64, _i64, _vp]),
    "q4_gemv_q40": (_i32, [_vp, _vp, _i32, _vp, _vp, _i32, _i64, _i64, _vp, _sz, _vp]),
    "q4_gemv_q8_native_workspace_bytes": (_sz, [_i32, _i64, _i64]),
    "q4_gemv_q8_native": (_i32, [_vp, _vp, _i32, _vp, _vp, _i32, _i64, _i64, _vp, _sz, _vp]),
    "q4_repack_pool_signed": (_i32, [_vp, _i32, _vp, _i64, _i64, _vp]),
    "q4_repack_q8_chunks": (_i32, [_vp, _i32, _vp, _i64, _i64, _vp]),
    "q4_repack_q8_split": (_i32, [_vp, _i32, _i32, _i32, _vp, _i64, _i64, _vp]),
    "q4_gemv_q8": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _i64, _i64, _vp, _sz, _vp]),
    "q4_dequant": (_i32, [_vp, _vp, _i64, _i64, _vp]),
    "q4_gemv_workspace_bytes": (_sz, [_i32, _i64, _i64]),
    "q4_gemv_rmsnorm_workspace_bytes": (_sz, [_i32, _i64, _i64]),
    "q4_gemv": (_i32, [_vp, _vp, _i32, _vp, _i32, _i64, _i64, _vp, _sz, _vp]),
    "q4_gemv_noalloc": (_i32, [_vp, _vp, _i32, _vp, _i32, _i64, _i64, _vp]),
    "q4_gemv_grouped": (_i32, [_vp, _i32, _i64, _i32, _i32, _vp]),
    "q4_gemv_residual": (_i32, [_vp, _vp, _i32, _vp, _vp, _i32, _i64, _i64, _vp, _sz, _vp]),
    "q4_gemv_rmsnorm": (_i32, [_vp, _vp, _vp, _i32, C.c_float, _vp, _i32, _i64, _i64, _vp, _sz, _vp]),
    "q4_gemv_swiglu_rmsnorm": (_i32, [_vp, _vp, _vp, _vp, _i32, C.c_float, _vp, _i32, _i32, _i64, _i64, _vp, _sz,
                                      _vp]),
    "q4_gemv_split_count": (_i32, [_i64, _i64]),
    "q4_gemv_partials": (_i32, [_vp, _vp, _i32, _vp, _i32, _i32, _i64, _i64, _vp]),
    "q4_gemv_rmsnorm_acc": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, C.c_float, _vp, _vp, _i32, _i64, _i64, _vp, _sz,
                                   _vp]),
    "q4_gemv_swiglu_rmsnorm_acc": (_i32, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, C.c_float, _vp, _vp, _i32, _i32,
                                          _i64, _i64, _vp, _sz, _vp]),
    "q4_gemv_swiglu_workspace_bytes": (_sz, [_i32, _i64, _i64]),
    "q4_gemv_swiglu": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _i32, _i64, _i64, _vp, _sz, _vp]),
    "q4_rmsnorm_add": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i64, C.c_float, _vp]),
    "q4_gemm_prefill_workspace_bytes": (_sz, [_i32, _i64, _i64]),
    "q4_gemm_prefill": (_i32, [_vp, _vp, _i32, _vp, _i32, _i64, _i64, _i32, _vp, _sz, _vp]),
    "q4_prefill_scales_bytes": (_sz, [_i64, _i64]),
    "q4_prefill_scales": (_i32, [_vp, _i64, _i64, _vp, _sz, _vp]),
    "q4_gemm_prefill_scaled_workspace_bytes": (_sz, [_i32, _i64, _i64]),
    "q4_gemm_prefill_scaled": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _i64, _i64, _vp, _sz, _vp]),
    "q4_topk_workspace_bytes": (_sz, [_i32, _i64, _i32]),
    "q4_logits_topk": (_i32, [_vp, _i64, _i32, _i64, _i32, _i32, _vp, _vp, _vp, _sz, _vp]),
    "q4_lm_head_workspace_bytes": (_sz, [_i32, _i64, _i64, _i32]),
    "q4_lm_head_topk": (_i32, [_vp, _vp, _i32, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _sz,
                               _vp]),
    "q4_prefill_prepared_bytes": (_sz, [_i32, _i64, _i32, _i32]),
    "q4_prefill_prepare": (_i32, [_vp, _i32, _i32, _i64, _i32, _vp, _sz, _vp]),
    "q4_gemm_prefill_swiglu": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _i64, _i64, _i32, _vp]),
    "q4_swiglu_prepare": (_i32, [_vp, _vp, _i64, _i64, _i32, _i64, _i32, _vp, _vp, _sz, _vp]),
    "q4_rmsnorm_prepare": (_i32, [_vp, _vp, _i32, _vp, _i32, _vp, _i32, _i64, C.c_float, _i32, _vp, _sz, _vp]),
    "q4_prefill_split_count": (_i32, [_i32, _i64, _i64]),
    "q4_gemm_prefill_prepared_partials": (_i32, [_vp, _vp, _vp, _i32, _vp, _sz, _i32, _i64, _i64, _i32, _vp]),
    "q4_gemm_prefill_prepared_workspace_bytes": (_sz, [_i32, _i64, _i64]),
    "q4_gemm_prefill_prepared": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _i64, _i64, _i32, _vp, _sz, _vp]),
    "q4_moe_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "q4_moe_prefill_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "q4_moe_prefill": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _i32, _i32, _i32, _i64, _i64, _i32, _vp,
                              _sz, _vp]),
    "q4_moe_gemv": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _vp, _i32, _i32, _i32, _i64, _i64, _vp, _sz, _vp]),
    "q4_moe_gemv_fin": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i64, _i64, _vp,
                               _sz, _vp]),
}

_LIB = None


class Q4Error(RuntimeError):
    def __init__(self, fn: str, status: int):
        self.status = status
        super().__init__(f"{fn} failed: status {status} ({strerror(status)})")


def load(path: Path | None = None) -> C.CDLL:
    """Load libq4mi.so once (raises if it was never built)."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.is_file():
        raise ImportError(f"{p} is missing: build it with `python openflowlm-next_amd/build.py` "
                          "(there is no CPU fallback)")
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def strerror(status: int) -> str:
    try:
        return load().q4mi_strerror(status).decode()
    except Exception:  # pragma: no cover - only when the library itself is unusable
        return "?"


def check(fn: str, status: int) -> None:
    if status != Q4MI_OK:
        raise Q4Error(fn, status)
