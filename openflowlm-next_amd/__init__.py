"""openflowlm-next_amd -- MI355X (gfx950) Q4_1 dequant-matmul kernels.

The hot path of OpenFlowLM (the q4_1 dequantize-and-multiply behind every
projection and FFN matmul) as hand-written HIP kernels behind a C ABI
(``include/q4mi.h``, ``libq4mi.so``), with the reference's Python-facing
operator surface on top (packed Q4_1 in, bf16/fp32 activations in, fp32 out).

Import with ``importlib.import_module("openflowlm-next_amd")`` (the directory
name is not a Python identifier).
"""
from . import _lib
from .q4 import (GemvGroup, PackedExperts, PackedQ4, PackedQ4K, PackedQ8, dequant, dequant_q4k, gemm_q4, gemm_q4k,
                 gemm_q4_prefill, gemm_q8, gemv_q4, pack_q4_k_native, pack_q4_k_chunks_native, q4k_packed_bytes,
                 PackedQ8N, pack_q8_native, dequant_q8_native, gemm_q8_native,
                 PackedQ40, pack_q4_0_native, dequant_q4_0_native, gemm_q4_0_native,
                 gemv_workspace_bytes, lm_head_topk, logits_topk, moe_batch, pack_chunks, gemm_q4_rmsnorm, gemm_q4_rmsnorm_acc, gemm_q4_partials, gemv_split_count, swiglu_q4_acc, PreparedActs, prefill_prepare, rmsnorm_prepare, swiglu_prepare, interleave_gate_up, gemm_q4_prefill_swiglu, gemm_q4_prefill_partials, moe_workspace_bytes, moe_shared_workspace_bytes, moe_prefill_workspace_bytes, MOE_DECODE_MAX_PAIRS, pack_moe_experts, pack_q4_1,
                 pack_q4_1_pool, pack_q4_k, pack_q4_k_chunks, pack_q8, packed_bytes, prefill_scales, prefill_workspace_bytes,
                 rmsnorm_add, swiglu_q4, decode_segment, decode_segment_splits, decode_segment_workspace)
from .gguf import GGUFError, GGUFFile
from .q4nx import Q4NXError, Q4NXFile

__all__ = [
    "PackedQ4", "PackedQ4K", "PackedQ8", "PackedExperts", "pack_q4_k_native", "pack_q4_k_chunks_native",
    "dequant_q4k", "gemm_q4k", "q4k_packed_bytes", "PackedQ8N", "pack_q8_native", "dequant_q8_native",
    "gemm_q8_native", "PackedQ40", "pack_q4_0_native", "dequant_q4_0_native", "gemm_q4_0_native",
    "packed_bytes", "pack_q8", "gemm_q8", "pack_q4_1", "pack_q4_1_pool", "pack_q4_k",
    "pack_q4_k_chunks", "pack_chunks", "GGUFFile", "GGUFError", "Q4NXFile", "Q4NXError", "dequant",
    "gemv_q4", "gemm_q4", "gemm_q4_prefill", "lm_head_topk", "logits_topk", "swiglu_q4", "rmsnorm_add", "moe_batch", "pack_moe_experts", "GemvGroup",
    "gemv_workspace_bytes", "prefill_workspace_bytes", "prefill_scales", "gemm_q4_rmsnorm", "gemm_q4_rmsnorm_acc", "gemm_q4_partials", "gemv_split_count", "swiglu_q4_acc", "PreparedActs", "prefill_prepare", "rmsnorm_prepare", "swiglu_prepare", "interleave_gate_up", "gemm_q4_prefill_swiglu", "gemm_q4_prefill_partials", "moe_workspace_bytes", "moe_shared_workspace_bytes", "moe_prefill_workspace_bytes", "MOE_DECODE_MAX_PAIRS",
    "decode_segment", "decode_segment_splits", "decode_segment_workspace",
    "load_library",
]


def load_library():
    """Load libq4mi.so (raises ImportError when it was never built)."""
    return _lib.load()
