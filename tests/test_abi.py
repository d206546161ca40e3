"""The C ABI: libq4mi.so loads on a CPU-only host, exports every function
include/q4mi.h declares, and rejects bad arguments before touching the GPU."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "q4mi.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if n not in ("if", "defined")))


def test_header_declares_the_expected_surface():
    names = declared_functions()
    for must in ("q4_packed_bytes", "q4_repack", "q4_repack_pool", "q4_repack_q4k", "q4_repack_q4k_chunks",
                 "q4_repack_pool_signed", "q4_repack_q8_chunks", "q4_repack_q8_split", "q4_gemv_q8", "q4_repack_pool_f32",
                 "q4_dequant", "q4_gemv", "q4_gemv_grouped", "q4_gemm_prefill", "q4_moe_gemv",
                 "q4_logits_topk", "q4_lm_head_topk", "q4_gemv_residual", "q4_gemv_swiglu", "q4_rmsnorm_add"):
        assert must in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared in q4mi.h but not exported: {missing}"


def test_python_binding_covers_the_header(pkg):
    from importlib import import_module
    sigs = import_module("openflowlm-next_amd._lib").SIGNATURES
    assert set(declared_functions()) <= set(sigs)


def test_version_and_strerror(lib):
    assert lib.q4mi_version() >= 100
    for code in (0, -1, -2, -3, -4, -5):
        assert lib.q4mi_strerror(code)
    assert lib.q4mi_strerror(-99) == b"unknown status"


@pytest.mark.parametrize("n,k,want", [(64, 32, 1280), (4096, 4096, 4096 * 4096 * 5 // 8),
                                      (128256, 4096, 128256 * 4096 * 5 // 8), (0, 32, 0),
                                      (63, 32, -1), (64, 48, -1), (-64, 32, -1), (64, 0, -1)])
def test_packed_bytes(lib, n, k, want):
    assert lib.q4_packed_bytes(n, k) == want


def test_argument_errors_before_any_launch(lib):
    """Every one of these returns before a HIP call (no GPU needed)."""
    fake = C.c_void_p(0x1000)   # never dereferenced: each call fails validation first
    assert lib.q4_repack(fake, 19, fake, 64, 32, 0, None) == -2          # block width
    assert lib.q4_repack(fake, 20, fake, 64, 32, 2, None) == -2          # scale mode
    assert lib.q4_repack(fake, 18, fake, 64, 32, 1, None) == -2          # fp16 scales: Q4_1 only
    assert lib.q4_dequant_fp16s(fake, None, 64, 32, None) == -2
    assert lib.q4_gemv_fp16s(fake, fake, 1, None, fake, 17, 64, 32, None, 0, None) == -5   # M > 16
    assert lib.q4_gemv_fp16s(fake, fake, 1, None, fake, 1, 1024, 4096, None, 0, None) == -3   # split: workspace
    assert lib.q4_gemv_grouped_fp16s(None, 1, 1, 1, 1, None) == -2
    assert lib.q4_repack(None, 20, fake, 64, 32, 0, None) == -2          # NULL
    assert lib.q4_repack(fake, 20, fake, 96, 32, 0, None) == -1          # N % 64
    assert lib.q4_repack(fake, 20, fake, 64, 40, 0, None) == -1          # K % 32
    assert lib.q4_repack(None, 20, None, 0, 32, 0, None) == 0            # empty is a no-op
    assert lib.q4_repack_pool(fake, 2, fake, 64, 128, None) == -1        # K % 256
    assert lib.q4_repack_pool(fake, 0, fake, 64, 256, None) == -2        # rs
    assert lib.q4_repack_pool(fake, 4, fake, 64, 256, None) == -1        # N % (32 rs)
    assert lib.q4_repack_q4k(fake, fake, 64, 128, None) == -1            # K % 256
    assert lib.q4_repack_q4k(fake, fake, 32, 256, None) == -1            # N % 64
    assert lib.q4_repack_q4k(None, fake, 64, 256, None) == -2            # NULL
    assert lib.q4_repack_q4k(None, None, 0, 256, None) == 0              # empty is a no-op
    assert lib.q4_repack_q4k_chunks(fake, 1, fake, 64, 128, None) == -1  # K % 256
    assert lib.q4_repack_q4k_chunks(fake, 0, fake, 64, 256, None) == -2  # rs
    assert lib.q4_repack_q4k_chunks(fake, 4, fake, 64, 256, None) == -1  # N % (32 rs)
    assert lib.q4_repack_q8_split(fake, 3, 1, 0, fake, 64, 256, None) == -2   # source format
    assert lib.q4_repack_q40(fake, 2, 1, fake, 64, 256, None) == -2          # source format
    assert lib.q4_repack_q40(fake, 1, 0, fake, 64, 256, None) == -2          # chunks: rs
    assert lib.q4_repack_q40(fake, 1, 1, fake, 64, 128, None) == -1          # chunks: K % 256
    assert lib.q4_repack_q40(fake, 0, 1, fake, 96, 32, None) == -1           # N % 64
    assert lib.q4_repack_q40(None, 0, 1, None, 0, 32, None) == 0             # empty is a no-op
    assert lib.q4_q40_packed_bytes(64, 32) == 1152 and lib.q4_q40_packed_bytes(96, 32) < 0
    assert lib.q4_gemv_q40(fake, fake, 1, None, fake, 17, 64, 32, None, 0, None) == -5   # M > 16
    assert lib.q4_dequant_q40(fake, None, 64, 32, None) == -2
    assert lib.q4_repack_pool_f32(fake, 1, fake, 64, 128, None) == -1          # K % 256
    assert lib.q4_repack_pool_f32(C.c_void_p(0x1002), 1, fake, 64, 256, None) == -2   # f32 scales misaligned
    assert lib.q4_repack_q8_split(fake, 0, 1, 2, fake, 64, 256, None) == -2   # part
    assert lib.q4_repack_q8_split(fake, 0, 1, 0, fake, 64, 128, None) == -1   # chunks need K % 256
    assert lib.q4_repack_q8_split(fake, 1, 1, 0, fake, 64, 48, None) == -1    # Q8_0 needs K % 32
    assert lib.q4_gemv_q8(fake, None, fake, 1, None, fake, 1, 64, 32, None, 0, None) == -2   # no lo plane
    for fn in (lib.q4_repack_pool_signed, lib.q4_repack_q8_chunks):
        assert fn(fake, 1, fake, 64, 128, None) == -1                    # K % 256
        assert fn(fake, 0, fake, 64, 256, None) == -2                    # rs
        assert fn(None, 1, fake, 64, 256, None) == -2                    # NULL
        assert fn(None, 1, None, 0, 256, None) == 0                      # empty
    assert lib.q4_dequant(fake, None, 64, 32, None) == -2
    assert lib.q4_dequant(None, None, 0, 32, None) == 0
    assert lib.q4_gemv(fake, fake, 2, fake, 1, 64, 32, None, 0, None) == -2    # dtype
    assert lib.q4_gemv(fake, fake, 1, fake, 25, 64, 32, None, 0, None) == -5   # M > 24
    assert lib.q4_gemv_q8(fake, fake, fake, 1, None, fake, 17, 64, 32, None, 0, None) == -5   # pair: M > 16
    assert lib.q4_gemv_noalloc(fake, fake, 1, fake, 17, 64, 32, None) == -5     # no-alloc: M > 16
    assert lib.q4_gemv(fake, fake, 1, fake, 1, 100, 32, None, 0, None) == -1   # N % 64
    assert lib.q4_gemv(None, None, 1, None, 0, 64, 32, None, 0, None) == 0     # M = 0
    # a short matrix is split along K and needs the workspace the query reports
    for n in (1024, 4096):
        need = lib.q4_gemv_workspace_bytes(1, n, 4096)
        assert need > 0 and lib.q4_gemv_split_count(n, 4096) > 1
        assert lib.q4_gemv(fake, fake, 1, fake, 1, n, 4096, None, 0, None) == -3
        assert lib.q4_gemv(fake, fake, 1, fake, 1, n, 4096, fake, need - 1, None) == -3
    assert lib.q4_gemv_split_count(6144, 4096) == 1     # 96 row groups: unsplit, 16 waves
    assert lib.q4_gemv_grouped(None, 1, 1, 1, 1, None) == -2
    assert lib.q4_gemv_grouped(fake, 1, 1, 17, 1, None) == -5
    # packed weights, activations, outputs and workspaces move in 16-byte vectors
    odd = C.c_void_p(0x1004)
    assert lib.q4_gemv(fake, odd, 1, fake, 1, 128256, 4096, None, 0, None) == -2
    assert lib.q4_gemv(odd, fake, 1, fake, 1, 128256, 4096, None, 0, None) == -2
    assert lib.q4_dequant(fake, odd, 64, 32, None) == -2
    assert lib.q4_repack(fake, 20, odd, 64, 32, 0, None) == -2
    assert lib.q4_repack_q4k(fake, odd, 64, 256, None) == -2
    assert lib.q4_repack_q4k_chunks(fake, 1, odd, 64, 256, None) == -2
    need = lib.q4_gemm_prefill_workspace_bytes(64, 256, 1024)
    assert lib.q4_gemm_prefill(fake, fake, 1, odd, 64, 256, 1024, 0, fake, need, None) == -2
    assert lib.q4_gemm_prefill(fake, fake, 1, fake, 64, 256, 1024, 0, odd, need, None) == -2
    assert lib.q4_gemm_prefill(fake, fake, 1, fake, 64, 256, 1024, 0, fake, need - 1, None) == -3
    assert lib.q4_gemm_prefill(fake, fake, 1, fake, 64, 256, 1024, 2, fake, need, None) == -2
    assert lib.q4_gemm_prefill(fake, fake, 1, fake, 64, 100, 1024, 0, fake, need, None) == -1
    assert lib.q4_logits_topk(fake, 10, 1, 10, 65, 1, fake, None, None, 0, None) == -5   # k > 64
    assert lib.q4_logits_topk(fake, 10, 1, 10, 0, 1, fake, None, None, 0, None) == -5    # k < 1
    assert lib.q4_logits_topk(fake, 10, 1, 10, 1, 2, fake, None, None, 0, None) == -5    # mode
    assert lib.q4_logits_topk(fake, 5, 1, 10, 1, 1, fake, None, None, 0, None) == -1     # ld < n
    assert lib.q4_logits_topk(None, 10, 1, 10, 1, 1, fake, None, None, 0, None) == -2    # NULL
    assert lib.q4_logits_topk(None, 10, 0, 10, 1, 1, None, None, None, 0, None) == 0     # M = 0
    need = lib.q4_topk_workspace_bytes(2, 128256, 40)
    assert need >= 2 * 32 * 40 * 8
    assert lib.q4_logits_topk(fake, 128256, 2, 128256, 40, 1, fake, None, fake, need - 1, None) == -3
    assert lib.q4_topk_workspace_bytes(1, 1024, 64) == 0          # one block per token: none
    assert lib.q4_lm_head_topk(fake, fake, 1, fake, 1, 128256, 4096, 128257, 1, 1, fake, None, None, 0,
                               None) == -1                        # n_valid > N
    assert lib.q4_gemv_residual(fake, fake, 1, None, fake, 1, 64, 32, None, 0, None) == -2  # no residual
    assert lib.q4_gemv_swiglu(fake, fake, fake, 1, fake, 2, 1, 64, 32, None, 0, None) == -2  # h dtype
    assert lib.q4_gemv_swiglu(fake, fake, fake, 1, fake, 1, 17, 64, 32, None, 0, None) == -5  # M > 16
    assert lib.q4_gemv_swiglu(fake, fake, fake, 1, fake, 1, 1, 100, 32, None, 0, None) == -1  # F % 64
    assert lib.q4_gemv_swiglu(fake, odd, fake, 1, fake, 1, 1, 64, 32, None, 0, None) == -2   # misaligned up
    sw = lib.q4_gemv_swiglu_workspace_bytes(1, 512, 4096)
    assert sw > 0 and lib.q4_gemv_swiglu(fake, fake, fake, 1, fake, 1, 1, 512, 4096, fake, sw - 1, None) == -3
    assert lib.q4_gemv_swiglu_workspace_bytes(1, 14336, 4096) == 0 or sw > 0
    assert lib.q4_rmsnorm_add(fake, None, fake, 3, None, fake, 1, 1, 64, 1e-6, None) == -2     # w dtype
    assert lib.q4_rmsnorm_add(fake, None, fake, 1, None, fake, 1, 1, 0, 1e-6, None) == -1      # N = 0
    assert lib.q4_rmsnorm_add(None, None, fake, 1, None, fake, 1, 1, 64, 1e-6, None) == -2     # NULL x
    assert lib.q4_rmsnorm_add(fake, None, fake, 1, None, fake, 1, 1, 64, -1.0, None) == -2     # eps < 0
    wsm = lib.q4_moe_workspace_bytes(16, 128, 8, 2048, 768)
    assert lib.q4_moe_gemv(fake, fake, odd, 1, fake, fake, fake, 16, 128, 8, 2048, 768, fake, wsm, None) == -2


def test_prefill_workspace_query(lib):
    """Activations in the kernel's layout (zero-padded to 256-token tiles) + per-token
    exponents, plus K-split partials when a grid of 256x256 tiles cannot fill the GPU."""
    x_only = lambda T, K: -(-((T + 255) // 256 * 256 * K * 2) // 256) * 256 + -(-(T * 4) // 256) * 256
    assert lib.q4_gemm_prefill_workspace_bytes(2048, 14336, 4096) >= x_only(2048, 4096)
    # 16 x 2 output tiles for 224 stages of K: split, partials [S][T][N] f32
    assert lib.q4_gemm_prefill_workspace_bytes(512, 4096, 14336) >= x_only(512, 14336) + 2 * 512 * 4096 * 4
    assert lib.q4_gemm_prefill_workspace_bytes(0, 4096, 4096) == 0
    assert lib.q4_gemm_prefill_workspace_bytes(64, 100, 4096) == 0
    # the per-call path also holds the matrix's prefill scales: exponents, the fp16 plane
    # (4 bytes per row and 32-K block) and the per-chunk maxima
    sc = lib.q4_prefill_scales_bytes(14336, 4096)
    assert sc >= 14336 * 4 + 14336 * 128 * 4
    assert lib.q4_gemm_prefill_workspace_bytes(2048, 14336, 4096) == \
        lib.q4_gemm_prefill_scaled_workspace_bytes(2048, 14336, 4096) + sc
    assert lib.q4_prefill_scales_bytes(100, 4096) == 0 and lib.q4_prefill_scales_bytes(64, 48) == 0


def test_prefill_scales_argument_errors(lib):
    fake, odd = C.c_void_p(0x1000), C.c_void_p(0x1004)
    need = lib.q4_prefill_scales_bytes(256, 1024)
    assert lib.q4_prefill_scales(fake, 100, 1024, fake, need, None) == -1       # N % 64
    assert lib.q4_prefill_scales(fake, 256, 1024, odd, need, None) == -2        # misaligned
    assert lib.q4_prefill_scales(None, 256, 1024, fake, need, None) == -2       # NULL
    assert lib.q4_prefill_scales(fake, 256, 1024, fake, need - 1, None) == -3   # short
    assert lib.q4_prefill_scales(fake, 0, 1024, fake, 0, None) == 0             # nothing to do
    ws = lib.q4_gemm_prefill_scaled_workspace_bytes(64, 256, 1024)
    assert lib.q4_gemm_prefill_scaled(fake, None, fake, 1, fake, 64, 256, 1024, fake, ws, None) == -2
    assert lib.q4_gemm_prefill_scaled(fake, odd, fake, 1, fake, 64, 256, 1024, fake, ws, None) == -2
    assert lib.q4_gemm_prefill_scaled(fake, fake, fake, 1, fake, 64, 256, 1024, fake, ws - 1, None) == -3
    assert lib.q4_gemm_prefill_scaled(fake, fake, fake, 5, fake, 64, 256, 1024, fake, ws, None) == -2
    assert lib.q4_gemm_prefill_scaled(fake, fake, fake, 1, fake, 0, 256, 1024, None, 0, None) == 0


def test_gemv_workspace_query(lib):
    assert lib.q4_gemv_workspace_bytes(1, 128256, 4096) == 0     # enough row groups: no split
    assert lib.q4_gemv_workspace_bytes(16, 4096, 14336) >= 16 * 4096 * 4 * 2
    assert lib.q4_gemv_workspace_bytes(0, 64, 32) == 0
    # the norm GEMVs: room for the bf16 rows at vocabulary size (>= 1024 row groups), after
    # the split partials rounded up to 256 bytes; else q4_gemv's
    assert lib.q4_gemv_rmsnorm_workspace_bytes(1, 128256, 4096) == 4096 * 2
    assert lib.q4_gemv_rmsnorm_workspace_bytes(16, 65536, 2048) == 16 * 2048 * 2
    assert lib.q4_gemv_rmsnorm_workspace_bytes(1, 4096, 4096) == lib.q4_gemv_workspace_bytes(1, 4096, 4096)
    assert lib.q4_gemv_rmsnorm_workspace_bytes(3, 6144, 4096) == lib.q4_gemv_workspace_bytes(3, 6144, 4096)
    assert lib.q4_gemv_rmsnorm_workspace_bytes(0, 64, 32) == 0
    assert lib.q4_gemv_rmsnorm_workspace_bytes(1, 65536 + 64, 4008) == 0   # K % 32 != 0


def test_loader_fails_loudly_without_the_library(tmp_path):
    from importlib import import_module
    L = import_module("openflowlm-next_amd._lib")
    with pytest.raises(ImportError):
        L.load(tmp_path / "libq4mi.so")


def test_native_q4k_argument_errors(lib):
    """The native Q4_K entry points validate before any launch, like the others."""
    fake = C.c_void_p(0x1000)
    assert lib.q4_q4k_packed_bytes(64, 256) == 9728
    assert lib.q4_q4k_packed_bytes(64, 128) == -1 and lib.q4_q4k_packed_bytes(32, 256) == -1
    assert lib.q4_repack_q4k_native(fake, fake, 64, 128, None) == -1           # K % 256
    assert lib.q4_repack_q4k_native(None, fake, 64, 256, None) == -2           # NULL
    assert lib.q4_repack_q4k_native(None, None, 0, 256, None) == 0             # empty
    assert lib.q4_repack_q4k_chunks_native(fake, 0, fake, 64, 256, None) == -2 # rs
    assert lib.q4_repack_q4k_chunks_native(fake, 4, fake, 64, 256, None) == -1 # N % (32 rs)
    assert lib.q4_dequant_q4k(fake, C.c_void_p(0x1004), 64, 256, None) == -2   # misaligned
    assert lib.q4_gemv_q4k(fake, fake, 1, None, fake, 1, 64, 128, None, 0, None) == -1   # K % 256
    assert lib.q4_gemv_q4k(fake, fake, 1, None, fake, 17, 64, 256, None, 0, None) == -5  # M > 16
    assert lib.q4_gemv_q4k(fake, fake, 2, None, fake, 1, 64, 256, None, 0, None) == -2   # dtype
    need = lib.q4_gemv_q4k_workspace_bytes(1, 256, 14336)
    assert need > 0
    assert lib.q4_gemv_q4k(fake, fake, 1, None, fake, 1, 256, 14336, fake, need - 1, None) == -3
    assert lib.q4_gemv_q4k_workspace_bytes(1, 128256, 4096) == 0


def test_native_q8_argument_errors(lib):
    fake = C.c_void_p(0x1000)
    assert lib.q4_q8_native_packed_bytes(64, 32) == 2176
    assert lib.q4_q8_native_packed_bytes(64, 48) == -1
    assert lib.q4_repack_q8_native(fake, 3, 1, fake, 64, 256, None) == -2       # source format
    assert lib.q4_repack_q8_native(fake, 0, 1, fake, 64, 128, None) == -1       # chunks need K % 256
    assert lib.q4_repack_q8_native(fake, 1, 1, fake, 64, 48, None) == -1        # Q8_0 needs K % 32
    assert lib.q4_repack_q8_native(None, 1, 1, None, 0, 32, None) == 0          # empty
    assert lib.q4_gemv_q8_native(fake, fake, 1, None, fake, 17, 64, 32, None, 0, None) == -5
    assert lib.q4_gemv_q8_native(fake, fake, 1, None, fake, 1, 64, 48, None, 0, None) == -1
    need = lib.q4_gemv_q8_native_workspace_bytes(1, 1024, 4096)
    assert need > 0
    assert lib.q4_gemv_q8_native(fake, fake, 1, None, fake, 1, 1024, 4096, fake, need - 1, None) == -3


def test_moe_fin_argument_errors(lib):
    """q4_moe_gemv_fin refuses a shared expert without its gate weights (and the reverse),
    misaligned residual / shared pointers and a short workspace, all before any launch."""
    fake = C.c_void_p(0x1000)
    odd = C.c_void_p(0x1004)
    ws = lib.q4_moe_workspace_bytes(16, 128, 8, 2048, 768)
    args = lambda res, sh, sgw, wsb: (fake, fake, fake, 1, fake, fake, res, sh, sgw, fake, 16, 128, 8, 2048, 768,
                                      fake, wsb, None)
    assert lib.q4_moe_gemv_fin(*args(None, fake, None, ws)) == -2      # shared without sgw
    assert lib.q4_moe_gemv_fin(*args(None, None, fake, ws)) == -2      # sgw without shared
    assert lib.q4_moe_gemv_fin(*args(odd, None, None, ws)) == -2       # misaligned residual
    assert lib.q4_moe_gemv_fin(*args(None, odd, fake, ws)) == -2       # misaligned shared
    assert lib.q4_moe_gemv_fin(*args(fake, fake, fake, ws - 1)) == -3  # short workspace


def test_deferred_reduction_argument_errors(lib):
    """q4_gemv_partials / the _acc norm GEMVs refuse bad split counts and outputs that
    overlap what other workgroups still read, before any launch."""
    fake = C.c_void_p(0x1000)
    assert lib.q4_gemv_split_count(4096, 14336) >= 2 and lib.q4_gemv_split_count(128256, 4096) == 1
    assert lib.q4_gemv_split_count(100, 4096) == 0
    for S in (0, 17):
        assert lib.q4_gemv_partials(fake, fake, 1, fake, S, 1, 4096, 4096, None) == -5
    assert lib.q4_gemv_partials(fake, fake, 1, fake, 4, 1, 4096, 96, None) == -5     # S > K / 32
    assert lib.q4_gemv_partials(fake, fake, 1, fake, 4, 17, 4096, 4096, None) == -5  # M
    assert lib.q4_gemv_partials(fake, fake, 7, fake, 4, 1, 4096, 4096, None) == -2   # x dtype
    assert lib.q4_gemv_partials(fake, fake, 1, fake, 4, 1, 4100, 4096, None) == -1   # N % 64
    assert lib.q4_gemv_partials(fake, fake, 1, fake, 4, 0, 4096, 4096, None) == 0    # nothing to do
    K, N = 4096, 1024
    res, part, xo, y = (C.c_void_p(0x10000000 * i) for i in (1, 2, 3, 4))
    rms = lambda *a: lib.q4_gemv_rmsnorm_acc(fake, *a, None, 0, None)
    assert rms(res, part, 17, fake, 1, C.c_float(1e-6), xo, y, 1, N, K) == -5          # S
    assert rms(res, None, 4, fake, 1, C.c_float(1e-6), xo, y, 1, N, K) == -2           # no planes
    assert rms(res, part, 4, fake, 1, C.c_float(1e-6), None, y, 1, N, K) == -2         # no x_out
    over = C.c_void_p(0x10000000 + 4 * K - 16)
    assert rms(res, part, 4, fake, 1, C.c_float(1e-6), over, y, 1, N, K) == -2         # x_out on res
    assert rms(res, part, 4, fake, 1, C.c_float(1e-6), xo, C.c_void_p(0x20000000 + 3 * 4 * K), 1, N, K) == -2
    assert rms(res, part, 4, fake, 1, C.c_float(1e-6), xo, C.c_void_p(0x30000000 + 64), 1, N, K) == -2
    h = C.c_void_p(0x40000000)
    sw = lambda *a: lib.q4_gemv_swiglu_rmsnorm_acc(fake, fake, *a, None, 0, None)
    assert sw(res, part, 4, fake, 1, C.c_float(1e-6), xo, C.c_void_p(0x10000000), 1, 1, 14336, K) == -2  # h on res
    assert sw(res, part, -1, fake, 1, C.c_float(1e-6), xo, h, 1, 1, 14336, K) == -5


def test_split_workspace_must_not_overlap_what_the_gemv_reads(lib):
    """A split norm GEMV (1024 x 4096 at M = 1 plans K splits and reduces the deferred
    planes inside its workgroups) stores its partials to the workspace while other
    workgroups still read res and the planes: a workspace carved over the planes, res, x_out
    or y is refused before any launch."""
    K, N = 4096, 1024
    need = lib.q4_gemv_workspace_bytes(1, N, K)
    assert need > 0 and lib.q4_gemv_split_count(N, K) > 1
    fake = C.c_void_p(0x1000)
    res, part, xo, y = (C.c_void_p(0x10000000 * i) for i in (1, 2, 3, 4))
    eps = C.c_float(1e-6)
    rms = lambda ws: lib.q4_gemv_rmsnorm_acc(fake, res, part, 2, fake, 1, eps, xo, y, 1, N, K,
                                              ws, need, None)
    for base in (0x20000000 + 4 * K, 0x10000000, 0x30000000 - 16, 0x40000000 + 4 * N - 16):
        assert rms(C.c_void_p(base)) == -2, hex(base)
    assert lib.q4_gemv_rmsnorm_acc(fake, res, part, 2, fake, 1, eps, xo, y, 1, N, K, C.c_void_p(0x50000000),
                                   need - 16, None) == -3                           # short, checked first
    F, h = 1024, C.c_void_p(0x40000000)
    need_sw = lib.q4_gemv_swiglu_workspace_bytes(1, F, K)
    if need_sw:   # the SwiGLU form splits too at this shape: same rule over its planes
        sw = lambda ws: lib.q4_gemv_swiglu_rmsnorm_acc(fake, fake, res, part, 2, fake, 1, eps, xo, h, 1, 1, F,
                                                       K, ws, need_sw, None)
        assert sw(C.c_void_p(0x20000000)) == -2
        assert sw(C.c_void_p(0x30000000 + 4 * K - 16)) == -2


def test_rmsnorm_prepare_argument_errors(lib):
    """q4_rmsnorm_prepare refuses bad enums, shapes, sizes and overlapping outputs before any
    launch."""
    T, K = 256, 4096
    need = lib.q4_prefill_prepared_bytes(T, K, 1, 0)
    assert need > T * K * 2
    x, add, w, y, prep = (C.c_void_p(0x10000000 * i) for i in (1, 2, 3, 4, 5))
    call = lambda x_, add_, *a: lib.q4_rmsnorm_prepare(x_, add_, 0 if add_ is None else 1, *a, None)
    eps = C.c_float(1e-6)
    assert lib.q4_rmsnorm_prepare(x, add, 0, w, 1, y, T, K, eps, 0, prep, need, None) == -2    # planes vs add
    assert lib.q4_rmsnorm_prepare(x, None, 2, w, 1, y, T, K, eps, 0, prep, need, None) == -2
    assert lib.q4_rmsnorm_prepare(x, add, 65, w, 1, y, T, K, eps, 0, prep, need, None) == -2
    # y on the second of two planes
    assert lib.q4_rmsnorm_prepare(x, add, 2, w, 1, C.c_void_p(0x20000000 + T * K * 4), T, K, eps, 0, prep, need,
                                  None) == -2
    assert call(x, add, w, 1, y, T, K, eps, 2, prep, need) == -2                     # precision
    assert call(x, add, w, 7, y, T, K, eps, 0, prep, need) == -2                     # w dtype
    assert call(x, add, w, 1, y, T, K + 16, eps, 0, prep, need) == -1                # K % 32
    assert call(x, add, w, 1, y, -1, K, eps, 0, prep, need) == -1                    # T
    assert call(x, add, w, 1, y, T, 16384 + 32, eps, 0, prep, need) == -5            # K > 16384
    assert call(x, add, w, 1, y, T, K, C.c_float(-1.0), 0, prep, need) == -2         # eps
    assert call(x, add, w, 1, y, 0, K, eps, 0, prep, need) == 0                      # nothing to do
    assert call(None, add, w, 1, y, T, K, eps, 0, prep, need) == -2                  # NULL x
    assert call(x, add, w, 1, y, T, K, eps, 0, C.c_void_p(0x50000008), need) == -2   # misaligned
    assert call(x, add, w, 1, y, T, K, eps, 0, prep, need - 1) == -3                 # too small
    assert call(x, add, w, 1, y, T, K, eps, 0, C.c_void_p(0x10000000 + 4096), need) == -2   # on x
    assert call(x, add, w, 1, C.c_void_p(0x10000000 + 64), T, K, eps, 0, prep, need) == -2  # y partly on x
    assert call(x, add, w, 1, C.c_void_p(0x20000000), T, K, eps, 0, prep, need) == -2      # y on add


def test_swiglu_prepare_argument_errors(lib):
    """q4_swiglu_prepare refuses bad enums, shapes, strides, sizes and overlapping outputs
    before any launch."""
    T, F = 256, 14336
    need = lib.q4_prefill_prepared_bytes(T, F, 1, 0)
    g, u, h, prep = (C.c_void_p(0x100000000 * i) for i in (1, 2, 3, 4))
    call = lambda *a: lib.q4_swiglu_prepare(*a, None)
    assert call(g, u, F, F, T, F, 2, h, prep, need) == -2                         # precision
    assert call(g, u, F, F, T, F + 16, 0, h, prep, need) == -1                    # F % 32
    assert call(g, u, F - 32, F, T, F, 0, h, prep, need) == -1                    # ldg < F
    assert call(g, u, F, F + 2, T, F, 0, h, prep, need) == -1                     # ldu % 4
    assert call(g, u, F, F, -1, F, 0, h, prep, need) == -1                        # T
    assert call(g, u, 16416, 16416, T, 16416, 0, h, prep, need) == -5             # F > 16384
    assert call(g, u, F, F, 0, F, 0, h, prep, need) == 0                          # nothing to do
    assert call(None, u, F, F, T, F, 0, h, prep, need) == -2                      # NULL g
    assert call(g, u, F, F, T, F, 0, C.c_void_p(0x300000008), prep, need) == -2   # misaligned h
    assert call(g, u, F, F, T, F, 0, h, prep, need - 1) == -3                     # too small
    assert call(g, u, F, F, T, F, 0, h, C.c_void_p(0x100000000 + 4096), need) == -2   # on g
    assert call(g, u, F, F, T, F, 0, C.c_void_p(0x200000000 + 64), prep, need) == -2  # h on u


def test_gemm_prefill_swiglu_argument_errors(lib):
    """q4_gemm_prefill_swiglu refuses two-pass activations and shapes the epilogue cannot pair
    before any launch."""
    gu, sc, prep, h = (C.c_void_p(0x10000000 * i) for i in (1, 2, 3, 4))
    call = lambda *a: lib.q4_gemm_prefill_swiglu(*a, None)
    assert call(gu, sc, prep, 1, h, 256, 14336, 4096, 2) == -2        # precision
    assert call(gu, sc, prep, 0, h, 256, 14336, 4096, 0) == -2        # f32 x, precision 0: two passes
    assert call(gu, sc, prep, 1, h, 256, 14336 + 64, 4096, 0) == -1   # F % 128
    assert call(gu, sc, prep, 1, h, 256, 14336, 4096 + 32, 0) == -1   # K % 64
    assert call(gu, sc, prep, 1, h, 0, 14336, 4096, 0) == 0           # nothing to do
    assert call(gu, None, prep, 1, h, 256, 14336, 4096, 0) == -2      # precision 0 needs scales
    assert call(gu, sc, prep, 1, C.c_void_p(0x40000008), 256, 14336, 4096, 0) == -2   # misaligned h


def test_prefill_partials_argument_errors(lib):
    """q4_gemm_prefill_prepared_partials refuses two-pass activations and bad shapes before any
    launch; the split count query follows the plan."""
    assert lib.q4_prefill_split_count(2048, 4096, 14336) >= 1
    assert lib.q4_prefill_split_count(2048, 4100, 14336) == 0
    w, sc, prep, part = (C.c_void_p(0x10000000 * i) for i in (1, 2, 3, 4))
    big = 1 << 40
    call = lambda w_, sc_, prep_, dt, part_, *a: lib.q4_gemm_prefill_prepared_partials(w_, sc_, prep_, dt, part_, big,
                                                                                       *a, None)
    assert call(w, sc, prep, 0, part, 256, 4096, 14336, 0) == -2      # f32 x, precision 0: two passes
    assert call(w, sc, prep, 1, part, 256, 4096, 14336, 3) == -2      # precision
    assert call(w, sc, prep, 1, part, 256, 4100, 14336, 0) == -1      # N % 64
    assert call(w, None, prep, 1, part, 256, 4096, 14336, 0) == -2    # precision 0 needs scales
    assert call(w, sc, prep, 1, part, 0, 4096, 14336, 0) == 0         # nothing to do
    # part smaller than the plan's S planes: refused before any launch
    S = lib.q4_prefill_split_count(256, 4096, 14336)
    need = S * 256 * 4096 * 4
    assert lib.q4_gemm_prefill_prepared_partials(w, sc, prep, 1, part, need - 4, 256, 4096, 14336, 0, None) == -3


def test_rmsnorm_prepare_weight_extent_follows_its_dtype(lib):
    """The norm weight's extent in the overlap check follows its dtype: K * 2 bytes for bf16,
    K * 4 for f32 (every call here is refused before any launch)."""
    T, K = 256, 4096
    need = lib.q4_prefill_prepared_bytes(T, K, 1, 0)
    x, y = C.c_void_p(0x10000000), C.c_void_p(0x30000000)
    w = 0x50000000
    eps = C.c_float(1e-6)
    call = lambda wdt, at: lib.q4_rmsnorm_prepare(x, None, 0, C.c_void_p(w), wdt, y, T, K, eps, 0, C.c_void_p(at),
                                                  need, None)
    assert call(1, w + K * 2 - 16) == -2       # bf16: the buffer's first 16 bytes on the weight's last 8 values
    assert call(0, w + K * 2) == -2            # f32: the same address is inside its K * 4 bytes
    assert call(0, w + K * 4 - 16) == -2


def test_probes_refuse_bad_arguments(lib):
    """The measurement probes validate before any launch."""
    assert lib.q4_probe_stream_read(None, 16, 0, None, None) == -5     # workgroups
    assert lib.q4_probe_stream_read(None, 17, 4, None, None) == -1     # bytes % 16
    assert lib.q4_probe_stream_read(None, 16, 4, None, None) == -2     # NULL
    assert lib.q4_probe_stream_read(None, 0, 4, None, None) == 0       # nothing to read
    assert lib.q4_probe_stream_read_out_bytes(8) == 128 and lib.q4_probe_stream_read_out_bytes(0) == 0
    assert lib.q4_probe_mfma(0, 1, None, None, None) == -5
    assert lib.q4_probe_mfma(1, 1, None, None, None) == -2
    assert lib.q4_probe_mfma(1, 1, C.c_void_p(0x1004), C.c_void_p(0x1000), None) == -2   # misaligned operands


def test_moe_shared_argument_errors(lib):
    """q4_moe_gemv_shared validates the shared expert before any launch."""
    f = C.c_void_p(0x1000)
    ws = lib.q4_moe_shared_workspace_bytes(16, 128, 8, 2048, 768, 768)
    assert ws > lib.q4_moe_workspace_bytes(16, 128, 8, 2048, 768)
    assert lib.q4_moe_shared_workspace_bytes(16, 128, 8, 2048, 768, 0) == 0
    call = lambda sgu, sdn, Fs, sgw, out=C.c_void_p(0x9000000), wsp=C.c_void_p(0x10000000), wsb=ws: \
        lib.q4_moe_gemv_shared(f, f, sgu, sdn, Fs, sgw, f, 1, f, f, None, out, 16, 128, 8, 2048, 768, wsp, wsb, None)
    assert call(None, f, 768, f) == -2                 # no shared gate/up
    assert call(f, None, 768, f) == -2                 # no shared down
    assert call(f, f, 768, None) == -2                 # no gate vector
    assert call(f, f, 96, f) == -1                     # Fs % 64
    assert call(f, f, 768, f, wsb=ws - 1) == -3        # short workspace
    assert call(f, f, 768, f, out=C.c_void_p(0x10000000 + 256)) == -2   # out inside the workspace


def test_decode_segment_plan_and_argument_errors(lib):
    """q4_decode_segment: the split plan and the workspace size need no GPU (256 CUs, as on
    MI355X, when none is visible); shapes, the norm dtype, pointers, overlaps and the
    workspace are checked before any launch."""
    sp = (C.c_int * 3)()
    assert lib.q4_decode_segment_splits(4096, 14336, 6144, sp) == 0 and list(sp) == [4, 4, 8]
    assert lib.q4_decode_segment_splits(4096, 14336, 0, sp) == 0 and list(sp) == [4, 4, 0]
    assert lib.q4_decode_segment_splits(4096, 14336, 100, sp) == -1
    assert lib.q4_decode_segment_splits(8192, 14336, 6144, sp) == -1          # H > 4096
    ws = lib.q4_decode_segment_workspace_bytes(4096, 14336, 6144)
    assert ws == 12800 + 4 * 4096 * 4 + 14336 * 2
    assert lib.q4_decode_segment_workspace_bytes(4096, 14336, 96) == 0
    f = lambda a: C.c_void_p(a)
    base = dict(o=0x1000, g=0x2000, u=0x3000, d=0x4000, q=0x5000, attn=0x6000, x=0x100000, n1=0x7000, n2=0x8000,
                nwd=1, xm=0x200000, xn=0x300000, pd=0x400000, pq=0x500000, H=4096, F=14336, NQ=6144,
                ws=0x600000, wsb=ws)

    def call(**kw):
        a = dict(base, **kw)
        return lib.q4_decode_segment(f(a["o"]), f(a["g"]), f(a["u"]), f(a["d"]), None if a["q"] is None else f(a["q"]),
                                     f(a["attn"]), f(a["x"]), f(a["n1"]), f(a["n2"]), a["nwd"], 1e-6, f(a["xm"]),
                                     f(a["xn"]), f(a["pd"]), f(a["pq"]), a["H"], a["F"], a["NQ"], f(a["ws"]),
                                     a["wsb"], None)
    assert call(H=4000) == -1                       # H % 64
    assert call(F=100) == -1                        # F % 64
    assert call(nwd=7) == -2                        # norm weight dtype
    assert call(o=0) == -2                          # NULL weights
    assert call(n2=0) == -2                         # qkv without its norm weight
    assert call(attn=0x6008) == -2                  # misaligned
    assert call(wsb=ws - 1) == -3                   # short workspace
    assert call(xm=0x100000) == -2                  # x_mid over x
    assert call(xn=0x200000 + 64) == -2             # x_next over x_mid
    assert call(pd=0x600000 + 12800) == -2          # planes inside the workspace
    assert call(pq=0x400000 + 4 * 4096 * 4 - 16) == -2   # qkv planes over the down planes
