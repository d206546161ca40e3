"""GPU parity of the native q8 path (mx8 layout: 8-bit codes + a bf16 scale per row and
block, the reference's q8 GEMV designs/gemv_q4/gemv_q8.h): repacked bytes bit-exact
against the oracle from all three sources, dequant = s * q exactly (the values of the
exact hi/lo split), GEMV maxrel <= 1e-3 against the fp64 product of those values and
within fp32 noise of the split-pair kernel, residual form equal to GEMV + residual."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu

MAXREL = 1e-3


def _src(oracle, fmt, n, k, rs, rng):
    if fmt == "q8_0":
        b = oracle.random_q8_0_blocks(n, k, rng)
        return b, oracle.q8_0_rows(b)
    if fmt == "chunks":
        ch = oracle.random_q8_chunks((n // 32) * (k // 256), rng)
        return ch, oracle.q8_chunks_rows(ch, n, k, rs)
    b = oracle.random_q8_0_blocks(n, k, rng)
    return oracle.pack_gguf_pool_q8_f32(b, rs), oracle.q8_0_rows(b)


@pytest.mark.parametrize("fmt,rs", [("chunks", 1), ("chunks", 2), ("q8_0", 1), ("chunks_f32", 2)])
@pytest.mark.parametrize("n,k", [(64, 256), (256, 4096)])
def test_repack_bytes_and_dequant(gpu, pkg, oracle, fmt, rs, n, k):
    say(f"q8 native repack {fmt} rs={rs} n={n} k={k}")
    rng = np.random.default_rng(n + k + rs)
    src, (s16, q) = _src(oracle, fmt, n, k, rs, rng)
    w = pkg.pack_q8_native(src, n, k, fmt, rs, gpu)
    torch.cuda.synchronize()
    assert w.nbytes == oracle.mx8_bytes(n, k)
    assert np.array_equal(w.data.cpu().numpy(), oracle.pack_mx8_from_parts(s16, q))
    want = oracle.q8_values(s16, q).astype(np.float32)
    assert pkg.dequant_q8_native(w).cpu().numpy().tobytes() == want.tobytes()


@pytest.mark.parametrize("n,k", [(64, 32), (1024, 4096), (4096, 4096), (256, 14336)])
@pytest.mark.parametrize("M", [1, 5, 16])
def test_gemv_matches_fp64_and_the_split_pair(gpu, pkg, oracle, n, k, M):
    say(f"q8 native gemv n={n} k={k} M={M}")
    rng = np.random.default_rng(n + k + M)
    b = oracle.random_q8_0_blocks(n, k, rng)
    s16, q = oracle.q8_0_rows(b)
    x = torch.from_numpy(rng.standard_normal((M, k)).astype(np.float32)).to(torch.bfloat16)
    y = pkg.gemm_q8_native(pkg.pack_q8_native(b, n, k, "q8_0", device=gpu), x.to(gpu)).cpu().numpy()
    ref = x.to(torch.float32).numpy().astype(np.float64) @ oracle.q8_values(s16, q).T
    assert oracle.maxrel(y, ref) <= MAXREL
    pair = pkg.gemm_q8(pkg.pack_q8(b, n, k, "q8_0", device=gpu), x.to(gpu)).cpu().numpy()
    assert oracle.maxrel(y, pair) <= 1e-5                  # same weights, fp32 accumulation order only


def test_f32_activations_and_residual(gpu, pkg, oracle):
    say("q8 native f32 x + residual")
    rng = np.random.default_rng(5)
    n, k, M = 512, 2048, 3
    b = oracle.random_q8_0_blocks(n, k, rng)
    s16, q = oracle.q8_0_rows(b)
    w = pkg.pack_q8_native(b, n, k, "q8_0", device=gpu)
    x = torch.from_numpy(rng.standard_normal((M, k)).astype(np.float32)).to(gpu)
    y = pkg.gemm_q8_native(w, x).cpu().numpy()
    assert oracle.maxrel(y, x.cpu().numpy().astype(np.float64) @ oracle.q8_values(s16, q).T) <= MAXREL
    res = torch.from_numpy(rng.standard_normal((M, n)).astype(np.float32)).to(gpu)
    yr = pkg.gemm_q8_native(w, x, residual=res).cpu().numpy()
    assert np.allclose(yr, y + res.cpu().numpy(), rtol=0, atol=1e-5 * np.abs(y).max())
    acc = res.clone()
    pkg.gemm_q8_native(w, x, y=acc, residual=acc)
    assert np.array_equal(acc.cpu().numpy(), yr)


def test_extreme_codes(gpu, pkg, oracle):
    """-128, 127, -1 and 0 in every position: the +128 offset and the nibble split hold."""
    say("q8 native extreme codes")
    n, k = 64, 256
    b = np.zeros((n, k // 32, 34), np.uint8)
    b[..., 0:2] = np.array([0.01], np.float16).view(np.uint8)
    vals = np.array([-128, 127, -1, 0], np.int8)
    b[..., 2:] = np.resize(vals, (n, k // 32, 32)).view(np.uint8)
    s16, q = oracle.q8_0_rows(b)
    w = pkg.pack_q8_native(b, n, k, "q8_0", device=gpu)
    assert pkg.dequant_q8_native(w).cpu().numpy().tobytes() == oracle.q8_values(s16, q).astype(np.float32).tobytes()
    x = torch.ones(1, k, dtype=torch.bfloat16, device=gpu)
    y = pkg.gemm_q8_native(w, x).cpu().numpy()
    assert np.allclose(y, oracle.q8_values(s16, q).sum(1)[None], rtol=1e-6, atol=1e-6)
