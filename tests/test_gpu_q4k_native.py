"""GPU parity of the native Q4_K path (the reference's Q4_K GEMM, gemm_q4.h:456-507): the
super-block's integers kept, no bf16 collapse.

Bars: repacked bytes bit-exact against the oracle (GGUF blocks and the container's
chunks), dequant bit-exact against the GGUF reader's values / the chunk's exact value,
GEMV maxrel <= 1e-3 against the fp64 product of the exact weights (and below the
q4_1 collapse's error on the same weights), residual form equal to GEMV + residual.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu

MAXREL = 1e-3


@pytest.mark.parametrize("n,k", [(64, 256), (192, 1024), (4096, 4096), (128, 14336)])
def test_repack_gguf_bytes_and_dequant(gpu, pkg, oracle, n, k):
    say(f"q4k native repack n={n} k={k}")
    rng = np.random.default_rng(n + 7 * k)
    blocks = oracle.random_q4_k_blocks(n, k, rng)
    w = pkg.pack_q4_k_native(blocks, gpu)
    torch.cuda.synchronize()
    assert w.nbytes == pkg.q4k_packed_bytes(n, k) == oracle.mxk_bytes(n, k)
    assert np.array_equal(w.data.cpu().numpy(), oracle.pack_mxk_q4_k(blocks))
    assert pkg.dequant_q4k(w).cpu().numpy().tobytes() == oracle.dequant_q4_k(blocks).tobytes()


@pytest.mark.parametrize("rs", [1, 2])
def test_repack_container_chunks(gpu, pkg, oracle, rs):
    say(f"q4k native chunks rs={rs}")
    n, k = 256, 2048
    chunks = oracle.q4k_vector((n // 32) * (k // 256))
    w = pkg.pack_q4_k_chunks_native(chunks, n, k, rs, gpu)
    torch.cuda.synchronize()
    assert np.array_equal(w.data.cpu().numpy(), oracle.pack_mxk_q4k_chunks(chunks, n, k, rs))
    want = oracle.dequant_mxk(oracle.pack_mxk_q4k_chunks(chunks, n, k, rs), n, k)
    assert pkg.dequant_q4k(w).cpu().numpy().tobytes() == want.tobytes()


@pytest.mark.parametrize("n,k", [(64, 256), (256, 4096), (4096, 4096), (1024, 14336)])
@pytest.mark.parametrize("M", [1, 3, 8, 16])
def test_gemv_matches_fp64_of_exact_weights(gpu, pkg, oracle, n, k, M):
    say(f"q4k native gemv n={n} k={k} M={M}")
    rng = np.random.default_rng(n + k + M)
    blocks = oracle.random_q4_k_blocks(n, k, rng)
    w = pkg.pack_q4_k_native(blocks, gpu)
    x = torch.from_numpy(rng.standard_normal((M, k)).astype(np.float32)).to(torch.bfloat16)
    y = pkg.gemm_q4k(w, x.to(gpu)).cpu().numpy()
    ref = x.to(torch.float32).numpy().astype(np.float64) @ oracle.dequant_q4_k(blocks).astype(np.float64).T
    err = oracle.maxrel(y, ref)
    assert err <= MAXREL, f"maxrel {err:.3e}"


def test_f32_activations_and_residual(gpu, pkg, oracle):
    say("q4k native f32 x + residual")
    rng = np.random.default_rng(11)
    n, k, M = 512, 4096, 5
    blocks = oracle.random_q4_k_blocks(n, k, rng)
    w = pkg.pack_q4_k_native(blocks, gpu)
    x = torch.from_numpy(rng.standard_normal((M, k)).astype(np.float32)).to(gpu)
    y = pkg.gemm_q4k(w, x).cpu().numpy()
    ref = x.cpu().numpy().astype(np.float64) @ oracle.dequant_q4_k(blocks).astype(np.float64).T
    assert oracle.maxrel(y, ref) <= MAXREL
    res = torch.from_numpy(rng.standard_normal((M, n)).astype(np.float32)).to(gpu)
    yr = pkg.gemm_q4k(w, x, residual=res).cpu().numpy()
    assert np.allclose(yr, y + res.cpu().numpy(), rtol=0, atol=1e-5 * np.abs(y).max())
    acc = res.clone()
    pkg.gemm_q4k(w, x, y=acc, residual=acc)           # in place
    assert np.array_equal(acc.cpu().numpy(), yr)


def test_native_beats_the_q4_1_collapse(gpu, pkg, oracle):
    """Same GGUF Q4_K weights through the native kernel and through the bf16-collapsed
    mx layout: against the fp64 product of the exact weights the native error is the
    smaller one (it carries no rounding of d sc, m mn)."""
    say("q4k native vs collapse")
    rng = np.random.default_rng(13)
    n, k = 2048, 4096
    blocks = oracle.random_q4_k_blocks(n, k, rng)
    x = torch.from_numpy(rng.standard_normal((4, k)).astype(np.float32)).to(torch.bfloat16)
    ref = x.to(torch.float32).numpy().astype(np.float64) @ oracle.dequant_q4_k(blocks).astype(np.float64).T
    native = pkg.gemm_q4k(pkg.pack_q4_k_native(blocks, gpu), x.to(gpu)).cpu().numpy()
    collapsed = pkg.gemm_q4(pkg.pack_q4_k(blocks, gpu), x.to(gpu)).cpu().numpy()
    e_native, e_collapsed = oracle.maxrel(native, ref), oracle.maxrel(collapsed, ref)
    assert e_native < e_collapsed, (e_native, e_collapsed)
    assert e_native < 1e-5


def test_gemv_is_deterministic_across_splits(gpu, pkg, oracle):
    say("q4k native determinism")
    rng = np.random.default_rng(17)
    n, k = 256, 14336                     # few row groups: K is split on super-blocks
    assert pkg.load_library().q4_gemv_q4k_workspace_bytes(1, n, k) > 0
    w = pkg.pack_q4_k_native(oracle.random_q4_k_blocks(n, k, rng), gpu)
    x = torch.from_numpy(rng.standard_normal((1, k)).astype(np.float32)).to(torch.bfloat16).to(gpu)
    a = pkg.gemm_q4k(w, x).cpu()
    for _ in range(3):
        assert torch.equal(a, pkg.gemm_q4k(w, x).cpu())


def test_file_readers_keep_q4k_native(gpu, pkg, oracle, tmp_path):
    """GGUFFile.packed(..., q4k="native") and Q4NXFile.packed(..., q4k="native") hand the
    file's own Q4_K bytes to the native repack: the oracle's bytes, and a GEMV at the bar."""
    from gguf_writer import STR, write_gguf
    from q4nx_writer import write_q4nx
    say("q4k native from gguf / q4nx files")
    rng = np.random.default_rng(23)
    n, k = 256, 1024
    blocks = oracle.random_q4_k_blocks(n, k, rng)
    pg = tmp_path / "m.gguf"
    write_gguf(pg, [("blk.0.ffn_gate.weight", "Q4_K", (n, k), blocks)], [("general.architecture", STR, "llama")])
    nch = (n // 32) * (k // 256)
    chunks = oracle.q4k_vector(nch)
    pq = tmp_path / "m.q4nx"
    write_q4nx(pq, [("d", "I8", (nch, 4736), chunks)])
    with pkg.GGUFFile(pg) as f:
        wg = f.packed("blk.0.ffn_gate.weight", gpu, q4k="native")
        with pytest.raises(ValueError):
            f.packed("blk.0.ffn_gate.weight", gpu, q4k="bogus")
    with pkg.Q4NXFile(pq) as f:
        wq = f.packed("d", n, k, gpu, q4k="native")
    torch.cuda.synchronize()
    assert isinstance(wg, pkg.PackedQ4K) and isinstance(wq, pkg.PackedQ4K)
    assert np.array_equal(wg.data.cpu().numpy(), oracle.pack_mxk_q4_k(blocks))
    assert np.array_equal(wq.data.cpu().numpy(), oracle.pack_mxk_q4k_chunks(chunks, n, k, 1))
    x = rng.standard_normal((2, k)).astype(np.float32)
    for w, wt in ((wg, oracle.dequant_q4_k(blocks)), (wq, oracle.dequant_mxk(oracle.pack_mxk_q4k_chunks(chunks, n, k, 1), n, k))):
        y = pkg.gemm_q4k(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
        assert oracle.maxrel(y, x.astype(np.float64) @ wt.astype(np.float64).T) <= MAXREL
