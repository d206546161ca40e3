"""GPU parity of the q8 path: q4_repack_q8_split (hi/lo planes bit-exact against the
oracle, from 8704 B chunks and from GGUF Q8_0 blocks) and q4_gemv_q8 (maxrel <= 1e-3
against the fp64 product with the exact q8 values; the residual form in place)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say
from gguf_writer import write_gguf
from q4nx_writer import write_q4nx

pytestmark = pytest.mark.gpu


def _planes_want(oracle, s16, q):
    n, k = q.shape
    return [oracle.pack_mx_from_parts(*oracle.q8_split_parts(s16, q, p)) for p in (0, 1)]


@pytest.mark.parametrize("rs", [1, 2])
@pytest.mark.parametrize("n,k", [(64, 256), (256, 1024), (4096, 4096)])
def test_split_from_chunks(gpu, pkg, oracle, n, k, rs):
    say(f"q8 split chunks n={n} k={k} rs={rs}")
    rng = np.random.default_rng(n + k + rs)
    src = oracle.random_q8_chunks((n // 32) * (k // 256), rng)
    w = pkg.pack_q8(src, n, k, "chunks", rs, gpu)
    torch.cuda.synchronize()
    hi, lo = _planes_want(oracle, *oracle.q8_chunks_rows(src, n, k, rs))
    assert np.array_equal(w.hi.data.cpu().numpy(), hi) and np.array_equal(w.lo.data.cpu().numpy(), lo)


@pytest.mark.parametrize("n,k", [(64, 32), (192, 4096)])
def test_split_from_q8_0(gpu, pkg, oracle, n, k):
    say(f"q8 split q8_0 n={n} k={k}")
    rng = np.random.default_rng(n * 7 + k)
    b = oracle.random_q8_0_blocks(n, k, rng)
    w = pkg.pack_q8(b, n, k, "q8_0", device=gpu)
    torch.cuda.synchronize()
    hi, lo = _planes_want(oracle, *oracle.q8_0_rows(b))
    assert np.array_equal(w.hi.data.cpu().numpy(), hi) and np.array_equal(w.lo.data.cpu().numpy(), lo)


@pytest.mark.parametrize("xdt", ["bf16", "f32"])
@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("n,k", [(4096, 4096), (14336, 4096), (4096, 14336)])
def test_gemm_q8(gpu, pkg, oracle, n, k, M, xdt):
    say(f"gemm_q8 n={n} k={k} M={M} x={xdt}")
    rng = np.random.default_rng(n + k + M)
    b = oracle.random_q8_0_blocks(n, k, rng)
    w = pkg.pack_q8(b, n, k, "q8_0", device=gpu)
    x = rng.standard_normal((M, k)).astype(np.float32)
    xt = torch.from_numpy(x)
    if xdt == "bf16":
        xt = xt.to(torch.bfloat16)
        x = xt.to(torch.float32).numpy()
    y = pkg.gemm_q8(w, xt.to(gpu)).cpu().numpy()
    ref = x.astype(np.float64) @ oracle.q8_values(*oracle.q8_0_rows(b)).T
    assert oracle.maxrel(y, ref) <= 1e-3
    if M == 4 and xdt == "bf16":
        res = torch.from_numpy(rng.standard_normal((M, n)).astype(np.float32)).to(gpu)
        r0 = res.clone()
        pkg.gemm_q8(w, xt.to(gpu), y=res, residual=res)
        assert torch.equal(res, r0 + torch.from_numpy(y).to(gpu))


def test_q8_from_files(gpu, pkg, oracle, tmp_path):
    """GGUF Q8_0 through GGUFFile.packed and .q4nx q8 chunks through packed(q8="exact")."""
    say("q8 from gguf and q4nx")
    rng = np.random.default_rng(3)
    n, k = 256, 1024
    b = oracle.random_q8_0_blocks(n, k, rng)
    p = tmp_path / "m.gguf"
    write_gguf(p, [("blk.0.attn_q.weight", "Q8_0", (n, k), b)])
    with pkg.GGUFFile(p) as f:
        w = f.packed("blk.0.attn_q.weight", gpu)
    hi, lo = _planes_want(oracle, *oracle.q8_0_rows(b))
    assert np.array_equal(w.hi.data.cpu().numpy(), hi) and np.array_equal(w.lo.data.cpu().numpy(), lo)
    src = oracle.random_q8_chunks((n // 32) * (k // 256), rng)
    q = tmp_path / "m.q4nx"
    write_q4nx(q, [("w", "I8", (src.shape[0], 8704), src)])
    with pkg.Q4NXFile(q) as f:
        we = f.packed("w", n, k, gpu, q8="exact")
        wr = f.packed("w", n, k, gpu)
    hi, lo = _planes_want(oracle, *oracle.q8_chunks_rows(src, n, k, 1))
    assert np.array_equal(we.hi.data.cpu().numpy(), hi) and np.array_equal(we.lo.data.cpu().numpy(), lo)
    x = rng.standard_normal((2, k)).astype(np.float32)
    ye = pkg.gemm_q8(we, torch.from_numpy(x).to(gpu)).cpu().numpy()
    yr = pkg.gemm_q4(wr, torch.from_numpy(x).to(gpu)).cpu().numpy()
    ref = x.astype(np.float64) @ oracle.q8_values(*oracle.q8_chunks_rows(src, n, k, 1)).T
    assert oracle.maxrel(ye, ref) <= 1e-3
    assert oracle.maxrel(yr, ref) > oracle.maxrel(ye, ref)          # the requant is the lossy one


@pytest.mark.parametrize("rs", [1, 2])
def test_gguf_direct_pools(gpu, pkg, oracle, rs):
    """The GGUF-direct pool's 6144 B q4 chunks land on the same mx bytes as q4_repack of
    the GGUF blocks; its 9216 B q8 chunks on the same planes as the Q8_0 blocks."""
    say(f"gguf direct pools rs={rs}")
    rng = np.random.default_rng(30 + rs)
    n, k = 256, 1024
    for blocks in (oracle.random_q4_1_blocks_ref(n, k, rng), oracle.random_q4_0_blocks_ref(n, k, rng)):
        w = pkg.pack_chunks(oracle.pack_gguf_pool_f32(blocks, rs), "q4_f32", n, k, rs, gpu)
        torch.cuda.synchronize()
        assert np.array_equal(w.data.cpu().numpy(), oracle.pack_mx(blocks))
    b8 = oracle.random_q8_0_blocks(n, k, rng)
    w8 = pkg.pack_q8(oracle.pack_gguf_pool_q8_f32(b8, rs), n, k, "chunks_f32", rs, gpu)
    torch.cuda.synchronize()
    hi, lo = _planes_want(oracle, *oracle.q8_0_rows(b8))
    assert np.array_equal(w8.hi.data.cpu().numpy(), hi) and np.array_equal(w8.lo.data.cpu().numpy(), lo)
