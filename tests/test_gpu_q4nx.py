"""GPU parity of the .q4nx chunk transcodes (q4_repack_pool with rs = 1,
q4_repack_pool_signed, q4_repack_q8_chunks, q4_repack_q4k_chunks) against the oracle --
bytes bit-exact -- and of matrices read straight out of a container, through to a
GEMV that meets the 1e-3 bar."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say
from q4nx_writer import write_q4nx

pytestmark = pytest.mark.gpu


def _want(oracle, pool_q4_1, n, k, rs):
    d16, m16, q = oracle.pool_to_blocks(pool_q4_1.reshape(-1), n, k, rs)
    return oracle.pack_mx_from_parts(d16, m16, q)


@pytest.mark.parametrize("rs", [1, 2])
@pytest.mark.parametrize("n,k", [(64, 256), (256, 1024), (128, 4096)])
def test_signed_pool(gpu, pkg, oracle, n, k, rs):
    say(f"repack signed n={n} k={k} rs={rs}")
    rng = np.random.default_rng(n + k + rs)
    sig = oracle.random_signed_pool((n // 32) * (k // 256), rng)
    w = pkg.pack_chunks(sig, "q4_0", n, k, rs, gpu)
    torch.cuda.synchronize()
    assert np.array_equal(w.data.cpu().numpy(), _want(oracle, oracle.signed_pool_to_q4_1(sig), n, k, rs))


@pytest.mark.parametrize("rs", [1, 2])
@pytest.mark.parametrize("n,k", [(64, 256), (256, 1024), (4096, 4096)])
def test_q8_requant(gpu, pkg, oracle, n, k, rs):
    say(f"repack q8 n={n} k={k} rs={rs}")
    rng = np.random.default_rng(3 * n + k + rs)
    q8 = oracle.random_q8_chunks((n // 32) * (k // 256), rng)
    w = pkg.pack_chunks(q8, "q8", n, k, rs, gpu)
    torch.cuda.synchronize()
    assert np.array_equal(w.data.cpu().numpy(), _want(oracle, oracle.requant_q4_1(q8), n, k, rs))


def test_q8_requant_edge_blocks(gpu, pkg, oracle):
    """Constant blocks, all-zero blocks, +-128 extremes and a zero scale."""
    say("repack q8 edges")
    rng = np.random.default_rng(5)
    q8 = oracle.random_q8_chunks(4, rng)
    q8[0, 512:] = 4
    q8[1, 512:] = 0
    q8[2, 512::2] = 0x80
    q8[2, 513::2] = 0x7F
    q8[3, :64] = 0                                     # 32 zero scales
    w = pkg.pack_chunks(q8, "q8", 64, 512, 1, gpu)
    torch.cuda.synchronize()
    assert np.array_equal(w.data.cpu().numpy(), _want(oracle, oracle.requant_q4_1(q8), 64, 512, 1))


def test_container_end_to_end(gpu, pkg, oracle, tmp_path):
    say("q4nx end to end")
    rng = np.random.default_rng(8)
    n, k = 256, 1024
    nch = (n // 32) * (k // 256)
    blocks = oracle.random_q4_1_blocks_ref(n, k, rng)
    q41 = oracle.pack_q4_1_pool(blocks, 1).reshape(nch, 5120)
    sig = oracle.random_signed_pool(nch, rng)
    q8 = oracle.random_q8_chunks(nch, rng)
    q4k = oracle.q4k_vector(nch)
    p = tmp_path / "m.q4nx"
    write_q4nx(p, [("a", "I8", (nch, 5120), q41), ("b", "I8", (nch, 5120), sig), ("c", "I8", (nch, 8704), q8),
                   ("d", "I8", (nch, 4736), q4k)])
    with pkg.Q4NXFile(p) as f:
        wa, wb, wc, wd = (f.packed(x, n, k, gpu) for x in "abcd")
        with pytest.raises(Exception, match="holds"):
            f.packed("a", n, 2 * k, gpu)
    torch.cuda.synchronize()
    assert np.array_equal(wa.data.cpu().numpy(), oracle.pack_mx(blocks))
    assert np.array_equal(wb.data.cpu().numpy(), _want(oracle, oracle.signed_pool_to_q4_1(sig), n, k, 1))
    assert np.array_equal(wc.data.cpu().numpy(), _want(oracle, oracle.requant_q4_1(q8), n, k, 1))
    assert np.array_equal(wd.data.cpu().numpy(), _want(oracle, oracle.q4k_chunks_to_pool(q4k), n, k, 1))
    x = rng.standard_normal((2, k)).astype(np.float32)
    for w in (wb, wc):
        y = pkg.gemm_q4(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
        ref = x.astype(np.float64) @ pkg.dequant(w).cpu().numpy().astype(np.float64).T
        assert oracle.maxrel(y, ref) <= 1e-3


def test_decode_benchmark_harness(gpu, pkg, oracle, tmp_path):
    """bench.py --model-dir: the reference harness's JSON (benchmark-q4-decode.py:37-54) on a
    container's q4_1 tensor, its two CPU decoders byte-identical, and the GPU repack + dequant
    byte-identical with them, with the logical shape given and without."""
    import bench
    say("q4nx decode benchmark harness")
    rng = np.random.default_rng(12)
    n, k = 512, 2048
    nch = (n // 32) * (k // 256)
    blocks = oracle.random_q4_1_blocks_ref(n, k, rng)
    name = "model.layers.0.mlp.up_proj.weight"
    write_q4nx(tmp_path / "model.q4nx", [(name, "I8", (nch, 5120), oracle.pack_q4_1_pool(blocks, 1).reshape(nch, 5120))])
    for shape in ((n, k), None):
        r = bench.q4nx_decode_harness(tmp_path, name, shape, reps=3)
        assert r["tensor"] == name and r["chunks"] == nch
        assert r["byte_identical"] and r["gpu"]["byte_identical"], r
        assert r["gpu"]["shape"] == ([n, k] if shape else [32 * nch, 256])
        assert r["legacy_seconds"] > 0 and r["contiguous_seconds"] > 0 and r["gpu"]["dequant_us"] > 0
