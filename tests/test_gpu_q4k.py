"""GPU parity for the source formats feeding the kernels: GGUF Q4_K super-blocks and the
reference container's Q4_K chunks transcoded on the device, and weights read straight
out of a GGUF file.

Bars: transcoded bytes and their dequant bit-exact against the oracle; GEMV / prefill
outputs maxrel <= 1e-3 against the fp64 product of the same (bf16-collapsed) weights.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say
from gguf_writer import STR, write_gguf

pytestmark = pytest.mark.gpu

MAXREL = 1e-3


@pytest.mark.parametrize("n,k", [(64, 256), (192, 1024), (4096, 4096), (128, 14336)])
def test_repack_q4k_bytes_and_dequant_match_oracle(gpu, pkg, oracle, n, k):
    say(f"repack_q4k n={n} k={k}")
    rng = np.random.default_rng(n + 3 * k)
    blocks = oracle.random_q4_k_blocks(n, k, rng)
    w = pkg.pack_q4_k(blocks, gpu)
    torch.cuda.synchronize()
    assert np.array_equal(w.data.cpu().numpy(), oracle.pack_mx_q4_k(blocks))
    wd = pkg.dequant(w).cpu().numpy()
    assert wd.tobytes() == oracle.dequant_q4_k_bf16(blocks).tobytes()


def test_repack_q4k_every_scale_min_code(gpu, pkg, oracle):
    """Uniform random bytes everywhere but d and dmin, over enough super-blocks that every
    6-bit scale and min value occurs in every sub-block slot."""
    say("repack_q4k exhaustive scales")
    rng = np.random.default_rng(99)
    blocks = oracle.random_q4_k_blocks(512, 2048, rng)
    D, M, _ = oracle.unpack_q4_k_blocks(blocks)
    for j in range(8):
        s6, m6 = oracle.q4_k_scale_min(blocks[..., 4:16], j)
        assert len(np.unique(s6)) == 64 and len(np.unique(m6)) == 64
    w = pkg.pack_q4_k(blocks, gpu)
    torch.cuda.synchronize()
    assert np.array_equal(w.data.cpu().numpy(), oracle.pack_mx_q4_k(blocks))


@pytest.mark.parametrize("M", [1, 4, 16])
def test_gemv_on_q4k_weights(gpu, pkg, oracle, M):
    say(f"gemv q4k M={M}")
    rng = np.random.default_rng(M)
    n, k = 1024, 4096
    blocks = oracle.random_q4_k_blocks(n, k, rng)
    w = pkg.pack_q4_k(blocks, gpu)
    x = rng.standard_normal((M, k)).astype(np.float32)
    y = pkg.gemm_q4(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
    ref = (x.astype(np.float64) @ oracle.dequant_q4_k_bf16(blocks).astype(np.float64).T)
    err = oracle.maxrel(y, ref)
    assert err <= MAXREL, f"maxrel {err:.3e}"


def test_prefill_on_q4k_weights(gpu, pkg, oracle):
    say("prefill q4k T=300 N=512 K=2048")
    rng = np.random.default_rng(7)
    T, n, k = 300, 512, 2048
    blocks = oracle.random_q4_k_blocks(n, k, rng)
    w = pkg.pack_q4_k(blocks, gpu)
    x = torch.from_numpy(rng.standard_normal((T, k)).astype(np.float32)).to(torch.bfloat16)
    y = pkg.gemm_q4_prefill(w, x.to(gpu)).cpu().numpy()
    ref = x.to(torch.float32).numpy().astype(np.float64) @ oracle.dequant_q4_k_bf16(blocks).astype(np.float64).T
    err = oracle.maxrel(y, ref)
    assert err <= MAXREL, f"maxrel {err:.3e}"


@pytest.mark.parametrize("rs", [1, 2])
@pytest.mark.parametrize("n,k", [(64, 256), (128, 512), (256, 2048)])
def test_repack_q4k_chunks_matches_oracle(gpu, pkg, oracle, rs, n, k):
    """Container Q4_K chunks in band order: the device transcode equals the oracle's
    q4k_to_q4_1 followed by the pool -> mx permutation, byte for byte."""
    if n % (32 * rs):
        pytest.skip("rows not a whole number of bands")
    say(f"repack_q4k_chunks n={n} k={k} rs={rs}")
    rng = np.random.default_rng(n + k + rs)
    nch = (n // 32) * (k // 256)
    chunks = rng.integers(0, 256, (nch, oracle.Q4K_CHUNK), dtype=np.uint8)
    sm = np.concatenate([0x3B00 | rng.integers(0, 256, (nch, 32)), 0xBB00 | rng.integers(0, 256, (nch, 32))], 1)
    chunks[:, 4608:] = sm.astype(np.uint16).view(np.uint8)
    pool = oracle.q4k_chunks_to_pool(chunks)
    d16, m16, q = oracle.pool_to_blocks(pool.reshape(-1), n, k, rs)
    want = oracle.pack_mx_from_parts(d16, m16, q)
    w = pkg.pack_q4_k_chunks(chunks, n, k, rs, gpu)
    torch.cuda.synchronize()
    assert np.array_equal(w.data.cpu().numpy(), want)


def test_weights_straight_from_a_gguf_file(gpu, pkg, oracle, tmp_path):
    """A GGUF with Q4_K, Q4_1 and Q4_0 matrices: each packs on the device to the oracle's
    bytes, and a GEMV over the Q4_K one meets the bar."""
    say("gguf end to end")
    rng = np.random.default_rng(21)
    gate = oracle.random_q4_k_blocks(256, 1024, rng)
    up = oracle.random_q4_1_blocks_ref(256, 1024, rng)
    down = oracle.random_q4_0_blocks_ref(128, 256, rng)
    p = tmp_path / "m.gguf"
    write_gguf(p, [("blk.0.ffn_gate.weight", "Q4_K", (256, 1024), gate),
                   ("blk.0.ffn_up.weight", "Q4_1", (256, 1024), up),
                   ("blk.0.ffn_down.weight", "Q4_0", (128, 256), down)],
               [("general.architecture", STR, "llama")])
    with pkg.GGUFFile(p) as f:
        wg = f.packed("blk.0.ffn_gate.weight", gpu)
        wu = f.packed("blk.0.ffn_up.weight", gpu)
        wdn = f.packed("blk.0.ffn_down.weight", gpu)
    torch.cuda.synchronize()
    assert np.array_equal(wg.data.cpu().numpy(), oracle.pack_mx_q4_k(gate))
    assert np.array_equal(wu.data.cpu().numpy(), oracle.pack_mx(up))
    assert np.array_equal(wdn.data.cpu().numpy(), oracle.pack_mx(down))
    x = rng.standard_normal((2, 1024)).astype(np.float32)
    y = pkg.gemm_q4(wg, torch.from_numpy(x).to(gpu)).cpu().numpy()
    ref = x.astype(np.float64) @ oracle.dequant_q4_k_bf16(gate).astype(np.float64).T
    assert oracle.maxrel(y, ref) <= MAXREL
