"""CPU pins of the native Q4_K layout's oracle (pack_mxk_* / unpack_mxk / dequant_mxk).

What fixes them independently of their own formulas:
* GGUF blocks: dequant_mxk of the packed matrix equals dequant_q4_k bit for bit, and
  dequant_q4_k is held to the reference's own C++ GGUF reader (tests/test_gguf.py);
* container chunks: it equals the f32 rounding of dequant_q4k_chunks_exact (the chunk's
  value S sc nib + M mn in f64, gemm_q4.h:456-507), placed by chunk_geometry;
* a scalar loop that reads single codes, multipliers and bases off the bytes by the
  layout's address formulas;
* round trips of the parts, and planted slips (d and m swapped, sc and mn swapped, a
  nibble order flipped) that the equalities above catch.
"""
from __future__ import annotations

import numpy as np
import pytest


def _chunk_value_f32(oracle, chunks, n, k, rs):
    nch, _, rows0, cols0 = oracle.chunk_geometry(n, k, rs)
    ex = oracle.dequant_q4k_chunks_exact(chunks)
    full = np.empty((n, k))
    for c in range(nch):
        r0, c0 = int(rows0[c]), int(cols0[c])
        full[r0:r0 + 32, c0:c0 + 256] = ex[c]
    return full.astype(np.float32)


@pytest.mark.parametrize("n,k", [(64, 256), (128, 1024), (192, 512)])
def test_gguf_blocks_pack_to_their_exact_value(oracle, n, k):
    rng = np.random.default_rng(n + k)
    b = oracle.random_q4_k_blocks(n, k, rng)
    pk = oracle.pack_mxk_q4_k(b)
    assert pk.size == oracle.mxk_bytes(n, k) == (n // 64) * (k // 256) * 9728
    w = oracle.dequant_mxk(pk, n, k)
    assert w.tobytes() == oracle.dequant_q4_k(b).tobytes()
    parts = oracle.unpack_mxk(pk, n, k)
    for got, want in zip(parts, oracle.q4_k_native_parts(b)):
        assert np.array_equal(got, want)


@pytest.mark.parametrize("rs", [1, 2])
def test_container_chunks_pack_to_their_exact_value(oracle, rs):
    n, k = 128, 1024
    chunks = oracle.q4k_vector((n // 32) * (k // 256))
    w = oracle.dequant_mxk(oracle.pack_mxk_q4k_chunks(chunks, n, k, rs), n, k)
    assert w.tobytes() == _chunk_value_f32(oracle, chunks, n, k, rs).tobytes()


def test_byte_addresses_by_scalar_loop(oracle):
    """Read values off the packed bytes one at a time by the layout's address formulas."""
    n, k = 128, 512
    rng = np.random.default_rng(5)
    b = oracle.random_q4_k_blocks(n, k, rng)
    d, m, sc, mn, q = oracle.q4_k_native_parts(b)
    pk = oracle.pack_mxk_q4_k(b)
    SB = k // 256
    for _ in range(300):
        row, col = int(rng.integers(n)), int(rng.integers(k))
        g, i = row // 64, row % 64
        r, i16 = i // 16, i % 16
        sb, kb = col // 256, col // 32
        j, kg, e = kb % 8, (col % 32) // 8, col % 8
        tile = (g * SB + sb) * 9728
        dword = int.from_bytes(pk[tile + j * 1024 + (kg * 16 + i16) * 16 + r * 4:][:4].tobytes(), "little")
        assert (dword >> (16 * (e % 2) + 4 * (e // 2))) & 0xF == q[row, col]
        pair = tile + 8192 + i16 * 64 + r * 16
        assert pk[pair + j] == sc[row, sb, j] and pk[pair + 8 + j] == mn[row, sb, j]
        dd = np.frombuffer(pk[tile + 9216 + i16 * 16 + r * 4:][:4].tobytes(), np.float32)[0]
        mm = np.frombuffer(pk[tile + 9472 + i16 * 16 + r * 4:][:4].tobytes(), np.float32)[0]
        assert dd == d[row, sb] and mm == m[row, sb]


def test_planted_slips_are_caught(oracle):
    n, k = 64, 256
    b = oracle.random_q4_k_blocks(n, k, np.random.default_rng(7))
    want = oracle.dequant_q4_k(b)
    d, m, sc, mn, q = oracle.q4_k_native_parts(b)
    for parts in ((m, d, sc, mn, q), (d, m, mn, sc, q), (d, m, sc, mn, (15 - q).astype(np.uint8))):
        w = oracle.dequant_mxk(oracle.pack_mxk_from_parts(*parts), n, k)
        assert w.tobytes() != want.tobytes()
