"""CPU pins of the native q8 layout's oracle (pack_mx8_from_parts / unpack_mx8 /
dequant_mx8): dequant equals q8_values (s * q, the sum of the reference's exact hi/lo
split, recipes/pack.py:94-117) bit for bit for all three sources; a scalar loop reads
codes and scales off the bytes by the layout's address formulas; round trips hold; and
planted slips (an unpermuted byte order, a missing +128) are caught."""
from __future__ import annotations

import numpy as np
import pytest


def _sources(oracle, n, k, rng):
    nch = (n // 32) * (k // 256)
    ch = oracle.random_q8_chunks(nch, rng)
    g = oracle.random_q8_0_blocks(n, k, rng)
    return {"chunks": oracle.q8_chunks_rows(ch, n, k, 1), "q8_0": oracle.q8_0_rows(g)}


@pytest.mark.parametrize("n,k", [(64, 256), (128, 512)])
def test_dequant_is_s_times_q(oracle, n, k):
    for name, (s16, q) in _sources(oracle, n, k, np.random.default_rng(n + k)).items():
        pk = oracle.pack_mx8_from_parts(s16, q)
        assert pk.size == oracle.mx8_bytes(n, k) == (n // 64) * (k // 32) * 2176
        assert oracle.dequant_mx8(pk, n, k).tobytes() == oracle.q8_values(s16, q).astype(np.float32).tobytes(), name
        s2, q2 = oracle.unpack_mx8(pk, n, k)
        assert np.array_equal(s2, s16) and np.array_equal(q2, q), name


def test_byte_addresses_by_scalar_loop(oracle):
    n, k = 128, 256
    rng = np.random.default_rng(3)
    s16, q = oracle.q8_0_rows(oracle.random_q8_0_blocks(n, k, rng))
    pk = oracle.pack_mx8_from_parts(s16, q)
    kb_n = k // 32
    perm = [0, 2, 1, 3]
    for _ in range(300):
        row, col = int(rng.integers(n)), int(rng.integers(k))
        g, i = row // 64, row % 64
        r, i16 = i // 16, i % 16
        kb, kg, e = col // 32, (col % 32) // 8, col % 8
        tile = (g * kb_n + kb) * 2176
        group = pk[tile + (r // 2) * 1024 + (kg * 16 + i16) * 16 + (r % 2) * 8:][:8]
        h, kk = e // 4, e % 4
        byte = group[4 * h + perm.index(kk)]
        assert int(byte) - 128 == int(q[row, col])
        sb = pk[tile + 2048 + i16 * 8 + r * 2:][:2].view(np.uint16)[0]
        assert sb == s16[row, kb]


def test_planted_slips_are_caught(oracle):
    n, k = 64, 64
    s16, q = oracle.q8_0_rows(oracle.random_q8_0_blocks(n, k, np.random.default_rng(4)))
    want = oracle.q8_values(s16, q).astype(np.float32)
    pk = oracle.pack_mx8_from_parts(s16, q).reshape(-1, 2176).copy()
    plain = pk.copy()
    codes = plain[:, :2048].reshape(-1, 512, 4)
    plain[:, :2048] = codes[..., [0, 2, 1, 3]].reshape(-1, 2048)     # bytes written in natural k order
    assert oracle.dequant_mx8(plain.reshape(-1), n, k).tobytes() != want.tobytes()
    raw = pk.copy()
    raw[:, :2048] ^= 0x80                                              # codes without the +128
    assert oracle.dequant_mx8(raw.reshape(-1), n, k).tobytes() != want.tobytes()
