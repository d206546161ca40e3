"""The Q4_0-native oracle (no GPU): the reference's 4608 B chunk and the mx0 layout.

Pins: the 4608 B chunk is the 5120 B chunk (pinned by the reference's KAT and pack ->
dequant identity in test_oracle.py) without its m plane, and that m plane is exactly
bf16(-8 d), so nothing is lost (q4_1_pack.py:87-88, :145-152); mx0's byte placement is
checked by a scalar loop over the layout's own definition on a tiny matrix, and its values
equal the reference dequant of the same Q4_0 blocks (dequant_q4_1 with bf16 scales) and
the mx layout's of pack_mx (itself pinned in test_oracle.py)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import q4_oracle as O


@pytest.mark.parametrize("n,k,rs", [(64, 256, 1), (128, 512, 2), (128, 256, 4)])
def test_native_chunk_is_the_pool_chunk_without_its_m_plane(n, k, rs):
    rng = np.random.default_rng(n + k + rs)
    b = O.random_q4_0_blocks_ref(n, k, rng)
    full = O.pack_q4_1_pool(b, rs).reshape(-1, O.CH)
    nat = O.pack_q4_0_native_pool(b, rs).reshape(-1, O.CH_Q4_0)
    assert nat.shape[0] == full.shape[0] == (n // 32) * (k // 256)
    assert np.array_equal(nat[:, :512], full[:, :512])
    assert np.array_equal(nat[:, 512:], full[:, 1024:])
    d = O.bf16_to_f32(np.ascontiguousarray(full[:, :512]).view(np.uint16))
    m = O.bf16_to_f32(np.ascontiguousarray(full[:, 512:1024]).view(np.uint16))
    assert np.array_equal(m, np.float32(-8.0) * d)          # the dropped plane is implied


def test_mx0_byte_placement_scalar_loop():
    rng = np.random.default_rng(7)
    n, k = 128, 64
    b = O.random_q4_0_blocks_ref(n, k, rng)
    p = O.pack_mx0(b)
    assert p.size == O.mx0_bytes(n, k) == (n // 64) * (k // 32) * 1152
    d, _, q = O.unpack_q4_1_blocks(b)
    d16 = O.f32_to_bf16(d)
    KB = k // 32
    for row in range(n):
        g, i = divmod(row, 64)
        r, i16 = divmod(i, 16)
        for kb in range(KB):
            t = (g * KB + kb) * 1152
            assert int(p[t + 1024 + i16 * 8 + r * 2]) | (int(p[t + 1024 + i16 * 8 + r * 2 + 1]) << 8) == int(d16[row, kb])
            for kg in range(4):
                w = int.from_bytes(p[t + (kg * 16 + i16) * 16 + r * 4: t + (kg * 16 + i16) * 16 + r * 4 + 4].tobytes(),
                                   "little")
                for e in range(8):
                    assert (w >> (16 * (e & 1) + 4 * (e >> 1))) & 0xF == q[row, kb * 32 + kg * 8 + e]


@pytest.mark.parametrize("n,k", [(64, 32), (192, 1024)])
def test_mx0_values_equal_the_reference_dequant(n, k):
    rng = np.random.default_rng(n * k)
    b = O.random_q4_0_blocks_ref(n, k, rng)
    p = O.pack_mx0(b)
    d16, q = O.unpack_mx0(p, n, k)
    d, _, q_ref = O.unpack_q4_1_blocks(b)
    assert np.array_equal(q, q_ref) and np.array_equal(d16, O.f32_to_bf16(d))
    w = O.dequant_mx0(p, n, k)
    assert np.array_equal(w, O.dequant_q4_1(b))
    assert np.array_equal(w, O.dequant_mx(O.pack_mx(b), n, k))


def test_planted_mistake_in_the_min_is_caught():
    """Plant m = -7 d instead of -8 d: the value check above fails."""
    rng = np.random.default_rng(3)
    b = O.random_q4_0_blocks_ref(64, 64, rng)
    d16, q = O.unpack_mx0(O.pack_mx0(b), 64, 64)
    d = np.repeat(O.bf16_to_f32(d16), 32, axis=1)
    wrong = q.astype(np.float32) * d + np.float32(-7.0) * d
    assert not np.array_equal(wrong, O.dequant_q4_1(b))
