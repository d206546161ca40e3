"""Pin the CPU oracle (oracle/q4_oracle.py) independently of its own formulas.

Each check below is chosen so a plausible mistake (swapped nibble halves, a
transposed index, a dropped min term, truncation instead of RNE) fails it:

* the seed-702 scalar-loop known-answer test of
  specs/open-engine/tests/test_q4nx_decode_layout.py:8-30 (restated);
* q4_1_pack._selftest's identity (q4_1_pack.py:194-209): pack -> dequant of
  the pool bytes equals the GGUF dequant with bf16 scales exactly, Q4_1 and Q4_0;
* torch's own fp16/f32 -> bf16 round-to-nearest-even;
* brute-force scalar loops on tiny shapes; one-hot and all-ones activations;
* the exact Q4_0 identity m = -8 d (test_quant_q4_0.py's transcode rule).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch


# --------------------------------------------------------------------------
# bf16 narrowing
# --------------------------------------------------------------------------

def test_f32_to_bf16_matches_torch_rne(oracle):
    rng = np.random.default_rng(1)
    f = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * np.float32(10.0) ** rng.integers(-6, 6, 100000),
        # exact ties: bf16 value + half an ulp, both parities of the kept LSB
        (np.arange(1, 2001, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
        np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 6.1e-5, 1e-4], np.float32),
    ])
    want = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.f32_to_bf16(f), want)


def test_fp16_to_bf16_of_every_finite_half(oracle):
    h = np.arange(0, 1 << 16, dtype=np.uint16).view(np.float16)
    h = h[np.isfinite(h)]
    want = torch.from_numpy(h.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.f32_to_bf16(h.astype(np.float32)), want)
    # and the widening back is exact
    assert np.array_equal(oracle.bf16_to_f32(want), torch.from_numpy(want.view(np.int16)).view(torch.bfloat16)
                          .to(torch.float32).numpy())


def test_planted_truncation_fails_rne_check(oracle):
    """A truncating narrowing (a plausible mistake) disagrees with RNE."""
    f = np.array([1.00390625 + 2 ** -9], np.float32)   # above a tie: RNE rounds up
    trunc = (f.view(np.uint32) >> 16).astype(np.uint16)
    assert not np.array_equal(trunc, oracle.f32_to_bf16(f))


# --------------------------------------------------------------------------
# GGUF blocks
# --------------------------------------------------------------------------

def _scalar_unpack(blocks):
    n, nb, w = blocks.shape
    d = np.zeros((n, nb), np.float32)
    m = np.zeros((n, nb), np.float32)
    q = np.zeros((n, nb * 32), np.uint8)
    for r in range(n):
        for b in range(nb):
            blk = blocks[r, b]
            d[r, b] = np.frombuffer(blk[0:2].tobytes(), np.float16)[0]
            if w == 20:
                m[r, b] = np.frombuffer(blk[2:4].tobytes(), np.float16)[0]
                qs = blk[4:20]
            else:
                m[r, b] = -8.0 * d[r, b]
                qs = blk[2:18]
            for j in range(16):
                q[r, b * 32 + j] = qs[j] & 0xF          # value j: low nibble of byte j
                q[r, b * 32 + j + 16] = qs[j] >> 4      # value j+16: high nibble
    return d, m, q


@pytest.mark.parametrize("kind", ["q4_1", "q4_0"])
def test_unpack_blocks_matches_scalar_loop(oracle, kind):
    rng = np.random.default_rng(3)
    make = oracle.random_q4_1_blocks_ref if kind == "q4_1" else oracle.random_q4_0_blocks_ref
    blocks = make(5, 96, rng)
    d, m, q = oracle.unpack_q4_1_blocks(blocks)
    sd, sm, sq = _scalar_unpack(blocks)
    assert np.array_equal(d, sd) and np.array_equal(m, sm) and np.array_equal(q, sq)


def test_baseline_distribution(oracle):
    rng = np.random.default_rng(4)
    blocks = oracle.baseline_q4_1_blocks(64, 4096, rng)
    d, m, q = oracle.unpack_q4_1_blocks(blocks)
    assert d.min() >= 9.9e-5 and d.max() < 0.02
    ratio = -m / (8 * d)
    assert ratio.min() > 0.899 and ratio.max() < 1.101
    assert q.min() == 0 and q.max() == 15
    assert abs(q.mean() - 7.5) < 0.05


def test_q4_0_reads_as_min_minus_8d(oracle):
    rng = np.random.default_rng(5)
    b0 = oracle.random_q4_0_blocks_ref(4, 64, rng)
    d, m, q = oracle.unpack_q4_1_blocks(b0)
    assert np.array_equal(m, -8 * d)
    # value rule (q - 8) * d, exactly, in f32 and after bf16 narrowing of d
    w = oracle.dequant_q4_1(b0, bf16_scales=False)
    assert np.array_equal(w, (q.astype(np.float32) - 8) * np.repeat(d, 32, axis=1))
    wb = oracle.dequant_q4_1(b0, bf16_scales=True)
    db = oracle.bf16_round(d)
    assert np.array_equal(wb, (q.astype(np.float32) - 8) * np.repeat(db, 32, axis=1))
    # the 18 -> 20 byte transcode is exact
    assert np.array_equal(oracle.dequant_q4_1(oracle.q4_0_to_q4_1(b0), False), w)


# --------------------------------------------------------------------------
# pool layout (q4_1_pack.py) and the chunk dequant (q4nx.py)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("count", [0, 1, 3, 33])
@pytest.mark.parametrize("strided", [False, True])
def test_dq_chunks_known_answer_seed702(oracle, count, strided):
    """Restates test_q4nx_decode_layout.py:8-30 (seed 702, scalar expected)."""
    rng = np.random.default_rng(702)
    storage = rng.integers(0, 256, (count * 2, 5120), dtype=np.uint8)
    chunks = storage[::2] if strided else storage[:count].copy()
    meta = oracle.f32_to_bf16(rng.uniform(-2, 2, (count, 512)).astype(np.float32))
    chunks[:, :1024] = meta.view(np.uint8)
    expected = np.empty((count, 32, 8, 32), dtype=np.float32)
    coeff = oracle.bf16_to_f32(meta)
    for c in range(count):
        for row in range(32):
            for block in range(8):
                d, m = coeff[c, block * 32 + row], coeff[c, 256 + block * 32 + row]
                for lane in range(32):
                    nibble = ((row // 16) * 8 + block) * 32 * 16 + lane * 16 + row % 16
                    packed = int(chunks[c, 1024 + nibble // 2])
                    q = np.float32((packed >> (4 * (nibble % 2))) & 15)
                    expected[c, row, block, lane] = q * d + m
    actual = oracle.dq_chunks_q4_1(chunks)
    assert actual.tobytes() == expected.tobytes()
    assert actual.flags.c_contiguous
    # the benchmark harness's frozen oracle is byte-identical (benchmark-q4-decode.py:50)
    if count:
        assert oracle.legacy_decode(np.ascontiguousarray(chunks)).tobytes() == expected.tobytes()


def test_planted_nibble_swap_fails_known_answer(oracle):
    """Swapping low/high nibble halves in the chunk decode must fail the KAT."""
    rng = np.random.default_rng(702)
    chunks = rng.integers(0, 256, (1, 5120), dtype=np.uint8)
    chunks[:, :1024] = oracle.f32_to_bf16(rng.uniform(-2, 2, (1, 512)).astype(np.float32)).view(np.uint8)
    good = oracle.dq_chunks_q4_1(chunks)
    swapped = chunks.copy()
    swapped[:, 1024:] = (chunks[:, 1024:] >> 4) | ((chunks[:, 1024:] & 0xF) << 4)
    assert not np.array_equal(oracle.dq_chunks_q4_1(swapped), good)


@pytest.mark.parametrize("kind", ["q4_1", "q4_0"])
@pytest.mark.parametrize("n,k,rs", [(512, 2048, 2), (2048, 512, 2), (512, 2048, 4)])
def test_pool_selftest_identity(oracle, kind, n, k, rs):
    """q4_1_pack._selftest (:194-209): pool bytes dequant == GGUF dequant with bf16 scales."""
    rng = np.random.default_rng(0)
    make = oracle.random_q4_1_blocks_ref if kind == "q4_1" else oracle.random_q4_0_blocks_ref
    blocks = make(n, k, rng)
    pool = oracle.pack_q4_1_pool(blocks, rs)
    assert pool.size == n * k * 5 // 8
    want = oracle.dequant_q4_1(blocks, bf16_scales=True)
    assert np.array_equal(oracle.dequant_pool(pool, n, k, rs), want)
    # and bf16 narrowing is the only loss against the GGUF bytes
    rel = np.abs(want - oracle.dequant_q4_1(blocks, bf16_scales=False)).max() / np.abs(want).max()
    assert 0 < rel < 1e-2


def test_pool_chunk_bytes_match_scalar_layout(oracle):
    """Each pool byte placed by the docstring's index formula (q4_1_pack.py:16-34)."""
    rng = np.random.default_rng(7)
    n, k, rs = 128, 512, 2
    blocks = oracle.random_q4_1_blocks_ref(n, k, rng)
    d, m, q = oracle.unpack_q4_1_blocks(blocks)
    d16, m16 = oracle.f32_to_bf16(d), oracle.f32_to_bf16(m)
    pool = oracle.pack_q4_1_pool(blocks, rs).reshape(-1, 5120)
    per_band = rs * k // 256
    for c in range(pool.shape[0]):
        band, ci = divmod(c, per_band)
        r0, c0 = 32 * rs * band + 32 * (ci % rs), 256 * (ci // rs)
        ch = pool[c]
        dd = ch[0:512].view(np.uint16)
        mm = ch[512:1024].view(np.uint16)
        for r in range(32):
            for kb in range(8):
                assert dd[kb * 32 + r] == d16[r0 + r, c0 // 32 + kb]
                assert mm[kb * 32 + r] == m16[r0 + r, c0 // 32 + kb]
        for r in (0, 5, 16, 31):
            for kk in (0, 1, 31, 32, 255):
                p = (r // 16) * 4096 + kk * 16 + r % 16
                v = (ch[1024 + p // 2] >> (4 * (p % 2))) & 0xF
                assert v == q[r0 + r, c0 + kk]


def test_dequant_chunk_agrees_with_dq_chunks(oracle):
    rng = np.random.default_rng(8)
    blocks = oracle.random_q4_1_blocks_ref(64, 256, rng)
    pool = oracle.pack_q4_1_pool(blocks, 2).reshape(-1, 5120)
    for c in range(pool.shape[0]):
        a = oracle.dequant_chunk(pool[c])
        b = oracle.dq_chunks_q4_1(pool[c:c + 1]).reshape(32, 256)
        assert a.tobytes() == b.tobytes()


# --------------------------------------------------------------------------
# GEMV references
# --------------------------------------------------------------------------

def test_pool_reference_brute_force(oracle):
    rng = np.random.default_rng(9)
    n, k = 64, 256
    blocks = oracle.random_q4_1_blocks_ref(n, k, rng)
    pool = oracle.pack_q4_1_pool(blocks, 2)
    x = rng.standard_normal(k).astype(np.float32)
    d, m, q = oracle.unpack_q4_1_blocks(blocks)
    d, m = oracle.bf16_round(d), oracle.bf16_round(m)
    y = np.zeros(n)
    for r in range(n):
        s = 0.0
        for kk in range(k):
            s += float(np.float32(np.float32(q[r, kk]) * d[r, kk // 32] + m[r, kk // 32])) * float(x[kk])
        y[r] = s
    assert np.allclose(oracle.pool_reference(pool, x, n, k, 2), y.astype(np.float32), rtol=1e-6, atol=1e-6)
    assert np.allclose(oracle.gemv_reference(blocks, x)[0], y.astype(np.float32), rtol=1e-6, atol=1e-6)


def test_gemv_reference_onehot_and_ones(oracle):
    rng = np.random.default_rng(10)
    blocks = oracle.baseline_q4_1_blocks(128, 512, rng)
    w = oracle.dequant_q4_1(blocks)
    for kk in (0, 31, 32, 511):
        x = np.zeros(512, np.float32)
        x[kk] = 1
        assert np.array_equal(oracle.gemv_reference(blocks, x)[0], w[:, kk])
    ones = oracle.gemv_reference(blocks, np.ones(512, np.float32))[0]
    assert np.allclose(ones, w.astype(np.float64).sum(axis=1), rtol=1e-6)


def test_gemv_reference_dropped_min_is_caught(oracle):
    """A GEMV that forgets the min term is far outside the 1e-3 bar."""
    rng = np.random.default_rng(11)
    blocks = oracle.baseline_q4_1_blocks(64, 1024, rng)
    x = rng.standard_normal(1024).astype(np.float32)
    d, m, q = oracle.unpack_q4_1_blocks(blocks)
    wrong = (q.astype(np.float64) * np.repeat(oracle.bf16_round(d), 32, axis=1)) @ x
    assert oracle.maxrel(wrong, oracle.gemv_reference(blocks, x)[0]) > 1e-1


def test_maxrel_definition(oracle):
    """maxrel = max|got-ref| / max|ref| (designs/gemv_q4/compare.py:13)."""
    assert oracle.maxrel(np.array([1.0, 2.0]), np.array([1.0, 4.0])) == pytest.approx(0.5)
    assert oracle.rel_fro(np.array([3.0, 4.0]), np.array([0.0, 0.0])) > 1e20


# --------------------------------------------------------------------------
# MoE routing and expert math
# --------------------------------------------------------------------------

def test_softmax_topk_brute_force(oracle):
    rng = np.random.default_rng(12)
    lg = rng.standard_normal((16, 128))
    ids, w = oracle.softmax_topk(lg, 8)
    for t in range(16):
        p = np.exp(lg[t] - lg[t].max())
        p /= p.sum()
        order = sorted(range(128), key=lambda e: (-p[e], e))[:8]     # stable: lower id wins ties
        assert list(ids[t]) == order
        assert np.allclose(w[t], p[order] / p[order].sum(), rtol=1e-6)
    assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6)


def test_softmax_topk_tie_rule(oracle):
    ids, _ = oracle.softmax_topk(np.zeros((1, 10)), 3)
    assert list(ids[0]) == [0, 1, 2]


def test_moe_reference_brute_force(oracle):
    rng = np.random.default_rng(13)
    E, H, F, T, K = 6, 64, 64, 3, 2
    gates = [oracle.dequant_q4_1(oracle.baseline_q4_1_blocks(F, H, rng)) for _ in range(E)]
    ups = [oracle.dequant_q4_1(oracle.baseline_q4_1_blocks(F, H, rng)) for _ in range(E)]
    downs = [oracle.dequant_q4_1(oracle.baseline_q4_1_blocks(H, F, rng)) for _ in range(E)]
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids, w = oracle.softmax_topk(rng.standard_normal((T, E)), K)
    got = oracle.moe_reference(gates, ups, downs, x, ids, w)
    want = np.zeros((T, H))
    for t in range(T):
        for j in range(K):
            e = ids[t, j]
            g = gates[e].astype(np.float64) @ x[t]
            u = ups[e].astype(np.float64) @ x[t]
            h = g / (1 + np.exp(-g)) * u
            want[t] += w[t, j] * (downs[e].astype(np.float64) @ h)
    assert np.allclose(got, want.astype(np.float32), rtol=1e-5, atol=1e-7)


# --------------------------------------------------------------------------
# the MI355X layout's oracle
# --------------------------------------------------------------------------

@pytest.mark.parametrize("kind", ["q4_1", "q4_0"])
def test_mx_round_trip(oracle, kind):
    rng = np.random.default_rng(14)
    make = oracle.baseline_q4_1_blocks if kind == "q4_1" else oracle.random_q4_0_blocks_ref
    blocks = make(192, 320, rng)
    packed = oracle.pack_mx(blocks)
    assert packed.size == oracle.mx_bytes(192, 320) == 192 * 320 * 5 // 8
    d16, m16, q = oracle.unpack_mx(packed, 192, 320)
    d, m, q0 = oracle.unpack_q4_1_blocks(blocks)
    assert np.array_equal(q, q0)
    assert np.array_equal(d16, oracle.f32_to_bf16(d)) and np.array_equal(m16, oracle.f32_to_bf16(m))
    assert np.array_equal(oracle.dequant_mx(packed, 192, 320), oracle.dequant_q4_1(blocks))


def test_mx_fp16_scales_keep_ggufs_scales(oracle):
    """The exact-scale mode: the scale word carries GGUF's fp16 d and m bits unchanged, and
    its dequant equals the f32-scale unpack (q4_1_pack.py:104-109 with f32 scales) -- pinned
    by a scalar loop in Python floats, each product rounded once to f32 (q d is exact) -- and
    differs from the bf16 mode on scales bf16 cannot hold."""
    rng = np.random.default_rng(17)
    n, k = 128, 96
    blocks = oracle.baseline_q4_1_blocks(n, k, rng)
    p = oracle.pack_mx(blocks, fp16_scales=True)
    d16, m16, q = oracle.unpack_mx(p, n, k)
    assert np.array_equal(d16, np.ascontiguousarray(blocks[..., 0:2]).view(np.uint16).reshape(n, k // 32))
    assert np.array_equal(m16, np.ascontiguousarray(blocks[..., 2:4]).view(np.uint16).reshape(n, k // 32))
    w = oracle.dequant_mx(p, n, k, fp16_scales=True)
    assert np.array_equal(w, oracle.dequant_q4_1(blocks, bf16_scales=False))
    for (row, kk) in [(0, 0), (5, 31), (64, 40), (127, 95), (77, 63)]:
        b = blocks[row, kk // 32]
        d = float(np.frombuffer(bytes(b[0:2]), np.float16)[0])
        m = float(np.frombuffer(bytes(b[2:4]), np.float16)[0])
        j = kk % 32
        code = (b[4 + j] & 0xF) if j < 16 else (b[4 + j - 16] >> 4)
        assert w[row, kk] == np.float32(code * d + m)
    assert not np.array_equal(w, oracle.dequant_q4_1(blocks))       # the bf16 mode's values differ
    with pytest.raises(ValueError):
        oracle.pack_mx(oracle.random_q4_0_blocks_ref(64, 32, rng), fp16_scales=True)


def test_mx_byte_positions_scalar(oracle):
    """Spot-check the layout formula: tile (g, kb), codes dword (lane, r), scales."""
    rng = np.random.default_rng(15)
    n, k = 128, 96
    blocks = oracle.baseline_q4_1_blocks(n, k, rng)
    d, m, q = oracle.unpack_q4_1_blocks(blocks)
    d16, m16 = oracle.f32_to_bf16(d), oracle.f32_to_bf16(m)
    p = oracle.pack_mx(blocks)
    KB = k // 32
    for (row, kk) in [(0, 0), (1, 7), (17, 33), (63, 95), (64, 8), (127, 64), (90, 50)]:
        g, kb = row // 64, kk // 32
        i = row % 64
        r, i16 = i // 16, i % 16
        kg, e = (kk % 32) // 8, kk % 8
        tile = (g * KB + kb) * 1280
        word = int(p[tile + (kg * 16 + i16) * 16 + r * 4: tile + (kg * 16 + i16) * 16 + r * 4 + 4].view(np.uint32)[0])
        assert (word >> (16 * (e % 2) + 4 * (e // 2))) & 0xF == q[row, kk]
        sw = int(p[tile + 1024 + i16 * 16 + r * 4: tile + 1024 + i16 * 16 + r * 4 + 4].view(np.uint32)[0])
        assert sw >> 16 == d16[row, kb] and sw & 0xFFFF == m16[row, kb]


@pytest.mark.parametrize("rs", [1, 2, 4])
def test_pool_to_mx_is_exact(oracle, rs):
    rng = np.random.default_rng(16)
    blocks = oracle.random_q4_1_blocks_ref(256, 512, rng)
    pool = oracle.pack_q4_1_pool(blocks, rs)
    d16, m16, q = oracle.pool_to_blocks(pool, 256, 512, rs)
    assert np.array_equal(oracle.pack_mx_from_parts(d16, m16, q), oracle.pack_mx(blocks))
