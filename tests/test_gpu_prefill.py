"""GPU parity of the prefill dequant GEMM against the fp64 oracle.

Bars: precision "fp16" (default) maxrel <= 1e-3 (the north star's bar) against
Y from the same bytes in fp64 over T distinct token activations
(gemm_q4_prefill/make_test.py:82-94); precision "bf16" (the reference's own
bf16 tile, gemm_q4_dequant.h:283-286) is held to the reference's rel_fro <= 5e-3
gate (gemm_q4_prefill/compare.py:26) and to bit-exact agreement with an fp64
product over the bf16-rounded weights to fp32 accumulation noise.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu


def _x(rng, T, K):
    return torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).to(torch.bfloat16)


@pytest.mark.parametrize("T,N,K", [(1, 64, 32), (17, 128, 256), (256, 512, 1024), (300, 1024, 2048),
                                   (512, 2560, 2560), (128, 4096, 14336)])
def test_prefill_fp16_matches_oracle(gpu, pkg, oracle, T, N, K):
    say(f"prefill fp16 T={T} N={N} K={K}")
    rng = np.random.default_rng(T + N + K)
    blocks = oracle.baseline_q4_1_blocks(N, K, rng)
    X = _x(rng, T, K)
    assert len({X[t].view(torch.int16).numpy().tobytes() for t in range(T)}) == T
    w = pkg.pack_q4_1(blocks, gpu)
    Y = pkg.gemm_q4_prefill(w, X.to(gpu)).cpu().numpy()
    ref = oracle.prefill_reference(blocks, X.to(torch.float32).numpy())
    assert Y.shape == (T, N) and np.isfinite(Y).all()
    mr = oracle.maxrel(Y, ref)
    assert mr <= 1e-3, mr


def test_prefill_reference_generator_weights(gpu, pkg, oracle):
    """The reference's own fixture recipe: random_q4_1_blocks (seed 0) packed to
    the pool at rs=2, T distinct tokens, fp64 reference from the pool bytes."""
    say("prefill reference fixture qkv T=256")
    rng = np.random.default_rng(0)
    N, K, T = 2560, 2560, 256
    blocks = oracle.random_q4_1_blocks_ref(N, K, rng)
    pool = oracle.pack_q4_1_pool(blocks, 2)
    X = torch.from_numpy(np.stack([rng.standard_normal(K).astype(np.float32) for _ in range(T)])).to(torch.bfloat16)
    w = pkg.pack_q4_1_pool(pool, N, K, 2, gpu)
    Y = pkg.gemm_q4_prefill(w, X.to(gpu)).cpu().numpy()
    Wd = oracle.dequant_pool(pool, N, K, 2).astype(np.float64)
    ref = (X.to(torch.float32).numpy().astype(np.float64) @ Wd.T).astype(np.float32)
    assert oracle.maxrel(Y, ref) <= 1e-3
    assert oracle.rel_fro(Y, ref) <= 5e-3


def test_prefill_bf16_mode_is_the_reference_tile(gpu, pkg, oracle):
    say("prefill bf16 mode")
    rng = np.random.default_rng(5)
    N, K, T = 512, 2048, 256
    blocks = oracle.baseline_q4_1_blocks(N, K, rng)
    X = _x(rng, T, K)
    w = pkg.pack_q4_1(blocks, gpu)
    Y = pkg.gemm_q4_prefill(w, X.to(gpu), precision="bf16").cpu().numpy()
    Wb = oracle.bf16_round(oracle.dequant_q4_1(blocks)).astype(np.float64)   # RNE_bf16(fl32(q*d+m))
    exact_tile = (X.to(torch.float32).numpy().astype(np.float64) @ Wb.T)
    assert oracle.maxrel(Y, exact_tile) < 1e-5            # fp32 accumulation noise only
    ref = oracle.prefill_reference(blocks, X.to(torch.float32).numpy())
    assert oracle.rel_fro(Y, ref) <= 5e-3                 # the reference's prefill gate


def test_prefill_f32_activations_and_large_values(gpu, pkg, oracle):
    """fp32 X, and a token whose max |x| is far beyond fp16's range: the row
    is scaled by a power of two on the way in and back on the way out."""
    say("prefill f32 + large tokens")
    rng = np.random.default_rng(6)
    N, K, T = 256, 1024, 40
    blocks = oracle.baseline_q4_1_blocks(N, K, rng)
    X = rng.standard_normal((T, K)).astype(np.float32)
    X[3] *= 1e6
    X[7, 5] = 3e5
    w = pkg.pack_q4_1(blocks, gpu)
    Y = pkg.gemm_q4_prefill(w, torch.from_numpy(X).to(gpu)).cpu().numpy()
    ref = oracle.prefill_reference(blocks, X)
    assert np.isfinite(Y).all()
    for t in range(T):
        assert oracle.maxrel(Y[t], ref[t]) <= 1e-3, t


def test_prefill_agrees_with_decode_gemm(gpu, pkg, oracle):
    """Both paths compute the same product; the decode path keeps exact codes."""
    say("prefill vs gemm_q4")
    rng = np.random.default_rng(8)
    N, K, T = 1024, 4096, 16
    w = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(N, K, rng), gpu)
    X = _x(rng, T, K).to(gpu)
    a = pkg.gemm_q4_prefill(w, X).cpu().numpy()
    b = pkg.gemm_q4(w, X).cpu().numpy()
    assert oracle.maxrel(a, b) <= 1e-3


def test_prefill_empty(gpu, pkg, oracle):
    say("prefill empty")
    rng = np.random.default_rng(9)
    w = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(64, 64, rng), gpu)
    Y = pkg.gemm_q4_prefill(w, torch.zeros(0, 64, dtype=torch.bfloat16, device=gpu))
    assert Y.shape == (0, 64)


@pytest.mark.parametrize("T,N,K", [(300, 1024, 2048), (512, 4096, 14336)])
def test_prefill_split_tiles_are_deterministic(gpu, pkg, oracle, T, N, K):
    """Shapes whose output tiles are shared by several workgroups along K (the partial sums
    meet in a fix-up): bit-identical across calls, and within the bar of the fp64 oracle."""
    say(f"prefill split-tile determinism T={T} N={N} K={K}")
    rng = np.random.default_rng(T + 7)
    blocks = oracle.baseline_q4_1_blocks(N, K, rng)
    X = _x(rng, T, K)
    w = pkg.pack_q4_1(blocks, gpu)
    xg = X.to(gpu)
    Y0 = pkg.gemm_q4_prefill(w, xg).cpu()
    for _ in range(2):
        Y1 = pkg.gemm_q4_prefill(w, xg).cpu()
        assert torch.equal(Y0.view(torch.int32), Y1.view(torch.int32))
    if T * N * K <= 1 << 31:
        ref = oracle.prefill_reference(blocks, X.to(torch.float32).numpy())
        assert oracle.maxrel(Y0.numpy(), ref) <= 1e-3


@pytest.mark.parametrize("T,N,K", [(256, 192, 64), (256, 448, 256), (1000, 704, 512)])
def test_prefill_192_row_tiles(gpu, pkg, oracle, T, N, K):
    """Shapes the planner gives 192-row tiles: N = 192 alone (one 192-row tile instead of a
    clamped 256-row one), 448 = 256 + 192 with a 4-way K split, 704 = 2 x 256 + 192 with a
    ragged token count. Same bar as the 256-row tiles."""
    say(f"prefill 192-row tiles T={T} N={N} K={K}")
    rng = np.random.default_rng(T + N + K + 1)
    blocks = oracle.baseline_q4_1_blocks(N, K, rng)
    X = _x(rng, T, K)
    w = pkg.pack_q4_1(blocks, gpu)
    Y = pkg.gemm_q4_prefill(w, X.to(gpu)).cpu().numpy()
    ref = oracle.prefill_reference(blocks, X.to(torch.float32).numpy())
    assert Y.shape == (T, N) and np.isfinite(Y).all()
    assert oracle.maxrel(Y, ref) <= 1e-3


_CFG3: dict = {}


def _cfg3_weights(oracle, gpu, pkg, N, K):
    """Blocks, exact f64 weights, bf16-tile f64 weights and the packed matrix of one
    config-3 projection, built once per session."""
    if (N, K) not in _CFG3:
        rng = np.random.default_rng(N + 2 * K)
        blocks = oracle.baseline_q4_1_blocks(N, K, rng)
        W = oracle.dequant_q4_1(blocks)
        _CFG3[(N, K)] = (W.astype(np.float64), oracle.bf16_round(W).astype(np.float64), pkg.pack_q4_1(blocks, gpu))
    return _CFG3[(N, K)]


@pytest.mark.parametrize("precision", ["fp16", "bf16"])
@pytest.mark.parametrize("T,N,K", [(512, 14336, 4096), (512, 4096, 14336), (2048, 14336, 4096),
                                   (2048, 4096, 14336)])
def test_prefill_config3_shapes(gpu, pkg, oracle, T, N, K, precision):
    """Every config-3 shape the bench times (Llama-3-8B gate/up 4096 -> 14336 and down
    14336 -> 4096 at T = 512 and 2048), in both precisions, on T distinct tokens. Per
    token, 3 tokens from each 256-token tile (gemm_q4_prefill/make_test.py:82-94 checks
    all; these shapes are too large for an fp64 product over every token here):
    fp16 maxrel <= 1e-3 against fp64 of the exact weights; bf16 within fp32 accumulation
    noise of fp64 over the reference's bf16 tile, and rel_fro <= 5e-3 against the exact
    weights (the reference's prefill gate, gemm_q4_prefill/compare.py:26)."""
    say(f"prefill config3 T={T} N={N} K={K} {precision}")
    W, Wb, w = _cfg3_weights(oracle, gpu, pkg, N, K)
    rng = np.random.default_rng(T + N)
    X = _x(rng, T, K)
    Y = pkg.gemm_q4_prefill(w, X.to(gpu), precision=precision).cpu().numpy()
    assert Y.shape == (T, N) and np.isfinite(Y).all()
    toks = np.array([bt * 256 + o for bt in range(T // 256) for o in (0, 131, 255)])
    Xs = X[toks].to(torch.float64).numpy()
    ref = Xs @ W.T
    if precision == "fp16":
        for i, t in enumerate(toks):
            assert oracle.maxrel(Y[t], ref[i]) <= 1e-3, int(t)
    else:
        tile = Xs @ Wb.T
        for i, t in enumerate(toks):
            assert oracle.maxrel(Y[t], tile[i]) < 1e-5, int(t)
        assert oracle.rel_fro(Y[toks], ref) <= 5e-3


def _wide_range_blocks(oracle, rng, N, K, lo_exp=-6.0, hi_exp=-2.0):
    """Q4_1 blocks whose rows have d ~ 10^U(lo_exp, hi_exp) (one decade draw per row, a
    +-50 % spread per block), m = -8 d U(0.9, 1.1), codes uniform; d and m rounded to fp16
    as GGUF stores them (below 2^-14 they are fp16 subnormals, kept as stored)."""
    nb = K // 32
    dec = 10.0 ** rng.uniform(lo_exp, hi_exp, (N, 1))
    d = (dec * rng.uniform(0.5, 1.5, (N, nb))).astype(np.float16)
    m = (-8.0 * d.astype(np.float32) * rng.uniform(0.9, 1.1, (N, nb))).astype(np.float16)
    q = rng.integers(0, 16, (N, nb, 32), dtype=np.uint8)
    return oracle._assemble_q4_1(d, m, q)


@pytest.mark.parametrize("xdt", ["bf16", "f32"])
@pytest.mark.parametrize("T,N,K", [(300, 512, 1024), (64, 256, 2080)])
def test_prefill_fp16_range_per_row(gpu, pkg, oracle, T, N, K, xdt):
    """fp16's exponent range costs nothing: weight rows with d from 1e-6 (fp16 subnormals) to
    ~5e3 (weights past fp16's 65504) and token rows from ~1e-6 to ~1e5 in magnitude, every
    token row and every weight row held to maxrel <= 1e-3 against the fp64 oracle on its own
    (per row, the bar the tiny rows would miss, and the large ones overflow, without their
    power-of-two scaling). K = 2080 takes the generic kernel (K % 64 != 0), K = 1024 the
    pipelined one."""
    say(f"prefill fp16 range T={T} N={N} K={K} {xdt}")
    rng = np.random.default_rng(T + N + K + (xdt == "f32"))
    blocks = _wide_range_blocks(oracle, rng, N, K, -6.0, 3.5)
    mag = 10.0 ** rng.uniform(-6.0, 5.0, (T, 1))
    mag[0], mag[1] = 1e-6, 1e5
    X = (rng.standard_normal((T, K)) * mag).astype(np.float32)
    Xt = torch.from_numpy(X).to(torch.bfloat16) if xdt == "bf16" else torch.from_numpy(X)
    w = pkg.pack_q4_1(blocks, gpu)
    Y = pkg.gemm_q4_prefill(w, Xt.to(gpu)).cpu().numpy()
    ref = oracle.prefill_reference(blocks, Xt.to(torch.float32).numpy())
    assert np.isfinite(Y).all()
    for t in range(T):
        assert oracle.maxrel(Y[t], ref[t]) <= 1e-3, f"token row {t} (|x| ~ {float(mag[t, 0]):.1e})"
    for n in range(N):
        assert oracle.maxrel(Y[:, n], ref[:, n]) <= 1e-3, f"weight row {n}"


def test_prefill_fp16_range_scaling_is_exact_on_powers_of_two(gpu, pkg, oracle):
    """Scaling a token row by 2^40 or 2^-40 scales its output by exactly that (the row's
    exponent absorbs it), bit for bit."""
    say("prefill fp16 range: power-of-two invariance")
    rng = np.random.default_rng(41)
    N, K, T = 256, 512, 16
    blocks = _wide_range_blocks(oracle, rng, N, K)
    X = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).to(torch.bfloat16)
    w = pkg.pack_q4_1(blocks, gpu)
    base = pkg.gemm_q4_prefill(w, X.to(gpu))
    for p in (40, -40):
        got = pkg.gemm_q4_prefill(w, (X.to(torch.float32) * 2.0 ** p).to(torch.bfloat16).to(gpu))
        assert torch.equal(got, base * 2.0 ** p), p


def _prefill_scales_numpy(oracle, blocks):
    """(wexp int32[N], fp16 scale words uint32[N/64, KB, 64]) of a matrix, restated on the CPU:
    e_n puts max_kb (15 |d| + |m|) (f32, bf16 d and m) in [2^14, 2^15) after 2^-e_n; each word
    is fp16(d 2^-e) << 16 | fp16(m 2^-e) at (row % 16) * 4 + (row % 64) / 16 of its tile."""
    b = np.asarray(blocks)
    N, KB, _ = b.shape
    d = oracle.bf16_to_f32(oracle.f32_to_bf16(np.ascontiguousarray(b[..., 0:2]).view(np.float16)[..., 0].astype(np.float32)))
    m = oracle.bf16_to_f32(oracle.f32_to_bf16(np.ascontiguousarray(b[..., 2:4]).view(np.float16)[..., 0].astype(np.float32)))
    bound = (np.float32(15) * np.abs(d) + np.abs(m)).astype(np.float32).max(axis=1)
    _, ex = np.frexp(bound)
    e = np.where((bound > 0) & (bound <= 3.0e38), ex - 15, 0).astype(np.int32)
    dh = np.ldexp(d, -e[:, None]).astype(np.float16).view(np.uint16).astype(np.uint32)
    mh = np.ldexp(m, -e[:, None]).astype(np.float16).view(np.uint16).astype(np.uint32)
    words = (dh << 16) | mh                                           # [N, KB]
    rows = np.arange(N)
    slot = (rows % 16) * 4 + (rows % 64) // 16
    plane = np.zeros((N // 64, KB, 64), np.uint32)
    plane[rows // 64, :, slot] = words
    return e, plane


def test_prefill_scales_match_numpy_and_paths_agree(gpu, pkg, oracle):
    """q4_prefill_scales bit for bit against a numpy restatement (over wide-range weights,
    fp16 subnormal d included), and the per-call path (q4_gemm_prefill) equal to the cached
    one (q4_gemm_prefill_scaled) bit for bit."""
    say("prefill scales")
    rng = np.random.default_rng(77)
    N, K, T = 320, 1536, 100
    blocks = _wide_range_blocks(oracle, rng, N, K, -6.0, 3.5)
    w = pkg.pack_q4_1(blocks, gpu)
    sc = pkg.prefill_scales(w).cpu().numpy()
    e, plane = _prefill_scales_numpy(oracle, blocks)
    assert np.array_equal(sc[:N * 4].view(np.int32), e)
    off = (N * 4 + 255) // 256 * 256
    got = sc[off:off + plane.size * 4].view(np.uint32).reshape(plane.shape)
    assert np.array_equal(got, plane)
    X = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).to(torch.bfloat16).to(gpu)
    lib = pkg.load_library()
    y_call = torch.empty(T, N, device=gpu)
    ws = torch.empty(lib.q4_gemm_prefill_workspace_bytes(T, N, K), dtype=torch.uint8, device=gpu)
    st = torch.cuda.current_stream(gpu).cuda_stream
    assert lib.q4_gemm_prefill(w.data.data_ptr(), X.data_ptr(), 1, y_call.data_ptr(), T, N, K, 0, ws.data_ptr(),
                               ws.numel(), st) == 0
    y_cached = pkg.gemm_q4_prefill(w, X)
    assert torch.equal(y_call, y_cached)


@pytest.mark.parametrize("T,N,K,xdt,precision", [
    (300, 256, 512, "bf16", "fp16"),       # one token tile + a ragged one, unsplit
    (300, 256, 512, "f32", "fp16"),        # value and remainder planes
    (512, 4096, 14336, "bf16", "fp16"),    # config 3's down at T = 512: K split and reduce
    (200, 192, 96, "bf16", "fp16"),        # K % 64 != 0: rows [T][K], the generic kernel
    (300, 256, 512, "f32", "bf16"),        # the reference tile
])
def test_prefill_prepared_activations_equal_the_one_call_path(gpu, pkg, oracle, T, N, K, xdt, precision):
    """Activations prepared once (q4_prefill_prepare) and read by two projections give the
    bits the one-call path gives for each."""
    say(f"prefill prepared T={T} N={N} K={K} {xdt} {precision}")
    rng = np.random.default_rng(T + N + K)
    w1 = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(N, K, rng), gpu)
    w2 = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(N, K, rng), gpu)
    xf = rng.standard_normal((T, K)).astype(np.float32)
    x = (torch.from_numpy(xf).to(torch.bfloat16) if xdt == "bf16" else torch.from_numpy(xf)).to(gpu)
    prep = pkg.prefill_prepare(x, precision)
    for w in (w1, w2):
        a = pkg.gemm_q4_prefill(w, prep).cpu().numpy()
        b = pkg.gemm_q4_prefill(w, x, precision=precision).cpu().numpy()
        assert a.tobytes() == b.tobytes()
