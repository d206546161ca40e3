"""GPU parity: repack, dequant and the decode GEMV / skinny GEMM against the oracle.

Bars: packing and dequant bit-exact; GEMV outputs maxrel <= 1e-3 against the
fp64 reference from the same bytes (the north star's bar; the reference's own
gemv gate is cos > 0.9999999 and maxrel < 1e-4, designs/gemv_q4/compare.py:13-16,
which these kernels also meet and which is asserted too).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu

MAXREL = 1e-3          # north-star bar (fp32 accumulate vs the fp64 reference)
REF_GATE = 1e-4        # the reference gemv's own gate (compare.py:16)


def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.astype(np.float32)).to(torch.bfloat16)


def _cos(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-30))


# --------------------------------------------------------------------------
# packing and dequant: bit-exact
# --------------------------------------------------------------------------

@pytest.mark.parametrize("kind", ["q4_1", "q4_0"])
@pytest.mark.parametrize("n,k", [(64, 32), (128, 512), (256, 4096), (192, 14336)])
def test_repack_bytes_match_oracle(gpu, pkg, oracle, kind, n, k):
    say(f"repack {kind} n={n} k={k}")
    rng = np.random.default_rng(n + k)
    blocks = (oracle.baseline_q4_1_blocks(n, k, rng) if kind == "q4_1"
              else oracle.random_q4_0_blocks_ref(n, k, rng))
    w = pkg.pack_q4_1(blocks, gpu)
    torch.cuda.synchronize()
    assert np.array_equal(w.data.cpu().numpy(), oracle.pack_mx(blocks))


@pytest.mark.parametrize("rs", [1, 2, 4])
def test_repack_pool_matches_oracle(gpu, pkg, oracle, rs):
    say(f"repack_pool rs={rs}")
    rng = np.random.default_rng(rs)
    n, k = 256, 1024
    blocks = oracle.random_q4_1_blocks_ref(n, k, rng)
    pool = oracle.pack_q4_1_pool(blocks, rs)
    w = pkg.pack_q4_1_pool(pool, n, k, rs, gpu)
    torch.cuda.synchronize()
    assert np.array_equal(w.data.cpu().numpy(), oracle.pack_mx(blocks))


@pytest.mark.parametrize("n,k", [(64, 32), (512, 2048), (2048, 512), (4096, 4096)])
def test_dequant_bit_exact(gpu, pkg, oracle, n, k):
    say(f"dequant n={n} k={k}")
    rng = np.random.default_rng(7)
    blocks = oracle.random_q4_1_blocks_ref(n, k, rng)
    w = pkg.dequant(pkg.pack_q4_1(blocks, gpu)).cpu().numpy()
    want = oracle.dequant_q4_1(blocks, bf16_scales=True)
    assert w.tobytes() == want.tobytes()
    if k % 256 == 0 and n % 64 == 0:
        assert w.tobytes() == oracle.dequant_pool(oracle.pack_q4_1_pool(blocks, 2), n, k, 2).tobytes()


def test_dequant_kat_chunks_via_pool(gpu, pkg, oracle):
    """The seed-702 known-answer chunks (test_q4nx_decode_layout.py) through the
    GPU: pool bytes -> mx -> dequant equals the scalar expectation bit for bit."""
    say("dequant seed-702 chunks")
    rng = np.random.default_rng(702)
    count = 4                         # 4 chunks = [64 rows, 512 k] at rs=1? use rs=2 band law
    chunks = rng.integers(0, 256, (count, 5120), dtype=np.uint8)
    meta = oracle.f32_to_bf16(rng.uniform(-2, 2, (count, 512)).astype(np.float32))
    chunks[:, :1024] = meta.view(np.uint8)
    n, k, rs = 64, 512, 2             # per_band = 4 chunks = one band of 64 rows x 512 k
    want = oracle.dequant_pool(chunks.reshape(-1), n, k, rs)
    got = pkg.dequant(pkg.pack_q4_1_pool(chunks.reshape(-1), n, k, rs, gpu)).cpu().numpy()
    assert got.tobytes() == want.tobytes()


def test_empty_inputs(gpu, pkg):
    say("empty")
    blocks = np.zeros((0, 4, 20), np.uint8)
    w = pkg.pack_q4_1(blocks, gpu)
    assert w.nbytes == 0
    assert pkg.dequant(w).shape == (0, 128)


# --------------------------------------------------------------------------
# GEMV / skinny GEMM
# --------------------------------------------------------------------------

@pytest.mark.parametrize("xdt", ["bf16", "f32"])
@pytest.mark.parametrize("n,k", [(64, 32), (64, 256), (1024, 4096), (4096, 4096), (4096, 14336), (14336, 4096)])
def test_gemv_matches_oracle(gpu, pkg, oracle, xdt, n, k):
    say(f"gemv M=1 {xdt} n={n} k={k}")
    rng = np.random.default_rng(n * 7 + k)
    blocks = oracle.baseline_q4_1_blocks(n, k, rng)
    x = rng.standard_normal(k).astype(np.float32)
    if xdt == "bf16":
        xt = _bf16(x)
        xref = xt.to(torch.float32).numpy()
    else:
        xt = torch.from_numpy(x)
        xref = x
    w = pkg.pack_q4_1(blocks, gpu)
    y = pkg.gemv_q4(w, xt.to(gpu)).cpu().numpy()
    ref = oracle.gemv_reference(blocks, xref)[0]
    assert y.shape == (n,)
    assert np.isfinite(y).all()
    mr = oracle.maxrel(y, ref)
    assert mr <= MAXREL, mr
    assert mr < REF_GATE and _cos(y, ref) > 0.9999999, (mr, _cos(y, ref))


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 13, 16, 17, 20, 21, 24])
def test_skinny_gemm_distinct_tokens(gpu, pkg, oracle, M):
    say(f"gemm_q4 M={M}")
    rng = np.random.default_rng(100 + M)
    n, k = 1024, 4096
    blocks = oracle.baseline_q4_1_blocks(n, k, rng)
    X = _bf16(rng.standard_normal((M, k)))
    assert len({X[i].view(torch.int16).numpy().tobytes() for i in range(M)}) == M
    w = pkg.pack_q4_1(blocks, gpu)
    Y = pkg.gemm_q4(w, X.to(gpu)).cpu().numpy()
    ref = oracle.gemv_reference(blocks, X.to(torch.float32).numpy())
    assert Y.shape == (M, n)
    assert oracle.maxrel(Y, ref) <= MAXREL
    # every token row of the batch equals that token run alone, bit for bit
    # (MFMA rows are independent and the epilogue is per token)
    for t in sorted({0, min(15, M - 1), min(16, M - 1), M - 1}):
        y1 = pkg.gemv_q4(w, X[t].to(gpu)).cpu().numpy()
        assert y1.tobytes() == Y[t].tobytes()


@pytest.mark.parametrize("xdt", ["bf16", "f32"])
@pytest.mark.parametrize("n,k", [(6144, 4096), (4096, 14336)])
def test_two_token_blocks_on_plan_shapes(gpu, pkg, oracle, xdt, n, k):
    """M = 17..24 runs two 16-token blocks over one weight stream (block 1 from token 16).
    On an unsplit 16-wave shape (6144 x 4096) and a split one (4096 x 14336, 16 K splits),
    with the residual epilogue: within the bar of the oracle, and every token row equal, bit
    for bit, to that token run alone."""
    M = 23
    say(f"gemm_q4 two token blocks M={M} {n}x{k} {xdt}")
    rng = np.random.default_rng(n + k + M)
    blocks = oracle.baseline_q4_1_blocks(n, k, rng)
    xf = rng.standard_normal((M, k)).astype(np.float32)
    X = _bf16(xf) if xdt == "bf16" else torch.from_numpy(xf)
    res = rng.standard_normal((M, n)).astype(np.float32)
    w = pkg.pack_q4_1(blocks, gpu)
    Y = pkg.gemm_q4(w, X.to(gpu), residual=torch.from_numpy(res).to(gpu)).cpu().numpy()
    ref = oracle.gemv_reference(blocks, X.to(torch.float32).numpy()) + res
    assert oracle.maxrel(Y, ref) <= MAXREL
    for t in (0, 3, 15, 16, 19, 22):
        y1 = pkg.gemm_q4(w, X[t:t + 1].to(gpu), residual=torch.from_numpy(res[t:t + 1]).to(gpu)).cpu().numpy()
        assert y1.tobytes() == Y[t:t + 1].tobytes(), t


@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_onehot_gives_a_weight_column_exactly(gpu, pkg, oracle, xdt):
    """x = e_k: y = W[:, k] bit for bit (gemv_q4/make_test.py --x onehot:K)."""
    say(f"gemv onehot {xdt}")
    rng = np.random.default_rng(21)
    n, k = 256, 1024
    blocks = oracle.baseline_q4_1_blocks(n, k, rng)
    W = oracle.dequant_q4_1(blocks)
    w = pkg.pack_q4_1(blocks, gpu)
    for kk in (0, 33, 1023):
        x = torch.zeros(k, dtype=torch.bfloat16 if xdt == "bf16" else torch.float32)
        x[kk] = 1
        y = pkg.gemv_q4(w, x.to(gpu)).cpu().numpy()
        assert y.tobytes() == W[:, kk].tobytes()


def test_ones_gives_row_sums(gpu, pkg, oracle):
    say("gemv ones")
    rng = np.random.default_rng(22)
    n, k = 512, 2048
    blocks = oracle.baseline_q4_1_blocks(n, k, rng)
    w = pkg.pack_q4_1(blocks, gpu)
    y = pkg.gemv_q4(w, torch.ones(k, dtype=torch.bfloat16, device=gpu)).cpu().numpy()
    ref = oracle.dequant_q4_1(blocks).astype(np.float64).sum(axis=1)
    assert oracle.maxrel(y, ref) < 1e-5


def test_gemv_reference_generator_weights(gpu, pkg, oracle):
    """The reference's own synthetic weights (q4_1_pack.py:70-81, nonzero-mean
    mins) through the pool layout, as gemv_q4/make_test.py builds its fixture."""
    say("gemv reference-generator fixture")
    rng = np.random.default_rng(0)
    n, k, rs = 8192, 2048, 2                       # the reference's qkv region shape
    blocks = oracle.random_q4_1_blocks_ref(n, k, rng)
    pool = oracle.pack_q4_1_pool(blocks, rs)
    x = np.random.default_rng(0).standard_normal(k).astype(np.float32)
    xt = _bf16(x)
    ref = oracle.pool_reference(pool, xt.to(torch.float32).numpy(), n, k, rs)
    w = pkg.pack_q4_1_pool(pool, n, k, rs, gpu)
    y = pkg.gemv_q4(w, xt.to(gpu)).cpu().numpy()
    assert oracle.maxrel(y, ref) < REF_GATE and _cos(y, ref) > 0.9999999


def test_repeated_calls_are_deterministic(gpu, pkg, oracle):
    """The split-K reduction adds partials in split order: same bits every call."""
    say("gemv determinism")
    rng = np.random.default_rng(23)
    n, k = 4096, 14336
    w = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(n, k, rng), gpu)
    x = _bf16(rng.standard_normal(k)).to(gpu)
    first = pkg.gemv_q4(w, x).cpu().numpy()
    for _ in range(5):
        assert pkg.gemv_q4(w, x).cpu().numpy().tobytes() == first.tobytes()


# Every Llama-3-8B decode shape of config 1 but lm_head (q/o, k/v, gate/up, down, the
# fused qkv and gate/up buffers), plus ragged small matrices: the grouped kernel's table
# search crosses every kind of boundary.
GROUP_SHAPES = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (6144, 4096), (64, 4096),
                (128, 256), (28672, 4096)]
_GROUP_CACHE: dict = {}


def _group_weights(oracle, gpu, pkg):
    """Blocks, f64 weights and packed matrices of GROUP_SHAPES, built once per session."""
    if "w" not in _GROUP_CACHE:
        rng = np.random.default_rng(300)
        out = []
        for (n, k) in GROUP_SHAPES:
            blocks = oracle.baseline_q4_1_blocks(n, k, rng)
            out.append((oracle.dequant_q4_1(blocks).astype(np.float64), pkg.pack_q4_1(blocks, gpu)))
        _GROUP_CACHE["w"] = out
    return _GROUP_CACHE["w"]


@pytest.mark.parametrize("xdt", ["bf16", "f32"])
@pytest.mark.parametrize("M", [1, 4, 5, 8, 13, 16])
def test_grouped_gemv(gpu, pkg, oracle, M, xdt):
    """The grouped kernel at every accumulator count (NTL = 1..4) the bench times, against
    the fp64 reference, and each token row equal to that token run alone through the
    single-matrix kernel up to fp32 summation order."""
    say(f"grouped gemv M={M} x={xdt}")
    rng = np.random.default_rng(30 + M)
    items, refs = [], []
    for (W, w) in _group_weights(oracle, gpu, pkg):
        n, k = W.shape
        X = rng.standard_normal((M, k)).astype(np.float32)
        Xt = _bf16(X) if xdt == "bf16" else torch.from_numpy(X)
        y = torch.full((M, n), float("nan"), device=gpu)
        items.append((w, Xt.to(gpu), y))
        refs.append(Xt.to(torch.float64).numpy() @ W.T)
    grp = pkg.GemvGroup(items)
    grp.run()
    torch.cuda.synchronize()
    for (w, X, y), ref in zip(items, refs):
        got = y.cpu().numpy()
        assert np.isfinite(got).all()
        assert oracle.maxrel(got, ref) <= MAXREL, f"{w.shape}"
        assert oracle.maxrel(got, ref) < REF_GATE and _cos(got, ref) > 0.9999999
    # the group agrees with single launches to fp32 summation-order noise
    for (w, X, y) in items:
        single = pkg.gemm_q4(w, X).cpu().numpy()
        assert oracle.maxrel(y.cpu().numpy(), single) < 1e-5
    # a token row does not depend on the other tokens in the launch
    if M > 1:
        w, X, y = items[0]
        lone = torch.full((1, w.n), float("nan"), device=gpu)
        pkg.GemvGroup([(w, X[M - 1:M].contiguous(), lone)]).run()
        torch.cuda.synchronize()
        assert lone.cpu().numpy().tobytes() == y[M - 1:M].cpu().numpy().tobytes()


@pytest.mark.parametrize("M", [2, 4, 8, 12, 16])
def test_grouped_shared_fragment_rows_equal_lone_tokens(gpu, pkg, oracle, M):
    """From M = 2 the grouped sweep shares each token fragment among 2 (M <= 8) or 4 row
    groups of a matrix. Matrices of 3, 5, 1 and 7 row groups put workgroups across matrix
    boundaries and past the end (those take their row groups one at a time). Every token
    row must equal that token run alone (M = 1, the one-group kernel) bit for bit, and the
    fp64 reference to the north-star bar."""
    say(f"grouped gemv, shared fragments, ragged row groups, M={M}")
    rng = np.random.default_rng(700 + M)
    items, refs = [], []
    for n, k in ((192, 256), (320, 512), (64, 128), (448, 256)):
        blocks = oracle.baseline_q4_1_blocks(n, k, rng)
        X = _bf16(rng.standard_normal((M, k)))
        y = torch.full((M, n), float("nan"), device=gpu)
        items.append((pkg.pack_q4_1(blocks, gpu), X.to(gpu), y))
        refs.append(X.to(torch.float64).numpy() @ oracle.dequant_q4_1(blocks).astype(np.float64).T)
    pkg.GemvGroup(items).run()
    torch.cuda.synchronize()
    for (w, X, y), ref in zip(items, refs):
        assert oracle.maxrel(y.cpu().numpy(), ref) <= MAXREL
    for m in range(M):
        lone = [(w, X[m:m + 1].contiguous(), torch.full((1, w.n), float("nan"), device=gpu)) for w, X, _ in items]
        pkg.GemvGroup(lone).run()
        torch.cuda.synchronize()
        for (_, _, y), (_, _, y1) in zip(items, lone):
            assert y1.cpu().numpy().tobytes() == y[m:m + 1].cpu().numpy().tobytes()


def test_rejects_bad_shapes(gpu, pkg, oracle):
    say("gemv bad shapes")
    rng = np.random.default_rng(40)
    w = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(64, 64, rng), gpu)
    with pytest.raises(ValueError):
        pkg.gemm_q4(w, torch.zeros(25, 64, dtype=torch.bfloat16, device=gpu))
    with pytest.raises(ValueError):
        pkg.gemv_q4(w, torch.zeros(96, dtype=torch.bfloat16, device=gpu))


def test_split_calls_share_one_workspace(gpu, pkg, oracle):
    """K-split GEMVs back to back on ONE workspace: 60 calls alternating shapes, token counts
    and operators (plain, residual, SwiGLU), every result bit-identical to the first call of
    its kind and within the bar of the fp64 oracle."""
    say("gemv splits: shared workspace")
    rng = np.random.default_rng(61)
    shapes = [(4096, 4096, 1), (1024, 4096, 3), (4096, 14336, 16), (6144, 4096, 5), (256, 2048, 2)]
    cases = []
    for n, k, M in shapes:
        blocks = oracle.baseline_q4_1_blocks(n, k, rng)
        X = _bf16(rng.standard_normal((M, k)))
        w = pkg.pack_q4_1(blocks, gpu)
        res = torch.from_numpy(rng.standard_normal((M, n)).astype(np.float32)).to(gpu)
        cases.append((w, X.to(gpu), res, oracle.gemv_reference(blocks, X.to(torch.float32).numpy())))
    gate = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(1024, 4096, rng), gpu)
    up = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(1024, 4096, rng), gpu)
    xs = _bf16(rng.standard_normal((2, 4096))).to(gpu)
    need = max([pkg.gemv_workspace_bytes(X.shape[0], w.n, w.k) for w, X, _, _ in cases] +
               [pkg.load_library().q4_gemv_swiglu_workspace_bytes(2, 1024, 4096)])
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    first = {}
    for it in range(60):
        i = it % (len(cases) + 1)
        if i == len(cases):
            got = pkg.swiglu_q4(gate, up, xs, workspace=ws)
        elif (it // (len(cases) + 1)) % 2:            # alternate rounds: residual, plain
            w, X, res, _ = cases[i]
            got = pkg.gemm_q4(w, X, workspace=ws, residual=res)
            i = -1 - i
        else:
            w, X, _, _ = cases[i]
            got = pkg.gemm_q4(w, X, workspace=ws)
        b = got.cpu().numpy().tobytes()
        assert first.setdefault(i, b) == b, f"call {it} ({i}) differs from its first run"
    for i, (w, X, res, ref) in enumerate(cases):
        assert oracle.maxrel(np.frombuffer(first[i], np.float32).reshape(ref.shape), ref) <= MAXREL
        if -1 - i in first:
            r = np.frombuffer(first[-1 - i], np.float32).reshape(ref.shape)
            assert oracle.maxrel(r, ref + res.cpu().numpy()) <= MAXREL
