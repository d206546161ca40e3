"""GPU parity of the fused epilogues either side of the GEMV:

* q4_gemv_swiglu: h = silu(gate x) * (up x) -- f32 out maxrel <= 1e-3 against fp64; bf16
  out against bf16(fp64) under the reference's silu_mul bars (designs/silu_mul/compare.py:
  maxrel < 8e-3, cos > 0.999999, < 5 % bf16 mismatches) and within one bf16 rounding;
* q4_gemv_residual: y = residual + W x, maxrel <= 1e-3, in place equal to out of place;
* q4_rmsnorm_add: y = x + add bit-exact; xn against fp64 under the reference's ln bars
  (designs/ln/compare.py: maxrel < 8e-3, cos > 0.999999, < 5 % mismatches) and within
  one bf16 rounding.
Shapes cover K-split (small F / N) and unsplit launches, M = 1..16, bf16 and f32 x."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu

MAXREL = 1e-3


def _bf16_bits_to_f64(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.float32).cpu().numpy().astype(np.float64)


def _ref_bf16(ref64: np.ndarray) -> np.ndarray:
    return torch.from_numpy(ref64.astype(np.float32)).to(torch.bfloat16).to(torch.float64).numpy()


def _bf16_bars(got: np.ndarray, ref64: np.ndarray):
    rb = _ref_bf16(ref64)
    rel = np.abs(got - rb).max() / (np.abs(rb).max() + 1e-30)
    cos = float(got.ravel() @ rb.ravel() / (np.linalg.norm(got) * np.linalg.norm(rb) + 1e-30))
    nd = int((got != rb).sum())
    assert rel < 8e-3 and cos > 0.999999 and nd < got.size // 20, (rel, cos, nd)


def _xs(rng, M, K, xdt):
    x = rng.standard_normal((M, K)).astype(np.float32)
    if xdt == "bf16":
        xt = torch.from_numpy(x).to(torch.bfloat16)
        return xt, xt.to(torch.float32).numpy()
    return torch.from_numpy(x), x


@pytest.mark.parametrize("xdt", ["bf16", "f32"])
@pytest.mark.parametrize("M", [1, 3, 4, 16])
@pytest.mark.parametrize("F,K", [(14336, 4096), (512, 4096), (64, 32), (768, 2048)])
def test_swiglu_f32(gpu, pkg, oracle, F, K, M, xdt):
    say(f"swiglu f32 F={F} K={K} M={M} x={xdt}")
    rng = np.random.default_rng(F + K + M)
    gb = oracle.baseline_q4_1_blocks(F, K, rng)
    ub = oracle.baseline_q4_1_blocks(F, K, rng)
    xt, x64 = _xs(rng, M, K, xdt)
    g, u = pkg.pack_q4_1(gb, gpu), pkg.pack_q4_1(ub, gpu)
    h = pkg.swiglu_q4(g, u, xt.to(gpu)).cpu().numpy()
    ref = oracle.swiglu_reference(gb, ub, x64)
    assert oracle.maxrel(h, ref) <= MAXREL


@pytest.mark.parametrize("F,K", [(14336, 4096), (512, 4096)])
def test_swiglu_bf16_out(gpu, pkg, oracle, F, K):
    say(f"swiglu bf16 F={F} K={K}")
    rng = np.random.default_rng(F)
    gb = oracle.baseline_q4_1_blocks(F, K, rng)
    ub = oracle.baseline_q4_1_blocks(F, K, rng)
    xt, x64 = _xs(rng, 2, K, "bf16")
    g, u = pkg.pack_q4_1(gb, gpu), pkg.pack_q4_1(ub, gpu)
    h = pkg.swiglu_q4(g, u, xt.to(gpu), out_dtype=torch.bfloat16)
    hf = pkg.swiglu_q4(g, u, xt.to(gpu))
    got = _bf16_bits_to_f64(h)
    ref = oracle.swiglu_reference(gb, ub, x64)
    _bf16_bars(got, ref)
    # the bf16 output is exactly the RNE of the kernel's own f32 result
    assert torch.equal(h, hf.to(torch.bfloat16))


def test_swiglu_is_deterministic_and_matches_separate_gemvs(gpu, pkg, oracle):
    say("swiglu determinism")
    rng = np.random.default_rng(5)
    F, K = 512, 4096                        # split along K
    gb = oracle.baseline_q4_1_blocks(F, K, rng)
    ub = oracle.baseline_q4_1_blocks(F, K, rng)
    g, u = pkg.pack_q4_1(gb, gpu), pkg.pack_q4_1(ub, gpu)
    x = torch.from_numpy(rng.standard_normal((4, K)).astype(np.float32)).to(torch.bfloat16).to(gpu)
    a = pkg.swiglu_q4(g, u, x)
    b = pkg.swiglu_q4(g, u, x)
    assert torch.equal(a, b)
    gy, uy = pkg.gemm_q4(g, x), pkg.gemm_q4(u, x)
    want = (gy / (1 + torch.exp(-gy))) * uy
    assert torch.allclose(a, want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("inplace", [False, True])
@pytest.mark.parametrize("N,K,M", [(4096, 14336, 1), (4096, 4096, 4), (128256, 4096, 2), (256, 1024, 16)])
def test_gemv_residual(gpu, pkg, oracle, N, K, M, inplace):
    say(f"gemv residual N={N} K={K} M={M} inplace={inplace}")
    rng = np.random.default_rng(N + K + M)
    blocks = oracle.baseline_q4_1_blocks(N, K, rng)
    w = pkg.pack_q4_1(blocks, gpu)
    xt, x64 = _xs(rng, M, K, "bf16")
    res = rng.standard_normal((M, N)).astype(np.float32) * 10
    rt = torch.from_numpy(res).to(gpu)
    if inplace:
        y = pkg.gemm_q4(w, xt.to(gpu), y=rt, residual=rt)
        assert y.data_ptr() == rt.data_ptr()
    else:
        y = pkg.gemm_q4(w, xt.to(gpu), residual=rt)
    ref = res.astype(np.float64) + oracle.gemv_reference(blocks, x64).astype(np.float64)
    got = y.cpu().numpy()
    assert oracle.maxrel(got, ref) <= MAXREL
    plain = pkg.gemm_q4(w, xt.to(gpu)).cpu().numpy()
    assert np.array_equal(got, (res + plain).astype(np.float32))     # the same f32 sum


@pytest.mark.parametrize("wdt", ["bf16", "f32"])
@pytest.mark.parametrize("N", [2048, 4096, 5120, 100])
@pytest.mark.parametrize("M", [1, 16])
def test_rmsnorm_add(gpu, pkg, oracle, N, M, wdt):
    say(f"rmsnorm_add N={N} M={M} w={wdt}")
    rng = np.random.default_rng(N + M)
    x = (rng.standard_normal((M, N)) * 0.5).astype(np.float32)
    add = (rng.standard_normal((M, N)) * 0.5).astype(np.float32)
    w = (1.0 + rng.standard_normal(N) * 0.1).astype(np.float32)
    wt = torch.from_numpy(w)
    if wdt == "bf16":
        wt = wt.to(torch.bfloat16)
        w = wt.to(torch.float32).numpy()
    y, xn = pkg.rmsnorm_add(torch.from_numpy(x).to(gpu), wt.to(gpu), torch.from_numpy(add).to(gpu), eps=1e-6)
    ry, rxn = oracle.rmsnorm_add_reference(x, add, w, 1e-6)
    assert np.array_equal(y.cpu().numpy(), ry)
    got = _bf16_bits_to_f64(xn)
    _bf16_bars(got, rxn)
    assert (np.abs(got - rxn) <= 2.0 ** -8 * np.abs(rxn) + 1e-30).all()
    _, xf = pkg.rmsnorm_add(torch.from_numpy(x).to(gpu), wt.to(gpu), torch.from_numpy(add).to(gpu), eps=1e-6,
                            out_dtype=torch.float32)
    assert oracle.maxrel(xf.cpu().numpy(), rxn) <= 1e-6


def test_rmsnorm_in_place_and_without_add(gpu, pkg, oracle):
    say("rmsnorm in place / no add")
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 4096)).astype(np.float32)
    add = rng.standard_normal((3, 4096)).astype(np.float32)
    w = np.ones(4096, np.float32)
    xt = torch.from_numpy(x).to(gpu)
    y, xn = pkg.rmsnorm_add(xt, torch.from_numpy(w).to(gpu), torch.from_numpy(add).to(gpu), y=xt)
    assert y.data_ptr() == xt.data_ptr() and np.array_equal(xt.cpu().numpy(), x + add)
    ry, rxn = oracle.rmsnorm_add_reference(x, add, w)
    _bf16_bars(_bf16_bits_to_f64(xn), rxn)
    y2, xn2 = pkg.rmsnorm_add(torch.from_numpy(x).to(gpu), torch.from_numpy(w).to(gpu))
    _, rxn2 = oracle.rmsnorm_add_reference(x, None, w)
    assert np.array_equal(y2.cpu().numpy(), x)
    _bf16_bars(_bf16_bits_to_f64(xn2), rxn2)


def test_fused_ffn_block_end_to_end(gpu, pkg, oracle):
    """rmsnorm_add -> swiglu (bf16 h) -> down with the residual in place: the decode
    FFN of one layer as three calls, against fp64 of the same bytes."""
    say("fused ffn block")
    rng = np.random.default_rng(11)
    H, F = 1024, 2048
    gb = oracle.baseline_q4_1_blocks(F, H, rng)
    ub = oracle.baseline_q4_1_blocks(F, H, rng)
    db = oracle.baseline_q4_1_blocks(H, F, rng)
    g, u, d = pkg.pack_q4_1(gb, gpu), pkg.pack_q4_1(ub, gpu), pkg.pack_q4_1(db, gpu)
    xres = rng.standard_normal((2, H)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    xr = torch.from_numpy(xres).to(gpu)
    _, xn = pkg.rmsnorm_add(xr, torch.from_numpy(w).to(gpu))
    h = pkg.swiglu_q4(g, u, xn, out_dtype=torch.bfloat16)
    pkg.gemm_q4(d, h, y=xr, residual=xr)
    # fp64 reference through the same bf16 roundings of xn and h
    _, rxn = oracle.rmsnorm_add_reference(xres, None, w)
    xnb = xn.to(torch.float32).cpu().numpy()
    assert (np.abs(xnb - rxn) <= 2.0 ** -8 * np.abs(rxn) + 1e-30).all()
    rh = oracle.swiglu_reference(gb, ub, xnb)
    hb = h.to(torch.float32).cpu().numpy()
    _bf16_bars(hb.astype(np.float64), rh)
    ref = xres.astype(np.float64) + oracle.gemv_reference(db, hb).astype(np.float64)
    assert oracle.maxrel(xr.cpu().numpy(), ref) <= MAXREL


@pytest.mark.parametrize("wdt", ["bf16", "f32"])
@pytest.mark.parametrize("N,K,M", [(6144, 4096, 1), (4096, 4096, 3), (1024, 4096, 16), (512, 14336, 2), (256, 96, 5)])
def test_gemv_with_its_rmsnorm_inside(gpu, pkg, oracle, N, K, M, wdt):
    """q4_gemv_rmsnorm: the norm formed per tile inside the GEMV gives the bits of
    q4_rmsnorm_add (bf16 out) followed by q4_gemv, on split and unsplit plans, 1..16 rows."""
    say(f"gemv with its rmsnorm N={N} K={K} M={M} w={wdt}")
    rng = np.random.default_rng(N + K + M)
    w = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(N, K, rng), gpu)
    x = torch.from_numpy((rng.standard_normal((M, K)) * 3).astype(np.float32)).to(gpu)
    nw = torch.from_numpy((1 + 0.1 * rng.standard_normal(K)).astype(np.float32)).to(gpu)
    if wdt == "bf16":
        nw = nw.to(torch.bfloat16)
    _, xn = pkg.rmsnorm_add(x, nw, eps=1e-5)
    ref = pkg.gemm_q4(w, xn)
    y = pkg.gemm_q4_rmsnorm(w, x, nw, eps=1e-5)
    assert torch.equal(y, ref)


@pytest.mark.parametrize("M", [1, 4, 9])
def test_swiglu_with_its_rmsnorm_inside(gpu, pkg, oracle, M):
    say(f"swiglu with its rmsnorm M={M}")
    F, K = 14336, 4096
    rng = np.random.default_rng(700 + M)
    g = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(F, K, rng), gpu)
    u = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(F, K, rng), gpu)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(gpu)
    nw = torch.from_numpy((1 + 0.1 * rng.standard_normal(K)).astype(np.float32)).to(torch.bfloat16).to(gpu)
    _, xn = pkg.rmsnorm_add(x, nw)
    for dt in (torch.bfloat16, torch.float32):
        ref = pkg.swiglu_q4(g, u, xn, out_dtype=dt)
        h = pkg.swiglu_q4(g, u, x, out_dtype=dt, norm_w=nw)
        assert torch.equal(h, ref)


def _acc_ref(res: torch.Tensor, part: torch.Tensor | None) -> torch.Tensor:
    """res + the planes in split order, in torch's IEEE f32 adds: res + p0 for one plane,
    res + (((0 + p0) + p1) + ...) for more (split_reduce's order)."""
    if part is None or part.shape[0] == 0:
        return res.clone()
    if part.shape[0] == 1:
        return res + part[0]
    s = torch.zeros_like(res)
    for q in range(part.shape[0]):
        s = s + part[q]
    return res + s


@pytest.mark.parametrize("N,K,M", [(4096, 4096, 1), (4096, 14336, 1), (6144, 4096, 1), (4096, 4096, 3), (256, 96, 2)])
def test_partials_add_up_to_the_split_gemv(gpu, pkg, oracle, N, K, M):
    """q4_gemv_partials at the plan's split count: the planes added in split order are
    q4_gemv's Y (and res + them q4_gemv_residual's) bit for bit; at another count they
    hold the K ranges' products (maxrel against fp64)."""
    say(f"partials N={N} K={K} M={M}")
    rng = np.random.default_rng(900 + N + K + M)
    blocks = oracle.baseline_q4_1_blocks(N, K, rng)
    w = pkg.pack_q4_1(blocks, gpu)
    xh = rng.standard_normal((M, K)).astype(np.float32)
    x = torch.from_numpy(xh).to(gpu).to(torch.bfloat16)
    res = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(gpu)
    S = pkg.gemv_split_count(w)
    part = pkg.gemm_q4_partials(w, x)
    assert part.shape == (S, M, N)
    y = pkg.gemm_q4(w, x)
    s = part[0] if S == 1 else _acc_ref(torch.zeros_like(y), part)
    assert torch.equal(s, y)
    assert torch.equal(_acc_ref(res, part), pkg.gemm_q4(w, x, residual=res))
    S2 = 3 if S != 3 else 5
    p2 = pkg.gemm_q4_partials(w, x, splits=S2).cpu().numpy().astype(np.float64)
    xb = x.to(torch.float32).cpu().numpy()
    dq = oracle.dequant_q4_1(blocks, bf16_scales=True).astype(np.float64)
    ref = oracle.gemv_reference(blocks, xb).astype(np.float64)
    assert oracle.maxrel(p2.sum(0), ref) <= MAXREL
    kb = K // 32                 # plane q: the 32-wide K positions [q KB / S, (q + 1) KB / S)
    for q in range(S2):
        k0, k1 = 32 * (q * kb // S2), 32 * ((q + 1) * kb // S2)
        rq = xb[:, k0:k1].astype(np.float64) @ dq[:, k0:k1].T
        assert np.abs(p2[q] - rq).max() <= MAXREL * np.abs(ref).max()


@pytest.mark.parametrize("wdt", ["bf16", "f32"])
@pytest.mark.parametrize("N,K,M,S", [(6144, 4096, 1, 0), (6144, 4096, 1, 1), (6144, 4096, 1, 4), (4096, 4096, 1, 16),
                                     (65536, 4096, 1, 16), (1024, 2048, 1, 3), (512, 8192, 1, 4), (1024, 4096, 3, 4),
                                     (256, 96, 5, 2)])
def test_gemv_rmsnorm_of_residual_plus_partials(gpu, pkg, oracle, N, K, M, S, wdt):
    """q4_gemv_rmsnorm_acc: x_out = res + partials in split order, bit for bit, and y the
    bits of q4_gemv_rmsnorm of that x -- fused inside the GEMV (one row, K <= 4096) and
    through the reduce launch (more rows, longer rows)."""
    say(f"gemv rmsnorm acc N={N} K={K} M={M} S={S} w={wdt}")
    rng = np.random.default_rng(1300 + N + K + M + S)
    w = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(N, K, rng), gpu)
    res = torch.from_numpy((rng.standard_normal((M, K)) * 3).astype(np.float32)).to(gpu)
    part = torch.from_numpy(rng.standard_normal((S, M, K)).astype(np.float32)).to(gpu) if S else None
    nw = torch.from_numpy((1 + 0.1 * rng.standard_normal(K)).astype(np.float32)).to(gpu)
    if wdt == "bf16":
        nw = nw.to(torch.bfloat16)
    x_ref = _acc_ref(res, part)
    y_ref = pkg.gemm_q4_rmsnorm(w, x_ref, nw, eps=1e-5)
    res0 = res.clone()
    for _ in range(2):      # the second call sees the first's x_out and y in place
        y, x_out = pkg.gemm_q4_rmsnorm_acc(w, res, part, nw, eps=1e-5)
        assert torch.equal(x_out, x_ref)
        assert torch.equal(y, y_ref)
    assert torch.equal(res, res0)
    _, xn = pkg.rmsnorm_add(x_ref, nw, eps=1e-5)
    ref = oracle.gemv_reference(oracle.baseline_q4_1_blocks(N, K, np.random.default_rng(1300 + N + K + M + S)),
                                xn.to(torch.float32).cpu().numpy()) if N * K <= 6144 * 4096 else None
    if ref is not None:
        assert oracle.maxrel(y.cpu().numpy(), ref) <= MAXREL


@pytest.mark.parametrize("wdt", ["bf16", "f32"])
@pytest.mark.parametrize("N,K,M,S", [(65536, 4096, 1, 0), (65536, 4096, 1, 4), (65536, 2048, 3, 1),
                                     (131072, 1024, 16, 2)])
def test_vocab_norm_gemv_normalises_once_with_the_same_bits(gpu, pkg, oracle, N, K, M, S, wdt):
    """At >= 1024 row groups (an lm_head) the norm GEMVs normalise the rows once into the
    workspace and run the plain GEMV when the workspace has q4_gemv_rmsnorm_workspace_bytes;
    with only q4_gemv_workspace_bytes every workgroup normalises per position. Both forms, and
    rmsnorm_add followed by gemm_q4, give the same bits; x_out too (S planes, S = 0: none)."""
    say(f"vocab norm gemv N={N} K={K} M={M} S={S} w={wdt}")
    rng = np.random.default_rng(2100 + N + K + M + S)
    w = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(N, K, rng), gpu)
    res = torch.from_numpy((rng.standard_normal((M, K)) * 3).astype(np.float32)).to(gpu)
    part = torch.from_numpy(rng.standard_normal((S, M, K)).astype(np.float32)).to(gpu) if S else None
    nw = torch.from_numpy((1 + 0.1 * rng.standard_normal(K)).astype(np.float32)).to(gpu)
    if wdt == "bf16":
        nw = nw.to(torch.bfloat16)
    lib = pkg.q4._lib_handle()
    small, big = lib.q4_gemv_workspace_bytes(M, N, K), lib.q4_gemv_rmsnorm_workspace_bytes(M, N, K)
    assert big >= small + M * K * 2
    x_ref = _acc_ref(res, part)
    _, xn = pkg.rmsnorm_add(x_ref, nw, eps=1e-5)
    ref = pkg.gemm_q4(w, xn)
    for nbytes in (max(small, 256), big):
        ws = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
        y = pkg.gemm_q4_rmsnorm(w, x_ref, nw, eps=1e-5, workspace=ws)
        assert torch.equal(y, ref), nbytes
        ya, x_out = pkg.gemm_q4_rmsnorm_acc(w, res, part, nw, eps=1e-5, workspace=ws)
        assert torch.equal(x_out, x_ref), nbytes
        assert torch.equal(ya, ref), nbytes


@pytest.mark.parametrize("M,S", [(1, 0), (1, 1), (1, 4), (1, 16), (2, 4)])
def test_swiglu_rmsnorm_of_residual_plus_partials(gpu, pkg, oracle, M, S):
    say(f"swiglu rmsnorm acc M={M} S={S}")
    F, K = 14336, 4096
    rng = np.random.default_rng(1700 + M + S)
    g = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(F, K, rng), gpu)
    u = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(F, K, rng), gpu)
    res = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(gpu)
    part = torch.from_numpy(rng.standard_normal((S, M, K)).astype(np.float32)).to(gpu) if S else None
    nw = torch.from_numpy((1 + 0.1 * rng.standard_normal(K)).astype(np.float32)).to(torch.bfloat16).to(gpu)
    x_ref = _acc_ref(res, part)
    for dt in (torch.bfloat16, torch.float32):
        ref = pkg.swiglu_q4(g, u, x_ref, out_dtype=dt, norm_w=nw)
        h, x_out = pkg.swiglu_q4_acc(g, u, res, part, nw, out_dtype=dt)
        assert torch.equal(x_out, x_ref)
        assert torch.equal(h, ref)


def test_deferred_reduction_chain_matches_the_residual_gemvs(gpu, pkg, oracle):
    """A decode layer's chain with the o / down reductions deferred into the next norm GEMV
    (partials at the plan's split counts) gives the residual stream and the outputs of the
    chain with q4_gemv_residual, bit for bit."""
    say("deferred reduction chain")
    H, F = 4096, 14336
    rng = np.random.default_rng(2024)
    wo = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(H, H, rng), gpu)
    wg = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(F, H, rng), gpu)
    wu = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(F, H, rng), gpu)
    wd = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(H, F, rng), gpu)
    wq = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(1024, H, rng), gpu)
    x0 = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32)).to(gpu)
    attn = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32)).to(gpu).to(torch.bfloat16)
    nw = torch.from_numpy((1 + 0.1 * rng.standard_normal(H)).astype(np.float32)).to(torch.bfloat16).to(gpu)
    xa = pkg.gemm_q4(wo, attn, residual=x0)
    h = pkg.swiglu_q4(wg, wu, xa, out_dtype=torch.bfloat16, norm_w=nw)
    xb = pkg.gemm_q4(wd, h, residual=xa)
    q = pkg.gemm_q4_rmsnorm(wq, xb, nw)
    po = pkg.gemm_q4_partials(wo, attn)
    h2, xa2 = pkg.swiglu_q4_acc(wg, wu, x0, po, nw, out_dtype=torch.bfloat16)
    pd = pkg.gemm_q4_partials(wd, h2)
    q2, xb2 = pkg.gemm_q4_rmsnorm_acc(wq, xa2, pd, nw)
    assert torch.equal(xa2, xa) and torch.equal(h2, h) and torch.equal(xb2, xb) and torch.equal(q2, q)
