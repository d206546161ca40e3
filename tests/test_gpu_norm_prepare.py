"""The producers that write the prefill GEMM's prepared activations in one launch: the
RMSNorm in front of gate/up (q4_rmsnorm_prepare: the same bytes as q4_rmsnorm_add (bf16
out) followed by q4_prefill_prepare, padding rows and token exponents included, and the
same GEMM bits) and the SwiGLU in front of down (q4_swiglu_prepare: h = bf16(silu(g) u)
and the bytes q4_prefill_prepare makes from it)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu


def _two_step(pkg, x, w, add, eps, precision, nbytes):
    y, xn = pkg.rmsnorm_add(x.clone(), w, add=add, eps=eps, out_dtype=torch.bfloat16,
                            y=None if add is None else torch.empty_like(x))
    out = torch.zeros(nbytes, dtype=torch.uint8, device=x.device)
    return y, pkg.prefill_prepare(xn, precision, out=out), xn


@pytest.mark.parametrize("T,K", [(1, 4096), (300, 4096), (512, 4128), (257, 14336), (33, 96)])
@pytest.mark.parametrize("precision", ["fp16", "bf16"])
@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("with_add", [False, True])
def test_rmsnorm_prepare_equals_norm_then_prepare(gpu, pkg, T, K, precision, wdt, with_add):
    say(f"rmsnorm_prepare T={T} K={K} {precision} w={wdt} add={with_add}")
    g = torch.Generator(device=gpu)
    g.manual_seed(T * 7 + K)
    x = torch.randn(T, K, generator=g, device=gpu) * 3.0
    add = torch.randn(T, K, generator=g, device=gpu) if with_add else None
    w = (1 + 0.1 * torch.randn(K, generator=g, device=gpu)).to(wdt)
    lib = pkg.load_library()
    nbytes = int(lib.q4_prefill_prepared_bytes(T, K, 1, 0 if precision == "fp16" else 1))
    y_ref, prep_ref, xn = _two_step(pkg, x, w, add, 1e-6, precision, nbytes)
    out = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    y, prep = pkg.rmsnorm_prepare(x, w, add=add, eps=1e-6, precision=precision,
                                  y=None if add is None else torch.empty_like(x), out=out)
    torch.cuda.synchronize()
    assert torch.equal(prep.data, prep_ref.data), "prepared bytes differ from norm + prepare"
    assert torch.equal(y, y_ref)
    if T == 300 and K == 4096 and wdt == torch.bfloat16:
        from oracle import q4_oracle as O
        blocks = O.baseline_q4_1_blocks(256, K, np.random.default_rng(T))
        wq = pkg.pack_q4_1(blocks, gpu)
        a = pkg.gemm_q4_prefill(wq, prep).cpu().numpy()
        b = pkg.gemm_q4_prefill(wq, xn, precision=precision).cpu().numpy()
        assert a.tobytes() == b.tobytes()


def test_rmsnorm_prepare_y_may_be_x(gpu, pkg):
    """y = x + add written over x itself (the residual stream updated in place)."""
    say("rmsnorm_prepare y aliasing x")
    g = torch.Generator(device=gpu)
    g.manual_seed(5)
    T, K = 260, 4096
    x = torch.randn(T, K, generator=g, device=gpu)
    add = torch.randn(T, K, generator=g, device=gpu)
    w = (1 + 0.1 * torch.randn(K, generator=g, device=gpu)).to(torch.bfloat16)
    nbytes = int(pkg.load_library().q4_prefill_prepared_bytes(T, K, 1, 0))
    y_ref, prep_ref, _ = _two_step(pkg, x, w, add, 1e-5, "fp16", nbytes)
    out = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    xx = x.clone()
    y, prep = pkg.rmsnorm_prepare(xx, w, add=add, eps=1e-5, y=xx, out=out)
    torch.cuda.synchronize()
    assert y.data_ptr() == xx.data_ptr()
    assert torch.equal(xx, y_ref)
    assert torch.equal(prep.data, prep_ref.data)


@pytest.mark.parametrize("T,F", [(1, 14336), (300, 14336), (257, 4128), (40, 96)])
@pytest.mark.parametrize("precision", ["fp16", "bf16"])
@pytest.mark.parametrize("fused", [False, True])
def test_swiglu_prepare_equals_swiglu_then_prepare(gpu, pkg, T, F, precision, fused):
    """h = bf16(silu(g) u) within one bf16 rounding of torch's, and the prepared image the
    bytes q4_prefill_prepare makes from that h; g and u as separate rows or the two halves of
    one fused gate/up output."""
    say(f"swiglu_prepare T={T} F={F} {precision} fused={fused}")
    gen = torch.Generator(device=gpu)
    gen.manual_seed(T + F)
    if fused:
        gu = torch.randn(T, 2 * F, generator=gen, device=gpu) * 4.0
        g, u = gu[:, :F], gu[:, F:]
    else:
        g = torch.randn(T, F, generator=gen, device=gpu) * 4.0
        u = torch.randn(T, F, generator=gen, device=gpu)
    lib = pkg.load_library()
    nbytes = int(lib.q4_prefill_prepared_bytes(T, F, 1, 0 if precision == "fp16" else 1))
    h = torch.empty(T, F, dtype=torch.bfloat16, device=gpu)
    prep = pkg.swiglu_prepare(gu if fused else g, None if fused else u, precision=precision,
                              out=torch.zeros(nbytes, dtype=torch.uint8, device=gpu), h=h)
    ref = pkg.prefill_prepare(h, precision, out=torch.zeros(nbytes, dtype=torch.uint8, device=gpu))
    torch.cuda.synchronize()
    assert torch.equal(prep.data, ref.data), "prepared bytes differ from prefill_prepare(h)"
    want = (g.double() / (1 + torch.exp(-g.double())) * u.double())
    got = h.double()
    # one RNE to bf16 of an f32 value within a few ulp of the fp64 one: <= 2^-8 relative
    err = ((got - want).abs() / want.abs().clamp_min(1e-30))
    assert float(err.max()) <= 2.0 ** -8 + 1e-6
    exact = (got == want.float().to(torch.bfloat16).double()).float().mean().item()
    assert exact >= 0.999


def test_swiglu_prepare_feeds_the_down_gemm(gpu, pkg, oracle):
    """down over the SwiGLU producer's prepared activations: the GEMM bits of the same h
    given as bf16 rows, and within 1e-3 of the fp64 reference on that h."""
    say("swiglu_prepare -> down GEMM")
    T, F, N = 300, 4096, 256
    gen = torch.Generator(device=gpu)
    gen.manual_seed(11)
    gu = torch.randn(T, 2 * F, generator=gen, device=gpu) * 3.0
    h = torch.empty(T, F, dtype=torch.bfloat16, device=gpu)
    prep = pkg.swiglu_prepare(gu, h=h)
    blocks = oracle.baseline_q4_1_blocks(N, F, np.random.default_rng(3))
    w = pkg.pack_q4_1(blocks, gpu)
    a = pkg.gemm_q4_prefill(w, prep).cpu().numpy()
    b = pkg.gemm_q4_prefill(w, h).cpu().numpy()
    assert a.tobytes() == b.tobytes()
    ref = oracle.gemv_reference(blocks, h.float().cpu().numpy())
    assert oracle.maxrel(a, ref) <= 1e-3


@pytest.mark.parametrize("precision", ["fp16", "bf16"])
def test_rmsnorm_prepare_sums_split_gemm_planes(gpu, pkg, oracle, precision):
    """A K-split prefill GEMM's unreduced planes (gemm_q4_prefill_partials), summed in order, are
    its reduced Y bit for bit, and the norm producer taking the planes as its addend gives the
    bytes it gives for that Y: the next layer's norm does the split reduce, no launch of its own."""
    T, N, K = 300, 512, 4096
    say(f"rmsnorm_prepare over split planes T={T} N={N} K={K} {precision}")
    lib = pkg.load_library()
    S = lib.q4_prefill_split_count(T, N, K)
    assert S > 1, "the shape should split"
    rng = np.random.default_rng(17)
    w = pkg.pack_q4_1(oracle.baseline_q4_1_blocks(N, K, rng), gpu)
    x = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).to(torch.bfloat16).to(gpu)
    prep = pkg.prefill_prepare(x, precision)
    part = pkg.gemm_q4_prefill_partials(w, prep)
    y = pkg.gemm_q4_prefill(w, prep)
    assert part.shape == (S, T, N)
    s = part[0].clone()
    for q in range(1, S):
        s += part[q]
    assert torch.equal(s, y)
    g = torch.Generator(device=gpu)
    g.manual_seed(3)
    res = torch.randn(T, N, generator=g, device=gpu)
    nw = (1 + 0.1 * torch.randn(N, generator=g, device=gpu)).to(torch.bfloat16)
    nbytes = int(lib.q4_prefill_prepared_bytes(T, N, 1, 0))
    ya, pa = pkg.rmsnorm_prepare(res, nw, add=part, y=torch.empty_like(res),
                                 out=torch.zeros(nbytes, dtype=torch.uint8, device=gpu))
    yb, pb = pkg.rmsnorm_prepare(res, nw, add=y, y=torch.empty_like(res),
                                 out=torch.zeros(nbytes, dtype=torch.uint8, device=gpu))
    torch.cuda.synchronize()
    assert torch.equal(ya, yb)
    assert torch.equal(pa.data, pb.data)


@pytest.mark.parametrize("precision", ["fp16", "bf16"])
def test_producers_hold_small_rows_to_the_oracle(gpu, pkg, oracle, precision):
    """Rows far below fp16's normal range (h ~ 1e-15 to 1e-5, normed rows ~ 1e-6): the producers write
    the bytes the pre-pass writes (each token row scaled by a power of two into fp16's top
    binade) and every row of the GEMM over them stays within 1e-3 of the fp64 reference."""
    say(f"producers at small magnitude {precision}")
    T, F, K, N = 64, 1024, 1024, 256
    gen = torch.Generator(device=gpu)
    gen.manual_seed(23)
    row_scale = (10.0 ** -torch.linspace(3, 7, T, device=gpu)).unsqueeze(1)
    gu = torch.randn(T, 2 * F, generator=gen, device=gpu) * row_scale
    lib = pkg.load_library()
    zeros = lambda K_: torch.zeros(int(lib.q4_prefill_prepared_bytes(T, K_, 1, 0 if precision == "fp16" else 1)),
                                   dtype=torch.uint8, device=gpu)
    h = torch.empty(T, F, dtype=torch.bfloat16, device=gpu)
    prep = pkg.swiglu_prepare(gu, precision=precision, h=h, out=zeros(F))
    ref_prep = pkg.prefill_prepare(h, precision, out=zeros(F))
    x = torch.randn(T, K, generator=gen, device=gpu)
    w = (5e-7 * (1 + 0.1 * torch.randn(K, generator=gen, device=gpu)) * (1 + torch.arange(K, device=gpu) % 7)
         ).to(torch.bfloat16)
    _, nprep = pkg.rmsnorm_prepare(x, w, eps=1e-6, precision=precision, out=zeros(K))
    _, xn = pkg.rmsnorm_add(x.clone(), w, eps=1e-6, out_dtype=torch.bfloat16)
    ref_nprep = pkg.prefill_prepare(xn, precision, out=zeros(K))
    torch.cuda.synchronize()
    assert float(h.float().abs().max()) < 2.0 ** -14, "h should lie below fp16's normal range"
    assert float(xn.float().abs().max()) < 2.0 ** -14
    assert torch.equal(prep.data, ref_prep.data)
    assert torch.equal(nprep.data, ref_nprep.data)
    blocks = oracle.baseline_q4_1_blocks(N, F, np.random.default_rng(5))
    wq = pkg.pack_q4_1(blocks, gpu)
    # the bf16 tile is RNE_bf16(q d + m), the reference's: its bar is over those weights
    wd = oracle.dequant_q4_1(blocks)
    wd = (oracle.bf16_round(wd) if precision == "bf16" else wd).astype(np.float64)
    for p, xin in ((prep, h), (nprep, xn)):
        got = pkg.gemm_q4_prefill(wq, p).cpu().numpy()
        ref = xin.double().cpu().numpy() @ wd.T
        worst = max(oracle.maxrel(got[t], ref[t]) for t in range(T))
        assert worst <= 1e-3, worst
