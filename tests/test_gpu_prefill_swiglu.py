"""The gate/up prefill GEMM with SwiGLU in its epilogue (q4_gemm_prefill_swiglu): h is the
bf16 h the SwiGLU producer forms from the plain GEMM's f32 gate and up outputs, bit for bit
where that GEMM runs unsplit, and within the GEMM's bar plus one bf16 rounding of the fp64
silu(g) u."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu


def _gate_up(pkg, oracle, F, K, rng, dev):
    bg = oracle.baseline_q4_1_blocks(F, K, rng)
    bu = oracle.baseline_q4_1_blocks(F, K, rng)
    g, u = pkg.pack_q4_1(bg, dev), pkg.pack_q4_1(bu, dev)
    return bg, bu, g, u, pkg.interleave_gate_up(g, u)


def test_interleave_gate_up_alternates_row_groups(gpu, pkg, oracle):
    say("interleave_gate_up layout")
    rng = np.random.default_rng(1)
    _, _, g, u, gu = _gate_up(pkg, oracle, 256, 128, rng, gpu)
    rg = g.nbytes // 4
    a = gu.data.view(8, rg)
    assert (gu.n, gu.k) == (512, 128)
    for j in range(4):
        assert torch.equal(a[2 * j], g.data.view(4, rg)[j]) and torch.equal(a[2 * j + 1], u.data.view(4, rg)[j])


@pytest.mark.parametrize("small", [False, True])
@pytest.mark.parametrize("precision", ["fp16", "bf16"])
def test_swiglu_epilogue_equals_plain_gemm_then_swiglu(gpu, pkg, oracle, precision, small):
    """At T = 2048, 2F = 8192 the plain GEMM's plan has no K split (256 tiles), so its f32
    outputs are the epilogue's accumulators: the h of both paths must be the same bits. small:
    token rows scaled by 1 .. 1e-7, so the fp16 path's per-token exponents span 24 binades."""
    T, F, K = 2048, 4096, 1024
    say(f"swiglu epilogue vs plain GEMM + swiglu_prepare T={T} F={F} K={K} {precision} small={small}")
    lib = pkg.load_library()
    assert lib.q4_gemm_prefill_prepared_workspace_bytes(T, 2 * F, K) == 0, "plain plan is split"
    rng = np.random.default_rng(7)
    _, _, _, _, gu = _gate_up(pkg, oracle, F, K, rng, gpu)
    xf = rng.standard_normal((T, K)).astype(np.float32)
    if small:
        xf *= (10.0 ** -np.linspace(0, 7, T)).astype(np.float32)[:, None]
    x = torch.from_numpy(xf).to(torch.bfloat16).to(gpu)
    prep = pkg.prefill_prepare(x, precision)
    h = pkg.gemm_q4_prefill_swiglu(gu, prep)
    y = pkg.gemm_q4_prefill(gu, prep).view(T, F // 64, 2, 64)
    g, u = y[:, :, 0, :].reshape(T, F).contiguous(), y[:, :, 1, :].reshape(T, F).contiguous()
    h_ref = torch.empty(T, F, dtype=torch.bfloat16, device=gpu)
    pkg.swiglu_prepare(g, u, h=h_ref)
    torch.cuda.synchronize()
    assert torch.equal(h, h_ref)
    if small:
        assert float(h[-1].float().abs().max()) < 2.0 ** -24 and bool((h[-1] != 0).any())


@pytest.mark.parametrize("T", [1, 300])
@pytest.mark.parametrize("precision", ["fp16", "bf16"])
def test_swiglu_epilogue_against_fp64(gpu, pkg, oracle, T, precision):
    """Ragged token counts against silu(g) u from the fp64 reference GEMMs. Bar: the GEMM's
    (1e-3 at precision fp16, the bf16 tile's ~2e-3 at bf16) plus one bf16 rounding of h."""
    F, K = 384, 512
    say(f"swiglu epilogue vs fp64 T={T} F={F} K={K} {precision}")
    rng = np.random.default_rng(T)
    bg, bu, _, _, gu = _gate_up(pkg, oracle, F, K, rng, gpu)
    xf = rng.standard_normal((T, K)).astype(np.float32)
    x = torch.from_numpy(xf).to(torch.bfloat16)
    h = pkg.gemm_q4_prefill_swiglu(gu, x.to(gpu), precision=precision).float().cpu().numpy()
    xb = x.float().numpy()
    g = oracle.prefill_reference(bg, xb).astype(np.float64)
    u = oracle.prefill_reference(bu, xb).astype(np.float64)
    ref = g / (1.0 + np.exp(-g)) * u
    bar = (1e-3 if precision == "fp16" else 2.5e-3) * 3 + 2.0 ** -8
    assert oracle.maxrel(h, ref) <= bar
    assert h.shape == (T, F)


def test_swiglu_epilogue_refuses_two_pass_activations(gpu, pkg, oracle):
    """f32 activations in precision fp16 take two GEMM passes: no epilogue can see the sum."""
    rng = np.random.default_rng(2)
    _, _, _, _, gu = _gate_up(pkg, oracle, 128, 128, rng, gpu)
    x = torch.randn(4, 128, device=gpu)
    with pytest.raises(ValueError):
        pkg.gemm_q4_prefill_swiglu(gu, x)
    prep = pkg.prefill_prepare(x, "fp16")
    with pytest.raises(RuntimeError):
        pkg.gemm_q4_prefill_swiglu(gu, prep)


def test_swiglu_epilogue_at_the_bench_geometry(gpu, pkg, oracle):
    """The bench's FFN block shape: Llama-3-8B gate/up interleaved (2F = 28672, K = 4096) at
    T = 2048. The plain GEMM's plan is unsplit there, so h equals GEMM + swiglu_prepare bit for
    bit; sampled tokens are also held to silu(g) u of the fp64 reference GEMMs (the GEMM's
    1e-3 bar, amplified by at most 3 through silu(g) u, plus one bf16 rounding of h)."""
    T, F, K = 2048, 14336, 4096
    say(f"swiglu epilogue at the bench geometry T={T} F={F} K={K}")
    lib = pkg.load_library()
    assert lib.q4_gemm_prefill_prepared_workspace_bytes(T, 2 * F, K) == 0, "plain plan is split"
    rng = np.random.default_rng(2024)
    bg, bu, _, _, gu = _gate_up(pkg, oracle, F, K, rng, gpu)
    x = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).to(torch.bfloat16)
    prep = pkg.prefill_prepare(x.to(gpu))
    h = pkg.gemm_q4_prefill_swiglu(gu, prep)
    y = pkg.gemm_q4_prefill(gu, prep).view(T, F // 64, 2, 64)
    g, u = y[:, :, 0, :].reshape(T, F).contiguous(), y[:, :, 1, :].reshape(T, F).contiguous()
    del y
    h_ref = torch.empty(T, F, dtype=torch.bfloat16, device=gpu)
    pkg.swiglu_prepare(g, u, h=h_ref)
    torch.cuda.synchronize()
    assert torch.equal(h, h_ref)
    pick = np.array([0, 1, 255, 256, 1023, 1500, 2046, 2047])
    xb = x.float().numpy()[pick].astype(np.float64)
    gr = xb @ oracle.dequant_q4_1(bg).astype(np.float64).T
    ur = xb @ oracle.dequant_q4_1(bu).astype(np.float64).T
    ref = gr / (1.0 + np.exp(-gr)) * ur
    got = h.float().cpu().numpy()[pick]
    assert oracle.maxrel(got, ref) <= 3e-3 + 2.0 ** -8, oracle.maxrel(got, ref)
