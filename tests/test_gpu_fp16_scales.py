"""The opt-in exact-scale mode (q4_repack scale_mode 1, pack_q4_1(..., scales="fp16")):
GGUF's fp16 d and m kept in the scale word, as the reference's GGUF-direct pool keeps them
(open_kernels/gguf_pool/gguf_pool.py:1-17, designs/gemv_q4/gemv_q4.h:54-65).

Bars: the repacked bytes equal the oracle's pack_mx(fp16_scales=True); the dequant is
bit-exact with the f32-scale unpack (dequant_q4_1(bf16_scales=False)); the GEMV and the
grouped sweep are within maxrel 1e-3 of the fp64 reference over those exact weights, and
closer to it than the bf16-scale mode on weights whose scales bf16 cannot hold."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu


def test_repack_and_dequant_are_exact(gpu, pkg, oracle):
    say("fp16 scales: repack bytes and dequant")
    rng = np.random.default_rng(61)
    for n, k in ((64, 32), (256, 1024), (4096, 4096)):
        blocks = oracle.baseline_q4_1_blocks(n, k, rng)
        w = pkg.pack_q4_1(blocks, gpu, scales="fp16")
        assert w.scales == "fp16"
        assert np.array_equal(w.data.cpu().numpy(), oracle.pack_mx(blocks, fp16_scales=True))
        got = pkg.dequant(w).cpu().numpy()
        assert got.tobytes() == oracle.dequant_q4_1(blocks, bf16_scales=False).tobytes()


@pytest.mark.parametrize("M", [1, 4, 13, 16])
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
@pytest.mark.parametrize("n,k", [(4096, 4096), (1024, 14336), (14336, 4096)])
def test_gemv_against_fp64(gpu, pkg, oracle, M, xdt, n, k):
    """Split and unsplit plans (4096 x 4096 splits K 4 ways), both activation dtypes, with and
    without the residual epilogue."""
    say(f"fp16 scales: gemv M={M} {xdt} {n}x{k}")
    rng = np.random.default_rng(M * 7 + n)
    blocks = oracle.baseline_q4_1_blocks(n, k, rng)
    w = pkg.pack_q4_1(blocks, gpu, scales="fp16")
    x = torch.from_numpy(rng.standard_normal((M, k)).astype(np.float32))
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    xr = x.float().numpy().astype(np.float64)
    ref = xr @ oracle.dequant_q4_1(blocks, bf16_scales=False).astype(np.float64).T
    y = pkg.gemm_q4(w, x.to(gpu)).cpu().numpy()
    assert oracle.maxrel(y, ref) <= 1e-3, oracle.maxrel(y, ref)
    res = torch.from_numpy(rng.standard_normal((M, n)).astype(np.float32)).to(gpu)
    yr = pkg.gemm_q4(w, x.to(gpu), residual=res).cpu().numpy()
    assert oracle.maxrel(yr, ref + res.cpu().numpy()) <= 1e-3


def test_fp16_scales_are_closer_to_the_exact_weights(gpu, pkg, oracle):
    """Scales spread over fp16's range: the bf16 mode's narrowing shows against the exact
    (f32-scale) reference; the fp16 mode does not have that error."""
    say("fp16 scales: against the bf16 mode")
    rng = np.random.default_rng(62)
    n, k = 512, 4096
    blocks = oracle.baseline_q4_1_blocks(n, k, rng)
    x = torch.from_numpy(rng.standard_normal((1, k)).astype(np.float32))
    ref = x.numpy().astype(np.float64) @ oracle.dequant_q4_1(blocks, bf16_scales=False).astype(np.float64).T
    e16 = oracle.rel_fro(pkg.gemm_q4(pkg.pack_q4_1(blocks, gpu, scales="fp16"), x.to(gpu)).cpu().numpy(), ref)
    eb = oracle.rel_fro(pkg.gemm_q4(pkg.pack_q4_1(blocks, gpu), x.to(gpu)).cpu().numpy(), ref)
    assert e16 < eb / 8, (e16, eb)


@pytest.mark.parametrize("M", [1, 8, 16])
def test_grouped_sweep_equals_single_gemvs(gpu, pkg, oracle, M):
    """GemvGroup over fp16-scale matrices (one launch, q4_gemv_grouped_fp16s) against the
    fp64 reference; every member within 1e-3."""
    say(f"fp16 scales: grouped M={M}")
    rng = np.random.default_rng(63 + M)
    shapes = [(1024, 4096), (4096, 4096), (4096, 14336), (2048, 1024)]
    items, refs = [], []
    for n, k in shapes:
        blocks = oracle.baseline_q4_1_blocks(n, k, rng)
        w = pkg.pack_q4_1(blocks, gpu, scales="fp16")
        x = torch.from_numpy(rng.standard_normal((M, k)).astype(np.float32)).to(torch.bfloat16)
        refs.append(x.float().numpy().astype(np.float64) @ oracle.dequant_q4_1(blocks, bf16_scales=False)
                    .astype(np.float64).T)
        items.append((w, x.to(gpu), torch.empty(M, n, device=gpu)))
    g = pkg.GemvGroup(items)
    g.run()
    torch.cuda.synchronize()
    for (w, x, y), ref in zip(items, refs):
        assert oracle.maxrel(y.cpu().numpy(), ref) <= 1e-3


def test_bf16_only_operators_refuse_fp16_scales(gpu, pkg, oracle):
    rng = np.random.default_rng(64)
    blocks = oracle.baseline_q4_1_blocks(256, 512, rng)
    w = pkg.pack_q4_1(blocks, gpu, scales="fp16")
    wb = pkg.pack_q4_1(blocks, gpu)
    x = torch.randn(2, 512, device=gpu)
    with pytest.raises(ValueError):
        pkg.gemm_q4_prefill(w, x.to(torch.bfloat16))
    with pytest.raises(ValueError):
        pkg.swiglu_q4(w, w, x)
    with pytest.raises(ValueError):
        pkg.lm_head_topk(w, x)
    with pytest.raises(ValueError):
        pkg.GemvGroup([(w, x, torch.empty(2, 256, device=gpu)), (wb, x, torch.empty(2, 256, device=gpu))])
    with pytest.raises(ValueError):
        pkg.gemm_q4(w, torch.randn(17, 512, device=gpu))
    with pytest.raises(ValueError):
        pkg.pack_q4_1(oracle.random_q4_0_blocks_ref(64, 32, rng), gpu, scales="fp16")
