"""Every operator refuses a bad caller buffer before any kernel launches, on the GPU
(the checks need device tensors). The refused calls launch nothing, so no kernel ever
sees the bad buffer; a correct call after them still gives the right answer."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu


def _bad_f32(dev, shape):
    """Buffers of the wrong dtype, count, layout and device for an f32 output of shape."""
    n = int(np.prod(shape))
    return [torch.empty(shape, dtype=torch.bfloat16, device=dev),
            torch.empty(n - 1, dtype=torch.float32, device=dev),
            torch.empty(n + 64, dtype=torch.float32, device=dev),
            torch.empty(shape[::-1], dtype=torch.float32, device=dev).t(),
            torch.empty(shape, dtype=torch.float32)]


def test_operators_refuse_bad_outputs(gpu, pkg, oracle):
    say("boundary: bad outputs refused")
    rng = np.random.default_rng(1)
    n, k, M = 256, 512, 3
    blocks = oracle.baseline_q4_1_blocks(n, k, rng)
    w = pkg.pack_q4_1(blocks, gpu)
    x = torch.from_numpy(rng.standard_normal((M, k)).astype(np.float32)).to(torch.bfloat16).to(gpu)
    for bad in _bad_f32(gpu, (M, n)):
        with pytest.raises((TypeError, ValueError)):
            pkg.gemm_q4(w, x, y=bad)
        with pytest.raises((TypeError, ValueError)):
            pkg.gemm_q4_prefill(w, x, y=bad)
    for bad in _bad_f32(gpu, (n, k)):
        with pytest.raises((TypeError, ValueError)):
            pkg.dequant(w, out=bad)
    with pytest.raises((TypeError, ValueError)):
        pkg.gemm_q4_prefill(w, x, precision="fp8")
    for bad in (torch.empty(2, n, dtype=torch.float32, device=gpu), torch.empty(M, n, dtype=torch.bfloat16,
                                                                               device=gpu)):
        with pytest.raises((TypeError, ValueError)):
            pkg.swiglu_q4(w, w, x, h=bad)
    ws_cpu = torch.empty(1 << 20, dtype=torch.uint8)
    with pytest.raises(ValueError):
        pkg.gemm_q4(w, x, workspace=ws_cpu)
    with pytest.raises((TypeError, ValueError)):
        pkg.pack_q4_1(blocks, gpu, out=torch.empty(w.nbytes - 16, dtype=torch.uint8, device=gpu))
    with pytest.raises((TypeError, ValueError)):
        pkg.lm_head_topk(w, x, k=2, ids=torch.empty(M, 2, dtype=torch.int64, device=gpu))
    with pytest.raises(ValueError):
        pkg.lm_head_topk(w, x, k=2, n_valid=n + 64)
    with pytest.raises(ValueError):
        pkg.logits_topk(torch.zeros(M, n, device=gpu), k=65)
    xr = torch.randn(M, k, device=gpu)
    with pytest.raises((TypeError, ValueError)):
        pkg.rmsnorm_add(xr, torch.ones(k, device=gpu), xn=torch.empty(M, k - 1, dtype=torch.bfloat16, device=gpu))
    with pytest.raises((TypeError, ValueError)):
        pkg.rmsnorm_add(xr, torch.ones(k, device=gpu), add=torch.randn(M, k, device=gpu).to(torch.bfloat16))
    # nothing was launched with a bad buffer: a good call still matches the oracle
    y = pkg.gemm_q4(w, x).cpu().numpy()
    ref = oracle.gemv_reference(blocks, x.to(torch.float32).cpu().numpy())
    assert oracle.maxrel(y, ref) <= 1e-3


def test_moe_refuses_bad_out(gpu, pkg, oracle):
    say("boundary: moe out refused")
    rng = np.random.default_rng(2)
    E, H, F, T = 4, 128, 64, 3
    gates = [oracle.baseline_q4_1_blocks(F, H, rng) for _ in range(E)]
    ups = [oracle.baseline_q4_1_blocks(F, H, rng) for _ in range(E)]
    downs = [oracle.baseline_q4_1_blocks(H, F, rng) for _ in range(E)]
    gu, dn = pkg.pack_moe_experts(gates, ups, downs, gpu)
    x = torch.randn(T, H, device=gpu).to(torch.bfloat16)
    ids = np.zeros((T, 2), np.int32)
    ids[:, 1] = 1
    wts = np.full((T, 2), 0.5, np.float32)
    for bad in _bad_f32(gpu, (T, H)):
        with pytest.raises((TypeError, ValueError)):
            pkg.moe_batch(gu, dn, x, ids, wts, out=bad)
