"""The RMSNorm producer that writes the prefill GEMM's prepared activations in one launch
(q4_rmsnorm_prepare): the same bytes as q4_rmsnorm_add (bf16 out) followed by
q4_prefill_prepare, padding rows and token exponents included, and the same GEMM bits."""
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
