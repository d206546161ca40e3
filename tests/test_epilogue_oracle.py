"""Pin the oracle's epilogue references against library routines and closed forms:
silu against scipy's logistic function, the RMSNorm against torch's own rms_norm in
fp64, and the SwiGLU reference against the (separately pinned) GEMV reference."""
from __future__ import annotations

import numpy as np
import torch
from scipy.special import expit


def test_silu_is_x_times_the_logistic(oracle):
    g = np.linspace(-30, 30, 10001)
    assert np.allclose(oracle.silu(g), g * expit(g), rtol=1e-14, atol=1e-300)
    assert oracle.silu(np.array([0.0]))[0] == 0.0


def test_rmsnorm_matches_torch_rms_norm(oracle):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 4096)).astype(np.float32)
    add = rng.standard_normal((5, 4096)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
    y, xn = oracle.rmsnorm_add_reference(x, add, w, 1e-6)
    assert np.array_equal(y, x + add)
    want = torch.nn.functional.rms_norm(torch.from_numpy(y.astype(np.float64)), (4096,),
                                        torch.from_numpy(w.astype(np.float64)), eps=1e-6).numpy()
    assert np.allclose(xn, want, rtol=1e-12, atol=1e-12)


def test_rmsnorm_closed_forms(oracle):
    """A constant row normalises to sign(c) * w (eps -> 0); scaling x leaves xn alone."""
    w = np.arange(1, 9, dtype=np.float32)
    _, xn = oracle.rmsnorm_add_reference(np.full((1, 8), -3.0, np.float32), None, w, 0.0)
    assert np.allclose(xn[0], -w, rtol=1e-15)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((1, 64)).astype(np.float32)
    _, a = oracle.rmsnorm_add_reference(x, None, np.ones(64), 0.0)
    _, b = oracle.rmsnorm_add_reference(x * np.float32(8.0), None, np.ones(64), 0.0)
    assert np.allclose(a, b, rtol=1e-12)


def test_swiglu_reference_composes_the_gemv_reference(oracle):
    rng = np.random.default_rng(2)
    g = oracle.random_q4_1_blocks_ref(64, 256, rng)
    u = oracle.random_q4_1_blocks_ref(64, 256, rng)
    x = rng.standard_normal((2, 256)).astype(np.float32)
    h = oracle.swiglu_reference(g, u, x)
    gg = oracle.gemv_reference(g, x).astype(np.float64)
    uu = oracle.gemv_reference(u, x).astype(np.float64)
    assert np.allclose(h, gg * expit(gg) * uu, rtol=1e-5, atol=1e-7)


def test_moe_fin_reference_pins(oracle):
    """moe_fin_reference (moe_fin.py:1-4): the gate against scipy's expit of the dot product,
    sgw = 0 gives the gate 0.5 exactly, no shared expert leaves residual + routed sum, and
    neither term leaves the routed sum alone."""
    from scipy.special import expit
    rng = np.random.default_rng(11)
    T, H = 5, 64
    acc = rng.standard_normal((T, H))
    res = rng.standard_normal((T, H))
    sh = rng.standard_normal((T, H))
    x = rng.standard_normal((T, H)).astype(np.float32)
    sgw = oracle.f32_to_bf16(rng.standard_normal(H).astype(np.float32) * 0.1)
    sgw_f = (sgw.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    g = expit(x.astype(np.float64) @ sgw_f)
    assert np.allclose(oracle.moe_fin_reference(acc, res, sh, x, sgw), res + acc + g[:, None] * sh, rtol=1e-14, atol=0)
    zero = np.zeros(H, np.uint16)
    assert np.array_equal(oracle.moe_fin_reference(acc, res, sh, x, zero), res + acc + 0.5 * sh)
    assert np.array_equal(oracle.moe_fin_reference(acc, res, None, x, None), acc + res)
    assert np.array_equal(oracle.moe_fin_reference(acc, None, None, x, None), acc)
