"""GPU parity of the routed MoE block against the fp64 oracle.

out[t] = sum_j w[t,j] down_e(silu(gate_e x_t) (up_e x_t)), ids/weights from a
seeded softmax top-k (model/replica.py:121-140 route + moe_decode without the
shared expert). Bar: maxrel <= 1e-3 per the north star (h is kept in fp32,
the replica's semantics); the reference's moe_batch gate is rel_fro <= 5e-3
(designs/moe_batch/compare.py:20), asserted too.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu


def _make(oracle, pkg, gpu, E, H, F, seed):
    rng = np.random.default_rng(seed)
    gates = [oracle.baseline_q4_1_blocks(F, H, rng) for _ in range(E)]
    ups = [oracle.baseline_q4_1_blocks(F, H, rng) for _ in range(E)]
    downs = [oracle.baseline_q4_1_blocks(H, F, rng) for _ in range(E)]
    gu, dn = pkg.pack_moe_experts(gates, ups, downs, gpu)
    deq = lambda blocks: (lambda e: oracle.dequant_q4_1(blocks[e]))
    return rng, gu, dn, deq(gates), deq(ups), deq(downs)


@pytest.mark.parametrize("E,H,F,T,K,xdt", [
    (8, 256, 128, 3, 2, "bf16"),
    (128, 512, 256, 16, 8, "bf16"),      # config 4's routing (128 experts, top-8, 16 tokens), smaller matrices
    (16, 2048, 768, 16, 8, "bf16"),      # config 4's matrices (H=2048, F=768), 16 experts
    (128, 2048, 768, 16, 8, "bf16"),     # config 4 exactly: 128 experts, top-8, 16 tokens, H=2048, F=768
    (4, 256, 192, 40, 2, "bf16"),        # ~20 tokens per expert: more than one 16-token chunk
    (8, 256, 128, 5, 3, "f32"),
    (8, 192, 128, 5, 2, "bf16"),         # H % 256 != 0: one 64-row group per down workgroup
    (16, 256, 128, 200, 4, "bf16"),      # 800 pairs: the routing's batched id loads and one-pass compaction
    (32, 256, 128, 512, 8, "bf16"),      # 4096 pairs, the decode path's maximum (T = 512, top-8)
])
def test_moe_matches_oracle(gpu, pkg, oracle, E, H, F, T, K, xdt):
    say(f"moe E={E} H={H} F={F} T={T} top{K} {xdt}")
    rng, gu, dn, g_of, u_of, d_of = _make(oracle, pkg, gpu, E, H, F, E + H + T)
    x = rng.standard_normal((T, H)).astype(np.float32)
    xt = torch.from_numpy(x).to(torch.bfloat16) if xdt == "bf16" else torch.from_numpy(x)
    ids, w = oracle.softmax_topk(rng.standard_normal((T, E)), K)
    out = pkg.moe_batch(gu, dn, xt.to(gpu), ids, w).cpu().numpy()
    ref = oracle.moe_reference(g_of, u_of, d_of, xt.to(torch.float32).numpy(), ids, w)
    assert out.shape == (T, H) and np.isfinite(out).all()
    assert oracle.maxrel(out, ref) <= 1e-3, oracle.maxrel(out, ref)
    assert oracle.rel_fro(out, ref) <= 5e-3


def test_moe_deterministic_and_order_free(gpu, pkg, oracle):
    """Same bits on every call; permuting a token's (id, weight) slots only
    reorders the combine sum (fp32 noise)."""
    say("moe determinism")
    E, H, F, T, K = 16, 256, 128, 8, 4
    rng, gu, dn, *_ = _make(oracle, pkg, gpu, E, H, F, 77)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16).to(gpu)
    ids, w = oracle.softmax_topk(rng.standard_normal((T, E)), K)
    a = pkg.moe_batch(gu, dn, x, ids, w).cpu().numpy()
    for _ in range(3):
        assert pkg.moe_batch(gu, dn, x, ids, w).cpu().numpy().tobytes() == a.tobytes()
    perm = np.array([3, 1, 0, 2])
    b = pkg.moe_batch(gu, dn, x, ids[:, perm], w[:, perm]).cpu().numpy()
    assert oracle.maxrel(b, a) < 1e-5


def test_moe_single_expert_equals_dense_path(gpu, pkg, oracle):
    """top-1 with weight 1: out = down(silu(gate x) * up x) -- the same product
    through the dense GEMV entry points and an elementwise silu on the host."""
    say("moe vs dense composition")
    E, H, F, T = 4, 512, 256, 6
    rng = np.random.default_rng(5)
    gates = [oracle.baseline_q4_1_blocks(F, H, rng) for _ in range(E)]
    ups = [oracle.baseline_q4_1_blocks(F, H, rng) for _ in range(E)]
    downs = [oracle.baseline_q4_1_blocks(H, F, rng) for _ in range(E)]
    gu, dn = pkg.pack_moe_experts(gates, ups, downs, gpu)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16).to(gpu)
    ids = np.full((T, 1), 2, np.int32)
    w = np.ones((T, 1), np.float32)
    out = pkg.moe_batch(gu, dn, x, ids, w).cpu().numpy()
    g = pkg.gemm_q4(pkg.pack_q4_1(gates[2], gpu), x)
    u = pkg.gemm_q4(pkg.pack_q4_1(ups[2], gpu), x)
    h = g / (1 + torch.exp(-g)) * u
    y = pkg.gemm_q4(pkg.pack_q4_1(downs[2], gpu), h).cpu().numpy()
    assert oracle.maxrel(out, y) < 1e-5


def test_moe_empty_and_limits(gpu, pkg, oracle):
    say("moe empty / limits")
    E, H, F = 4, 128, 64
    rng, gu, dn, *_ = _make(oracle, pkg, gpu, E, H, F, 3)
    out = pkg.moe_batch(gu, dn, torch.zeros(0, H, dtype=torch.bfloat16, device=gpu),
                        np.zeros((0, 2), np.int32), np.zeros((0, 2), np.float32))
    assert out.shape == (0, H)
    with pytest.raises(Exception):
        pkg.moe_batch(gu, dn, torch.zeros(600, H, dtype=torch.bfloat16, device=gpu),
                      np.zeros((600, 8), np.int32), np.zeros((600, 8), np.float32),
                      path="decode")                                           # 4800 pairs > 4096
    with pytest.raises(Exception):                                             # prefill path: H % 256
        pkg.moe_batch(gu, dn, torch.zeros(600, H, dtype=torch.bfloat16, device=gpu),
                      np.zeros((600, 8), np.int32), np.zeros((600, 8), np.float32))


def test_moe_few_pairs_path_with_popular_experts(gpu, pkg, oracle):
    """T * topk <= 2E takes the one-accumulator kernels (chunks of 4 routed tokens): here
    every token picks the same 8 of 32 experts, so each of those streams its rows in two
    chunks. Same bar as the other shapes."""
    say("moe few-pairs path, 8 tokens on the same 8 experts")
    E, H, F, T, K = 32, 512, 256, 8, 8
    rng, gu, dn, g_of, u_of, d_of = _make(oracle, pkg, gpu, E, H, F, 321)
    x = rng.standard_normal((T, H)).astype(np.float32)
    xt = torch.from_numpy(x).to(torch.bfloat16)
    ids = np.tile(np.arange(3, 3 + K, dtype=np.int32), (T, 1))
    w = rng.uniform(0.5, 1.5, (T, K)).astype(np.float32)
    w /= w.sum(1, keepdims=True)
    out = pkg.moe_batch(gu, dn, xt.to(gpu), ids, w).cpu().numpy()
    ref = oracle.moe_reference(g_of, u_of, d_of, xt.to(torch.float32).numpy(), ids, w)
    assert np.isfinite(out).all()
    assert oracle.maxrel(out, ref) <= 1e-3, oracle.maxrel(out, ref)
    assert oracle.rel_fro(out, ref) <= 5e-3


def test_moe_routed_experts_past_the_first_words(gpu, pkg, oracle):
    """The expert kernels map their workgroups onto the routed experts in ascending order
    (a bitmap of 32-expert words): with E = 300 and every token routed into experts
    250..299, the routed experts sit in words 7..9 and the last word is partial. Also a
    single token (8 workgroup rows of routed experts, the rest of the grid idle)."""
    E, H, F = 300, 128, 64
    rng, gu, dn, g_of, u_of, d_of = _make(oracle, pkg, gpu, E, H, F, 4242)
    for T, K in ((12, 4), (1, 8)):
        say(f"moe E={E} T={T} top{K}, experts 250..299")
        x = rng.standard_normal((T, H)).astype(np.float32)
        xt = torch.from_numpy(x).to(torch.bfloat16)
        ids = np.stack([rng.choice(np.arange(250, 300), K, replace=False) for _ in range(T)]).astype(np.int32)
        w = rng.uniform(0.5, 1.5, (T, K)).astype(np.float32)
        out = pkg.moe_batch(gu, dn, xt.to(gpu), ids, w).cpu().numpy()
        ref = oracle.moe_reference(g_of, u_of, d_of, xt.to(torch.float32).numpy(), ids, w)
        assert np.isfinite(out).all()
        assert oracle.maxrel(out, ref) <= 1e-3, oracle.maxrel(out, ref)


@pytest.mark.parametrize("E,H,F,T,K,xdt", [(16, 512, 256, 6, 4, "bf16"), (8, 256, 128, 5, 3, "f32"),
                                            (128, 2048, 768, 16, 8, "bf16")])
def test_moe_fin_residual_and_shared_expert(gpu, pkg, oracle, E, H, F, T, K, xdt):
    """The block's finish folded into the combine (moe_fin.py:1-4):
    out = (residual + routed sum) + sigmoid(x . sgw) * shared. Against fp64 of the same
    formula; the residual-only form equals moe_batch + residual bit for bit; sgw = 0 gives the
    gate 0.5 exactly; the residual may be the output buffer."""
    say(f"moe fin E={E} H={H} F={F} T={T} top{K} {xdt}")
    rng, gu, dn, g_of, u_of, d_of = _make(oracle, pkg, gpu, E, H, F, 900 + H)
    x = rng.standard_normal((T, H)).astype(np.float32)
    xt = (torch.from_numpy(x).to(torch.bfloat16) if xdt == "bf16" else torch.from_numpy(x)).to(gpu)
    ids, w = oracle.softmax_topk(rng.standard_normal((T, E)), K)
    res = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(gpu)
    sh = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(gpu)
    sgw = torch.from_numpy(rng.standard_normal(H).astype(np.float32) * 0.05).to(torch.bfloat16).to(gpu)
    out = pkg.moe_batch(gu, dn, xt, ids, w, residual=res, shared=sh, shared_gate_w=sgw).cpu().numpy()
    xr = xt.to(torch.float32).cpu().numpy()
    acc = oracle.moe_reference(g_of, u_of, d_of, xr, ids, w)
    ref = oracle.moe_fin_reference(acc, res.cpu().numpy(), sh.cpu().numpy(), xr, sgw.cpu().view(torch.int16).numpy().view(np.uint16))
    assert np.isfinite(out).all()
    assert oracle.maxrel(out, ref) <= 1e-3, oracle.maxrel(out, ref)
    plain = pkg.moe_batch(gu, dn, xt, ids, w)
    only_res = pkg.moe_batch(gu, dn, xt, ids, w, residual=res)
    assert torch.equal(only_res, res + plain)
    half = pkg.moe_batch(gu, dn, xt, ids, w, residual=res, shared=sh,
                         shared_gate_w=torch.zeros(H, dtype=torch.bfloat16, device=gpu))
    assert torch.equal(half, (res + plain) + 0.5 * sh)
    acc_buf = res.clone()
    pkg.moe_batch(gu, dn, xt, ids, w, out=acc_buf, residual=acc_buf, shared=sh, shared_gate_w=sgw)
    assert np.array_equal(acc_buf.cpu().numpy(), out)


@pytest.mark.parametrize("E,H,F,Fs,T,K,xdt", [
    (128, 2048, 768, 768, 16, 8, "bf16"),   # config 4 with a shared expert of an expert's size
    (8, 256, 128, 192, 5, 2, "bf16"),        # Fs != F; 4-token chunks, the last one partial
    (4, 256, 192, 128, 40, 2, "f32"),        # 16-token chunks (more than 2 pairs per expert)
    (8, 192, 128, 256, 7, 3, "bf16"),        # H % 256 != 0: one row group per down workgroup
])
def test_moe_block_with_shared_expert(gpu, pkg, oracle, E, H, F, Fs, T, K, xdt):
    """The shared expert inside the block's launches (q4_moe_gemv_shared):
    out = (residual + routed sum) + sigmoid(x . sgw) * down_s(silu(gate_s x) (up_s x)), the
    replica's moe_decode (replica.py:131-144), against fp64 with fp32 h; the same within fp32
    noise as the two-step form (the shared expert run as a one-expert block, its output given
    as `shared`); the residual may be the output buffer."""
    say(f"moe block + shared expert E={E} H={H} F={F} Fs={Fs} T={T} top{K} {xdt}")
    rng, gu, dn, g_of, u_of, d_of = _make(oracle, pkg, gpu, E, H, F, 700 + Fs)
    bgs, bus = oracle.baseline_q4_1_blocks(Fs, H, rng), oracle.baseline_q4_1_blocks(Fs, H, rng)
    bds = oracle.baseline_q4_1_blocks(H, Fs, rng)
    sgu = pkg.interleave_gate_up(pkg.pack_q4_1(bgs, gpu), pkg.pack_q4_1(bus, gpu))
    sdn = pkg.pack_q4_1(bds, gpu)
    x = rng.standard_normal((T, H)).astype(np.float32)
    xt = (torch.from_numpy(x).to(torch.bfloat16) if xdt == "bf16" else torch.from_numpy(x)).to(gpu)
    ids, w = oracle.softmax_topk(rng.standard_normal((T, E)), K)
    res = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(gpu)
    sgw = torch.from_numpy(rng.standard_normal(H).astype(np.float32) * 0.05).to(torch.bfloat16).to(gpu)
    out = pkg.moe_batch(gu, dn, xt, ids, w, residual=res, shared_gate_w=sgw, shared_expert=(sgu, sdn))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    xr = xt.to(torch.float32).cpu().numpy()
    acc = oracle.moe_reference(g_of, u_of, d_of, xr, ids, w)
    one = np.zeros((T, 1), np.int32)
    sh = oracle.moe_reference(lambda e: oracle.dequant_q4_1(bgs), lambda e: oracle.dequant_q4_1(bus),
                              lambda e: oracle.dequant_q4_1(bds), xr, one, np.ones((T, 1), np.float32))
    ref = oracle.moe_fin_reference(acc, res.cpu().numpy(), sh, xr, sgw.cpu().view(torch.int16).numpy().view(np.uint16))
    assert np.isfinite(got).all()
    assert oracle.maxrel(got, ref) <= 1e-3, oracle.maxrel(got, ref)
    # two-step form: the shared expert as a one-expert block, then the finish with its output
    sgu_e = pkg.PackedExperts(sgu.data, 1, 2 * Fs, H)
    sdn_e = pkg.PackedExperts(sdn.data, 1, H, Fs)
    ys = pkg.moe_batch(sgu_e, sdn_e, xt, one, np.ones((T, 1), np.float32))
    two = pkg.moe_batch(gu, dn, xt, ids, w, residual=res, shared=ys, shared_gate_w=sgw)
    assert oracle.maxrel(got, two.cpu().numpy()) <= 1e-6
    acc_buf = res.clone()
    pkg.moe_batch(gu, dn, xt, ids, w, out=acc_buf, residual=acc_buf, shared_gate_w=sgw, shared_expert=(sgu, sdn))
    assert np.array_equal(acc_buf.cpu().numpy(), got)
