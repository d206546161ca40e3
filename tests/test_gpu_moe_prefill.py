"""GPU parity of the routed MoE block at prefill scale (q4_moe_prefill: each expert's tokens
batched into 256-token tiles of the prefill GEMM, as the reference batches them into slots
of its expert dispatches, moe_batch.h:98-172 and core.cpp:5163-5178).

Bars: precision "fp16" against the fp64 oracle with the exact weights and fp32 h
(moe_reference): maxrel <= 1e-3 per the north star, and the reference's moe_batch gate
rel_fro <= 5e-3 (designs/moe_batch/compare.py:20). Precision "bf16" (the reference's tile,
RNE_bf16(q d + m), h rounded to bf16 as moe_batch.h:181-202 does) against the oracle over
the same bf16-rounded weights with h_bf16: maxrel <= 1e-3. At config 4's matrices and
T = 2048 (16384 pairs) the oracle runs on sampled tokens (the routing of one token does not
involve the others)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu


def _make(oracle, pkg, gpu, E, H, F, seed, bf16_weights=False):
    rng = np.random.default_rng(seed)
    gates = [oracle.baseline_q4_1_blocks(F, H, rng) for _ in range(E)]
    ups = [oracle.baseline_q4_1_blocks(F, H, rng) for _ in range(E)]
    downs = [oracle.baseline_q4_1_blocks(H, F, rng) for _ in range(E)]
    gu, dn = pkg.pack_moe_experts(gates, ups, downs, gpu)
    if bf16_weights:
        deq = lambda blocks: (lambda e: oracle.bf16_round(oracle.dequant_q4_1(blocks[e])))
    else:
        deq = lambda blocks: (lambda e: oracle.dequant_q4_1(blocks[e]))
    return rng, gu, dn, deq(gates), deq(ups), deq(downs)


@pytest.mark.parametrize("E,H,F,T,K,xdt,prec", [
    (8, 256, 128, 300, 2, "bf16", "fp16"),        # several token tiles per expert
    (8, 256, 128, 300, 2, "f32", "fp16"),         # f32 x: value and remainder passes
    (16, 512, 256, 97, 4, "bf16", "fp16"),        # ragged tiles, some experts empty
    (8, 256, 128, 300, 2, "bf16", "bf16"),
    (16, 512, 256, 97, 4, "f32", "bf16"),
    (8, 256, 128, 300, 2, "bf16", "fp16h"),       # fp16 tile, h rounded to bf16: one down pass
    (16, 512, 256, 97, 4, "f32", "fp16h"),
])
def test_moe_prefill_matches_oracle(gpu, pkg, oracle, E, H, F, T, K, xdt, prec):
    say(f"moe prefill E={E} H={H} F={F} T={T} top{K} {xdt} {prec}")
    rng, gu, dn, g_of, u_of, d_of = _make(oracle, pkg, gpu, E, H, F, E + H + T, bf16_weights=prec == "bf16")
    x = rng.standard_normal((T, H)).astype(np.float32)
    xt = torch.from_numpy(x).to(torch.bfloat16) if xdt == "bf16" else torch.from_numpy(x)
    ids, w = oracle.softmax_topk(rng.standard_normal((T, E)), K)
    out = pkg.moe_batch(gu, dn, xt.to(gpu), ids, w, path="prefill", precision="bf16" if prec == "bf16" else "fp16",
                        h_bf16=prec == "fp16h").cpu().numpy()
    xr = xt.to(torch.float32).numpy()
    if prec == "bf16":
        xr = oracle.bf16_round(xr)
    ref = oracle.moe_reference(g_of, u_of, d_of, xr, ids, w, h_bf16=prec != "fp16")
    assert out.shape == (T, H) and np.isfinite(out).all()
    assert oracle.maxrel(out, ref) <= 1e-3, oracle.maxrel(out, ref)
    assert oracle.rel_fro(out, ref) <= 5e-3


def test_moe_prefill_deterministic_and_equal_to_decode_path(gpu, pkg, oracle):
    """Same bits on every call; within fp32-level noise of the decode path (fp32 h) at a
    batch both paths take."""
    say("moe prefill determinism / decode agreement")
    E, H, F, T, K = 16, 512, 256, 200, 4
    rng, gu, dn, *_ = _make(oracle, pkg, gpu, E, H, F, 31)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16).to(gpu)
    ids, w = oracle.softmax_topk(rng.standard_normal((T, E)), K)
    a = pkg.moe_batch(gu, dn, x, ids, w, path="prefill", h_bf16=False).cpu().numpy()
    for _ in range(2):
        assert pkg.moe_batch(gu, dn, x, ids, w, path="prefill", h_bf16=False).cpu().numpy().tobytes() == a.tobytes()
    d = pkg.moe_batch(gu, dn, x, ids, w, path="decode").cpu().numpy()
    assert oracle.maxrel(a, d) <= 1e-3


@pytest.mark.parametrize("prec", ["bf16", "fp16"])
def test_moe_prefill_ids_at_any_4_byte_offset(gpu, pkg, oracle, prec):
    """The routing loads each thread's 16 ids as 16-byte vectors when the ids are 16-byte
    aligned and one by one otherwise: ids 4 bytes past an aligned base (and a pair count
    that is no multiple of 16) give the aligned call's bits."""
    say(f"moe prefill unaligned ids {prec}")
    E, H, F, T, K = 16, 512, 256, 97, 4
    rng, gu, dn, *_ = _make(oracle, pkg, gpu, E, H, F, 47)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16).to(gpu)
    ids, w = oracle.softmax_topk(rng.standard_normal((T, E)), K)
    a = pkg.moe_batch(gu, dn, x, ids, w, path="prefill", precision=prec).cpu()
    buf = torch.empty(T * K + 4, dtype=torch.int32, device=gpu)
    for shift in (1, 2, 3):
        view = buf[shift:shift + T * K].view(T, K)
        view.copy_(torch.from_numpy(ids.astype(np.int32)))
        assert view.data_ptr() % 16 != 0
        b = pkg.moe_batch(gu, dn, x, view, w, path="prefill", precision=prec).cpu()
        assert torch.equal(a, b), shift


@pytest.mark.parametrize("E,H,F,T,K", [(8, 256, 128, 300, 2), (16, 512, 256, 97, 4), (6, 256, 128, 700, 2),
                                       (128, 2048, 768, 512, 8)])
def test_moe_prefill_bf16_gather_equals_tiled_image(gpu, pkg, oracle, E, H, F, T, K):
    """The bf16 tile on bf16 x DMAs its token rows straight from x and h (gather form); on
    f32 x it runs the per-slot activation images (x prep, h prep). x's values are bf16 in
    both calls, so both forms feed the MFMAs the same operands: the outputs are equal bit
    for bit (ragged tiles, empty experts, several tiles per expert, ids outside [0, E),
    config 4's shapes)."""
    say(f"moe prefill bf16 gather vs image E={E} H={H} F={F} T={T} top{K}")
    rng, gu, dn, *_ = _make(oracle, pkg, gpu, E, H, F, 5 * E + T, bf16_weights=True)
    xb = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16)
    ids, w = oracle.softmax_topk(rng.standard_normal((T, E)), K)
    if E == 6:                                    # one expert takes every token; -1 ids add nothing
        ids = np.stack([np.full(T, 4), np.full(T, -1)], axis=1).astype(np.int32)
        w = np.stack([np.ones(T), np.full(T, 3.0)], axis=1).astype(np.float32)
    a = pkg.moe_batch(gu, dn, xb.to(gpu), ids, w, path="prefill", precision="bf16").cpu().numpy()
    b = pkg.moe_batch(gu, dn, xb.to(torch.float32).to(gpu), ids, w, path="prefill", precision="bf16").cpu().numpy()
    assert np.isfinite(a).all()
    assert a.tobytes() == b.tobytes()


@pytest.mark.parametrize("E", [6, 16])
def test_moe_prefill_one_expert_takes_every_token(gpu, pkg, oracle, E):
    """All pairs on one expert (many full tiles), the rest empty; ids outside [0, E) add nothing.
    E = 6: 256-token tiles (1400 pairs > 192 per expert); E = 16: the same expert's three tiles
    as 128-token halves, the last one's upper half partly empty."""
    say(f"moe prefill, one popular expert, E={E}")
    H, F, T = 256, 128, 700
    rng, gu, dn, g_of, u_of, d_of = _make(oracle, pkg, gpu, E, H, F, 77)
    x = rng.standard_normal((T, H)).astype(np.float32)
    xt = torch.from_numpy(x).to(torch.bfloat16)
    ids = np.stack([np.full(T, 4), np.full(T, -1)], axis=1).astype(np.int32)
    w = np.stack([np.ones(T), np.full(T, 3.0)], axis=1).astype(np.float32)
    out = pkg.moe_batch(gu, dn, xt.to(gpu), ids, w, path="prefill", h_bf16=False).cpu().numpy()
    ref = oracle.moe_reference(g_of, u_of, d_of, xt.to(torch.float32).numpy(), ids[:, :1], w[:, :1])
    assert oracle.maxrel(out, ref) <= 1e-3


@pytest.mark.parametrize("T,prec", [(512, "fp16"), (2048, "fp16"), (2048, "fp16h"), (2048, "bf16"), (512, "auto")])
def test_moe_prefill_config4_matrices_sampled_tokens(gpu, pkg, oracle, T, prec):
    """Config 4's experts (128 x [1536, 2048] gate/up, [2048, 768] down, top-8 routing) at
    prefill scale: T * 8 = 4096 and 16384 pairs through the prefill path, in each form the
    bench times (fp16 tile with f32 h; fp16 tile with bf16 h and the SwiGLU epilogue, the
    default; the reference's bf16 tile), so moe_dma_kernel runs at K = 2048 over 1536-row
    expert matrices and at down's K = 768. "auto" at T = 512 is the decode path (4096 pairs).
    Sampled tokens are held to the fp64 oracle (bf16 h where the form rounds h, over
    bf16-rounded weights for the bf16 tile)."""
    E, H, F, K = 128, 2048, 768, 8
    say(f"moe prefill config-4 matrices T={T} {prec}")
    rng, gu, dn, g_of, u_of, d_of = _make(oracle, pkg, gpu, E, H, F, 4000 + T, bf16_weights=prec == "bf16")
    x = rng.standard_normal((T, H)).astype(np.float32)
    xt = torch.from_numpy(x).to(torch.bfloat16)
    ids, w = oracle.softmax_topk(rng.standard_normal((T, E)), K)
    if prec == "auto":
        out = pkg.moe_batch(gu, dn, xt.to(gpu), ids, w).cpu().numpy()
    else:
        out = pkg.moe_batch(gu, dn, xt.to(gpu), ids, w, path="prefill", precision="bf16" if prec == "bf16" else "fp16",
                            h_bf16=prec != "fp16").cpu().numpy()
    assert np.isfinite(out).all()
    pick = np.sort(rng.choice(T, 12, replace=False))
    xr = xt.to(torch.float32).numpy()[pick]
    if prec == "bf16":
        xr = oracle.bf16_round(xr)
    ref = oracle.moe_reference(g_of, u_of, d_of, xr, ids[pick], w[pick], h_bf16=prec in ("fp16h", "bf16"))
    assert oracle.maxrel(out[pick], ref) <= 1e-3, oracle.maxrel(out[pick], ref)
    assert oracle.rel_fro(out[pick], ref) <= 5e-3


@pytest.mark.parametrize("prec", ["fp16", "fp16h", "bf16"])
def test_moe_prefill_small_rows(gpu, pkg, oracle, prec):
    """Token rows scaled by 1 .. 1e-6 (h down to ~1e-13, far below fp16's normal range): the fp16
    paths' per-token power-of-two exponents for x and h keep every output row within 1e-3 of the
    fp64 oracle, measured row by row."""
    E, H, F, T, K = 8, 256, 128, 300, 2
    say(f"moe prefill small rows {prec}")
    rng, gu, dn, g_of, u_of, d_of = _make(oracle, pkg, gpu, E, H, F, 91, bf16_weights=prec == "bf16")
    x = rng.standard_normal((T, H)).astype(np.float32) * (10.0 ** -np.linspace(0, 6, T)).astype(np.float32)[:, None]
    xt = torch.from_numpy(x).to(torch.bfloat16)
    ids, w = oracle.softmax_topk(rng.standard_normal((T, E)), K)
    out = pkg.moe_batch(gu, dn, xt.to(gpu), ids, w, path="prefill", precision="bf16" if prec == "bf16" else "fp16",
                        h_bf16=prec == "fp16h").cpu().numpy()
    ref = oracle.moe_reference(g_of, u_of, d_of, xt.to(torch.float32).numpy(), ids, w, h_bf16=prec != "fp16")
    assert np.abs(ref[-1]).max() < 1e-9
    worst = max(oracle.maxrel(out[t], ref[t]) for t in range(T))
    assert worst <= 1e-3, worst
