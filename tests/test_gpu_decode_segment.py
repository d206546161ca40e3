"""GPU parity of q4_decode_segment, the layer's GEMV chain between two attentions in one
persistent launch (o -> RMSNorm -> SwiGLU -> down -> RMSNorm -> next qkv):

* at Llama-3-8B's shapes the outputs equal, bit for bit, the same chain of separate launches
  at the same split counts (q4_gemv_partials, q4_gemv_swiglu_rmsnorm_acc, q4_gemv_partials,
  q4_rmsnorm_add + q4_gemv_partials): same tiles per wave, same wave sums, same plane order;
* at small shapes (idle workgroups in every phase) and with a grid smaller than the items
  (every phase's item loop), each stage is held to fp64 from the kernel's own inputs to that
  stage (the bf16 roundings of the normalised rows and of h at the kernel's points):
  maxrel <= 1e-3 per output;
* the last layer's form (no qkv) ends with the down planes; x_next may be x; repeated calls
  and graph replays give the same bits and leave the workspace counters at zero."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu

MAXREL = 1e-3


def _layer(pkg, oracle, gpu, H, F, NQ, seed, nw_dtype=torch.bfloat16):
    rng = np.random.default_rng(seed)
    blk = {"o": oracle.baseline_q4_1_blocks(H, H, rng), "gate": oracle.baseline_q4_1_blocks(F, H, rng),
           "up": oracle.baseline_q4_1_blocks(F, H, rng), "down": oracle.baseline_q4_1_blocks(H, F, rng),
           "qkv": oracle.baseline_q4_1_blocks(NQ, H, rng)}
    w = {k: pkg.pack_q4_1(v, gpu) for k, v in blk.items()}
    x = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32)).to(gpu)
    attn = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32)).to(gpu).to(torch.bfloat16)
    nw1 = torch.from_numpy((1 + 0.1 * rng.standard_normal(H)).astype(np.float32)).to(gpu).to(nw_dtype)
    nw2 = torch.from_numpy((1 + 0.1 * rng.standard_normal(H)).astype(np.float32)).to(gpu).to(nw_dtype)
    return blk, w, x, attn, nw1, nw2


def _acc(res: torch.Tensor, planes: torch.Tensor) -> torch.Tensor:
    """res + the planes in split order: res + (((0 + p0) + p1) + ...) (res + p0 for one)."""
    if planes.shape[0] == 1:
        return res + planes[0]
    s = torch.zeros_like(res)
    for q in range(planes.shape[0]):
        s = s + planes[q]
    return res + s


def _check_sync(ws: torch.Tensor, qkv: bool = True) -> None:
    """After a completed call: hand-over 0's 16 counters (256 bytes apart) back at zero,
    hand-overs 1 and 2 holding one arrival per workgroup (2: none without qkv; the next
    call zeroes them as it starts), the time-out flag clear."""
    w = ws[:12800].view(torch.int32).view(50, 64)[:, 0].cpu().tolist()
    h0, h1, h2, flag = sum(w[0:16]), sum(w[16:32]), sum(w[32:48]), w[49]
    assert flag == 0 and h0 == 0 and h1 > 0 and h2 == (h1 if qkv else 0), (h0, h1, h2, flag)


def test_segment_equals_the_separate_launches_at_llama3_8b(gpu, pkg, oracle):
    H, F, NQ = 4096, 14336, 6144
    say(f"decode segment vs separate launches H={H} F={F} NQ={NQ}")
    _, w, x, attn, nw1, nw2 = _layer(pkg, oracle, gpu, H, F, NQ, 31)
    So, Sd, Sq = pkg.decode_segment_splits(H, F, NQ)
    ws = pkg.decode_segment_workspace(H, F, NQ, gpu)
    xm, xn, pd, pq = pkg.decode_segment(w["o"], w["gate"], w["up"], w["down"], w["qkv"], attn, x, nw1, nw2,
                                        workspace=ws)
    torch.cuda.synchronize()
    _check_sync(ws)
    po = pkg.gemm_q4_partials(w["o"], attn, splits=So)
    h, xm_ref = pkg.swiglu_q4_acc(w["gate"], w["up"], x, po, nw1, out_dtype=torch.bfloat16)
    pd_ref = pkg.gemm_q4_partials(w["down"], h, splits=Sd)
    xn_ref = _acc(xm_ref, pd_ref)
    _, n2 = pkg.rmsnorm_add(xn_ref, nw2)
    pq_ref = pkg.gemm_q4_partials(w["qkv"], n2, splits=Sq)
    assert torch.equal(xm, xm_ref)
    assert torch.equal(pd, pd_ref)
    assert torch.equal(xn, xn_ref)
    assert torch.equal(pq, pq_ref)


def _check_against_fp64(pkg, oracle, blk, x, attn, nw1, nw2, xm, xn, pd, pq, eps):
    """Each stage against fp64 from the kernel's own inputs to it."""
    x64 = x.cpu().numpy().astype(np.float64)
    a64 = attn.to(torch.float32).cpu().numpy().astype(np.float64)
    xm_ref = x64 + oracle.gemv_reference(blk["o"], a64).astype(np.float64)
    assert oracle.maxrel(xm.cpu().numpy(), xm_ref) <= MAXREL
    # n1 = bf16(RMSNorm(x_mid) w) exactly as the kernel forms it (rmsnorm_add's bits)
    _, n1 = pkg.rmsnorm_add(xm, nw1, eps=eps)
    h64 = oracle.swiglu_reference(blk["gate"], blk["up"], n1.to(torch.float32).cpu().numpy())
    hb = torch.from_numpy(h64.astype(np.float32)).to(torch.bfloat16).to(torch.float32).numpy().astype(np.float64)
    down = xm.cpu().numpy().astype(np.float64) + oracle.gemv_reference(blk["down"], hb).astype(np.float64)
    got = (xm + pd.sum(0)).cpu().numpy() if xn is None else xn.cpu().numpy()
    assert oracle.maxrel(got, down) <= MAXREL
    if xn is not None:
        _, n2 = pkg.rmsnorm_add(xn, nw2, eps=eps)
        q_ref = oracle.gemv_reference(blk["qkv"], n2.to(torch.float32).cpu().numpy())
        assert oracle.maxrel(pq.sum(0).cpu().numpy(), q_ref) <= MAXREL


@pytest.mark.parametrize("wgs", [None, 3, 24])
@pytest.mark.parametrize("nwd", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("H,F,NQ", [(256, 512, 384), (512, 1536, 768), (1024, 2048, 1536)])
def test_segment_against_fp64(gpu, pkg, oracle, monkeypatch, H, F, NQ, nwd, wgs):
    """Small shapes leave workgroups idle in every phase; grids of 3 and 24 workgroups
    (Q4MI_SEGMENT_WGS) make the phases loop over several items per workgroup (at 3: o,
    gate/up and down on every shape, qkv on the largest)."""
    if wgs is not None:
        monkeypatch.setenv("Q4MI_SEGMENT_WGS", str(wgs))
    say(f"decode segment vs fp64 H={H} F={F} NQ={NQ} nw={nwd} wgs={wgs}")
    blk, w, x, attn, nw1, nw2 = _layer(pkg, oracle, gpu, H, F, NQ, H + F + NQ, nwd)
    ws = pkg.decode_segment_workspace(H, F, NQ, gpu)
    xm, xn, pd, pq = pkg.decode_segment(w["o"], w["gate"], w["up"], w["down"], w["qkv"], attn, x, nw1, nw2,
                                        eps=1e-5, workspace=ws)
    torch.cuda.synchronize()
    _check_sync(ws)
    _check_against_fp64(pkg, oracle, blk, x, attn, nw1, nw2, xm, xn, pd, pq, 1e-5)


def test_last_layer_form_and_in_place_residual(gpu, pkg, oracle):
    """No qkv: the chain stops at the down planes, which gemm_q4_rmsnorm_acc takes on; with
    qkv and x_next = x, the residual stream advances in place with the same bits."""
    H, F, NQ = 1024, 2048, 1536
    say(f"decode segment last layer / in place H={H} F={F}")
    blk, w, x, attn, nw1, nw2 = _layer(pkg, oracle, gpu, H, F, NQ, 77)
    ws = pkg.decode_segment_workspace(H, F, NQ, gpu)
    xm, xn, pd, pq = pkg.decode_segment(w["o"], w["gate"], w["up"], w["down"], w["qkv"], attn, x, nw1, nw2,
                                        workspace=ws)
    xm2, xn2, pd2, pq2 = pkg.decode_segment(w["o"], w["gate"], w["up"], w["down"], None, attn, x, nw1,
                                            workspace=ws)
    assert xn2 is None and pq2 is None
    torch.cuda.synchronize()
    _check_sync(ws, qkv=False)
    assert torch.equal(xm2, xm) and torch.equal(pd2, pd)
    _check_against_fp64(pkg, oracle, blk, x, attn, nw1, nw2, xm2, None, pd2, None, 1e-6)
    y, xo = pkg.gemm_q4_rmsnorm_acc(w["qkv"], xm2, pd2, nw2)
    assert torch.equal(xo, xn)
    xi = x.clone()
    xm3, xn3, pd3, pq3 = pkg.decode_segment(w["o"], w["gate"], w["up"], w["down"], w["qkv"], attn, xi, nw1, nw2,
                                            x_next=xi, workspace=ws)
    assert xn3.data_ptr() == xi.data_ptr()
    assert torch.equal(xi, xn) and torch.equal(xm3, xm) and torch.equal(pq3, pq)
    torch.cuda.synchronize()
    _check_sync(ws)


def test_segment_repeats_and_replays_bit_for_bit(gpu, pkg, oracle):
    """Eager calls and graph replays (the counters return to zero after every launch, so a
    replay needs no memset node) give the same bits."""
    H, F, NQ = 4096, 14336, 6144
    say("decode segment repeats and graph replays")
    _, w, x, attn, nw1, nw2 = _layer(pkg, oracle, gpu, H, F, NQ, 5)
    So, Sd, Sq = pkg.decode_segment_splits(H, F, NQ)
    ws = pkg.decode_segment_workspace(H, F, NQ, gpu)
    xm = torch.empty(1, H, device=gpu)
    xn = torch.empty(1, H, device=gpu)
    pd = torch.empty(Sd, 1, H, device=gpu)
    pq = torch.empty(Sq, 1, NQ, device=gpu)

    def run():
        pkg.decode_segment(w["o"], w["gate"], w["up"], w["down"], w["qkv"], attn, x, nw1, nw2, x_mid=xm,
                           x_next=xn, down_planes=pd, qkv_planes=pq, workspace=ws)
    run()
    ref = [t.clone() for t in (xm, xn, pd, pq)]
    for _ in range(3):
        for t in (xm, xn, pd, pq):
            t.fill_(float("nan"))
        run()
        assert all(torch.equal(a, b) for a, b in zip((xm, xn, pd, pq), ref))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        run()
    torch.cuda.synchronize()
    for _ in range(3):
        for t in (xm, xn, pd, pq):
            t.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip((xm, xn, pd, pq), ref))
        _check_sync(ws)


def test_segment_refuses_bad_arguments(gpu, pkg, oracle):
    H, F, NQ = 256, 512, 384
    _, w, x, attn, nw1, nw2 = _layer(pkg, oracle, gpu, H, F, NQ, 3)
    with pytest.raises(RuntimeError):   # x_mid over x (Q4MI_E_ARG from the C ABI)
        pkg.decode_segment(w["o"], w["gate"], w["up"], w["down"], w["qkv"], attn, x, nw1, nw2, x_mid=x)
    with pytest.raises(ValueError):     # attn not bf16
        pkg.decode_segment(w["o"], w["gate"], w["up"], w["down"], w["qkv"], attn.float(), x, nw1, nw2)
    with pytest.raises(ValueError):     # swapped gate / down shapes
        pkg.decode_segment(w["o"], w["down"], w["up"], w["gate"], w["qkv"], attn, x, nw1, nw2)
    with pytest.raises(ValueError):     # qkv without its norm weight
        pkg.decode_segment(w["o"], w["gate"], w["up"], w["down"], w["qkv"], attn, x, nw1, None)
