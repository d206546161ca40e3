"""The measurement probes behind the bench's on-box peaks read and compute what they claim:
the streaming read folds every word of its buffer (the xor of each workgroup's share), and
the MFMA probe's per-lane sums equal the closed form of its operands' product, which also
pins the 16x16x32 fp16 MFMA's lane layout that the probe's flop count assumes."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,wgs", [(16 * 256 * 8 * 3 + 16 * 7, 5), (1 << 22, 64), (4096, 300)])
def test_stream_read_folds_every_word(gpu, lib, nbytes, wgs):
    say(f"probe stream read {nbytes} B over {wgs} workgroups")
    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 2**32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    buf = torch.from_numpy(host.view(np.int32)).to(gpu)
    out = torch.full((lib.q4_probe_stream_read_out_bytes(wgs) // 4,), -1, dtype=torch.int32, device=gpu)
    assert lib.q4_probe_stream_read(buf.data_ptr(), nbytes, wgs, out.data_ptr(), None) == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32).reshape(wgs, 4)
    n16 = nbytes // 16
    per = -(-n16 // wgs)
    words = host.reshape(n16, 4)
    for b in range(wgs):
        share = words[b * per:min((b + 1) * per, n16)]
        want = np.bitwise_xor.reduce(share.ravel()) if share.size else np.uint32(0)
        assert np.bitwise_xor.reduce(got[b]) == want, b   # the 4 waves' xors fold to the share's


def _frag_matrices(ops):
    """[16 sets][8] fp16 per lane -> A_i (16 x 32) from sets 0..7 and B_j (32 x 16) from 8..15:
    lane l holds A[l % 16][8 (l // 16) + e] and B[8 (l // 16) + e][l % 16]."""
    A = np.zeros((8, 16, 32))
    B = np.zeros((8, 32, 16))
    for l in range(64):
        for i in range(8):
            A[i, l % 16, 8 * (l // 16):8 * (l // 16) + 8] = ops[l, i]
            B[i, 8 * (l // 16):8 * (l // 16) + 8, l % 16] = ops[l, 8 + i]
    return A, B


def _lane_sums(D, iters):
    """Per lane: iters x the sum of its 4 output rows of each chain's D (16 x 16)."""
    return np.array([iters * sum(D[c][4 * (l // 16) + r, l % 16] for c in range(len(D)) for r in range(4))
                     for l in range(64)])


def test_mfma_probe_matches_the_closed_form(gpu, lib):
    say("probe mfma closed form (constant operands)")
    wgs, iters = 3, 5
    out = torch.empty(wgs * 256, dtype=torch.float32, device=gpu)
    assert lib.q4_probe_mfma(wgs, iters, None, out.data_ptr(), None) == 0
    torch.cuda.synchronize()
    ops = np.zeros((64, 16, 8))
    for l in range(64):
        for e in range(8):
            ops[l, 0, e] = ((l + e) & 7) * 0.125
            ops[l, 8, e] = ((3 * l + e) & 7) * 0.0625
    A, B = _frag_matrices(ops)
    want = _lane_sums([A[0] @ B[0]] * 8, iters)
    got = out.cpu().numpy().reshape(wgs * 4, 64)
    assert np.array_equal(got, np.broadcast_to(want.astype(np.float32), got.shape))


def test_mfma_probe_with_operand_sets(gpu, lib):
    """The toggling form: round u pairs A set (u + c) % 8 with B set c in chain c. Operands are
    multiples of 1/8 below 2, so every sum is exact in fp32."""
    say("probe mfma closed form (operand sets)")
    rng = np.random.default_rng(5)
    ops = (rng.integers(-15, 16, (64, 16, 8)) / 8.0).astype(np.float16)
    dops = torch.from_numpy(ops).to(gpu)
    wgs, iters = 2, 3
    out = torch.empty(wgs * 256, dtype=torch.float32, device=gpu)
    assert lib.q4_probe_mfma(wgs, iters, dops.data_ptr(), out.data_ptr(), None) == 0
    torch.cuda.synchronize()
    A, B = _frag_matrices(ops.astype(np.float64))
    D = [sum(A[(u + c) & 7] @ B[c] for u in range(8)) for c in range(8)]
    want = _lane_sums(D, iters)
    got = out.cpu().numpy().reshape(wgs * 4, 64)
    assert np.array_equal(got, np.broadcast_to(want.astype(np.float32), got.shape))
