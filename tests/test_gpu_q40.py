"""GPU parity of the Q4_0-native path (mx0 layout: the mx codes plus one bf16 d per row and
block, m = -8 d; the reference's 4608 B Q4_0-native chunk, q4_1_pack.py:145-152, and the
GEMV build that reads it, designs/gemv_q4/gemv_q4.h:66-82): repacked bytes bit-exact
against the oracle from GGUF Q4_0 blocks and from the reference's chunks (rs 1, 2, 4),
dequant bit-exact, and the GEMV bit-identical to the widened Q4_1 path's (q4_repack of the
same 18-byte blocks: the same d, m = -8 d and arithmetic) and within the bar of the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu

MAXREL = 1e-3


@pytest.mark.parametrize("n,k", [(64, 32), (192, 512), (256, 4096)])
def test_repack_from_gguf_blocks_and_dequant(gpu, pkg, oracle, n, k):
    say(f"q4_0 native repack gguf n={n} k={k}")
    rng = np.random.default_rng(n + k)
    b = oracle.random_q4_0_blocks_ref(n, k, rng)
    w = pkg.pack_q4_0_native(b, n, k, "q4_0", device=gpu)
    torch.cuda.synchronize()
    assert w.nbytes == oracle.mx0_bytes(n, k)
    assert np.array_equal(w.data.cpu().numpy(), oracle.pack_mx0(b))
    deq = pkg.dequant_q4_0_native(w).cpu().numpy()
    assert deq.tobytes() == oracle.dequant_q4_1(b).tobytes()


@pytest.mark.parametrize("rs", [1, 2, 4])
def test_repack_from_reference_chunks(gpu, pkg, oracle, rs):
    n, k = 256, 1024
    say(f"q4_0 native repack chunks rs={rs}")
    rng = np.random.default_rng(50 + rs)
    b = oracle.random_q4_0_blocks_ref(n, k, rng)
    chunks = oracle.pack_q4_0_native_pool(b, rs)
    w = pkg.pack_q4_0_native(chunks, n, k, "chunks", rs, gpu)
    torch.cuda.synchronize()
    assert np.array_equal(w.data.cpu().numpy(), oracle.pack_mx0(b))


@pytest.mark.parametrize("xdt", ["bf16", "f32"])
@pytest.mark.parametrize("n,k,M", [(1024, 4096, 1), (6144, 4096, 4), (4096, 14336, 16), (4096, 4096, 3)])
def test_gemv_equals_the_widened_path_bit_for_bit(gpu, pkg, oracle, xdt, n, k, M):
    say(f"q4_0 native gemv n={n} k={k} M={M} {xdt}")
    rng = np.random.default_rng(n + k + M)
    b = oracle.random_q4_0_blocks_ref(n, k, rng)
    w0 = pkg.pack_q4_0_native(b, n, k, "q4_0", device=gpu)
    w1 = pkg.pack_q4_1(b, gpu)
    assert w0.nbytes * 10 == w1.nbytes * 9                   # 0.5625 against 0.625 B per weight
    xf = rng.standard_normal((M, k)).astype(np.float32)
    x = (torch.from_numpy(xf).to(torch.bfloat16) if xdt == "bf16" else torch.from_numpy(xf)).to(gpu)
    y0 = pkg.gemm_q4_0_native(w0, x).cpu().numpy()
    y1 = pkg.gemm_q4(w1, x).cpu().numpy()
    assert y0.tobytes() == y1.tobytes()
    ref = oracle.gemv_reference(b, x.to(torch.float32).cpu().numpy())
    assert oracle.maxrel(y0, ref) <= MAXREL
    res = torch.from_numpy(rng.standard_normal((M, n)).astype(np.float32)).to(gpu)
    yr = pkg.gemm_q4_0_native(w0, x, residual=res).cpu().numpy()
    assert yr.tobytes() == pkg.gemm_q4(w1, x, residual=res).cpu().numpy().tobytes()


def test_rejects_bad_arguments(gpu, pkg, oracle):
    say("q4_0 native bad arguments")
    rng = np.random.default_rng(9)
    b = oracle.random_q4_0_blocks_ref(64, 64, rng)
    w = pkg.pack_q4_0_native(b, 64, 64, "q4_0", device=gpu)
    with pytest.raises(ValueError):
        pkg.gemm_q4_0_native(w, torch.zeros(17, 64, dtype=torch.bfloat16, device=gpu))
    with pytest.raises(ValueError):
        pkg.pack_q4_0_native(b[:, :1], 64, 64, "q4_0", device=gpu)
    with pytest.raises(ValueError):
        pkg.pack_q4_0_native(b, 64, 64, "chunks", device=gpu)     # 18-byte blocks are not chunks
