"""q4_gemv_noalloc: the decode GEMV with its K-split partials in the library's static
device array instead of a caller workspace, called through the C ABI (ctypes).

It must give q4_gemv's bits exactly (same kernels, same split order) on two calls in a row,
the second smaller than the first, so a stale partial of the first call could not hide;
and meet the 1e-3 bar against the fp64 oracle. The argument checks run on the CPU."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

from conftest import say

SCRATCH_BYTES = 8 << 20          # Q4MI_NOALLOC_SCRATCH_BYTES


def test_scratch_covers_every_split_shape(lib):
    """Under the split policy no M <= 16 shape needs more partials than the array holds."""
    worst = 0
    for g in range(1, 1100):
        for k in (256, 2048, 4096, 14336, 65536):
            worst = max(worst, lib.q4_gemv_workspace_bytes(16, g * 64, k))
    assert 0 < worst <= SCRATCH_BYTES


def test_noalloc_argument_errors(lib):
    """Rejected before any HIP call (no GPU needed)."""
    fake = C.c_void_p(0x1000)
    assert lib.q4_gemv_noalloc(fake, fake, 7, fake, 1, 64, 32, None) == -2       # dtype
    assert lib.q4_gemv_noalloc(fake, fake, 1, fake, 17, 64, 32, None) == -5      # M > 16
    assert lib.q4_gemv_noalloc(fake, fake, 1, fake, 1, 63, 32, None) == -1       # N % 64
    assert lib.q4_gemv_noalloc(fake, fake, 1, fake, 1, 64, 48, None) == -1       # K % 32
    assert lib.q4_gemv_noalloc(fake, fake, 1, fake, 0, 64, 32, None) == 0        # nothing to do


def _call(lib, fn, *args):
    st = fn(*args)
    assert st == 0, f"{fn.__name__}: status {st} ({lib.q4mi_strerror(st).decode()})"


@pytest.mark.gpu
def test_noalloc_matches_q4_gemv_on_two_calls(gpu, pkg, lib, oracle):
    stream = C.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    rng = np.random.default_rng(77)
    # first a large split call (4096 x 14336 at M = 16: 16 splits, 4 MiB of partials), then a
    # smaller one (1024 x 2048 at M = 3) that reuses the start of the same array
    for (M, N, K, xdt) in ((16, 4096, 14336, "bf16"), (3, 1024, 2048, "f32")):
        say(f"noalloc M={M} N={N} K={K} x={xdt}")
        need = lib.q4_gemv_workspace_bytes(M, N, K)
        assert 0 < need <= SCRATCH_BYTES
        blocks = oracle.baseline_q4_1_blocks(N, K, rng)
        w = pkg.pack_q4_1(blocks, gpu)
        x = rng.standard_normal((M, K)).astype(np.float32)
        xt = (torch.from_numpy(x).to(torch.bfloat16) if xdt == "bf16" else torch.from_numpy(x)).to(gpu)
        enum = 1 if xdt == "bf16" else 0
        y_na = torch.full((M, N), float("nan"), device=gpu)
        y_ws = torch.full((M, N), float("nan"), device=gpu)
        ws = torch.empty(need, dtype=torch.uint8, device=gpu)
        _call(lib, lib.q4_gemv_noalloc, w.data.data_ptr(), xt.data_ptr(), enum, y_na.data_ptr(), M, N, K, stream)
        _call(lib, lib.q4_gemv, w.data.data_ptr(), xt.data_ptr(), enum, y_ws.data_ptr(), M, N, K,
              ws.data_ptr(), need, stream)
        torch.cuda.synchronize()
        a, b = y_na.cpu().numpy(), y_ws.cpu().numpy()
        assert a.tobytes() == b.tobytes(), "q4_gemv_noalloc differs from q4_gemv"
        ref = oracle.gemv_reference(blocks, xt.to(torch.float32).cpu().numpy())
        assert oracle.maxrel(a, ref) <= 1e-3
