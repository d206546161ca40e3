"""GPU parity of the lm_head's sampling epilogue (q4_logits_topk, q4_lm_head_topk)
against oracle.topk_reference: ids exact, values equal (NaN where NaN), on random
logits, dense ties, special values, padded vocabularies, and row lengths that take
one, two and three passes."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu


def _check(pkg, oracle, lg: np.ndarray, k: int, mode: int, n_valid=None, gpu=None):
    ids, vals = pkg.logits_topk(torch.from_numpy(lg).to(gpu), k, "sampler" if mode else "f32", n_valid)
    wi, wv = oracle.topk_reference(lg, k, mode, n_valid)
    gi, gv = ids.cpu().numpy(), vals.cpu().numpy()
    assert np.array_equal(gi, wi), f"ids differ at {np.argwhere(gi != wi)[:5].tolist()}"
    assert np.array_equal(gv, wv, equal_nan=True)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("n", [1, 100, 1023, 1024, 1025, 4097, 128256, 248320])
@pytest.mark.parametrize("k", [1, 8, 40, 64])
def test_random_logits(gpu, pkg, oracle, n, k, mode):
    say(f"topk n={n} k={k} mode={mode}")
    rng = np.random.default_rng(n + k + mode)
    lg = (rng.standard_normal((3, n)) * 4).astype(np.float32)
    _check(pkg, oracle, lg, k, mode, gpu=gpu)


@pytest.mark.parametrize("M", [1, 5, 16])
def test_three_passes_and_many_tokens(gpu, pkg, oracle, M):
    """300000 logits at k = 64: 74 blocks -> 74 sorted runs of 64 -> 2 blocks -> 1."""
    say(f"topk three passes M={M}")
    rng = np.random.default_rng(M)
    lg = rng.standard_normal((M, 300000)).astype(np.float32)
    _check(pkg, oracle, lg, 64, 1, gpu=gpu)


@pytest.mark.parametrize("mode", [0, 1])
def test_dense_ties_pick_the_lowest_ids(gpu, pkg, oracle, mode):
    say(f"topk ties mode={mode}")
    rng = np.random.default_rng(4)
    lg = (rng.integers(0, 40, (4, 128256)) / 16).astype(np.float32)
    for k in (1, 40, 64):
        _check(pkg, oracle, lg, k, mode, gpu=gpu)
    # values that differ in f32 but tie once rounded to bf16
    base = np.float32(3.0)
    lg2 = np.full((1, 5000), -10.0, np.float32)
    lg2[0, [4999, 17, 2500]] = [base + 1e-6, base, base + 2e-6]
    _check(pkg, oracle, lg2, 3, 1, gpu=gpu)
    ids, _ = pkg.logits_topk(torch.from_numpy(lg2).to(gpu), 1, "sampler")
    assert int(ids[0, 0]) == 17


def test_special_values(gpu, pkg, oracle):
    say("topk special values")
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    quiet_nan_low = np.array([0x7F800001], np.uint32).view(np.float32)[0]   # rounds to +inf in bf16
    rows = np.zeros((6, 300), np.float32)
    rows[0, :4] = [-0.0, 0.0, -1.0, nan]
    rows[0, 4:] = -3.0
    rows[1] = nan
    rows[2] = -inf
    rows[3, :] = np.array([1e-40, -1e-40, 0.0, -0.0] * 75, np.float32)      # subnormals and zeros
    rows[4, :] = -1.0
    rows[4, [7, 200]] = [inf, quiet_nan_low]
    rows[5, :] = np.linspace(-1, 1, 300, dtype=np.float32)
    rows[5, 150] = nan
    for mode in (0, 1):
        for k in (1, 4, 64):
            _check(pkg, oracle, rows, k, mode, gpu=gpu)


def test_short_rows_and_padded_vocabulary(gpu, pkg, oracle):
    say("topk short rows / n_valid")
    lg = np.array([[3.0, 1.0, 2.0]], np.float32)
    _check(pkg, oracle, lg, 5, 0, gpu=gpu)
    rng = np.random.default_rng(9)
    big = rng.standard_normal((2, 128256)).astype(np.float32)
    big[:, 128000:] = 1e30                    # padding rows past the vocabulary: never picked
    _check(pkg, oracle, big, 40, 1, n_valid=128000, gpu=gpu)


def test_rejects_bad_arguments(gpu, pkg):
    lg = torch.zeros((1, 10), device=gpu)
    with pytest.raises(Exception):
        pkg.logits_topk(lg, 65)
    with pytest.raises(Exception):
        pkg.logits_topk(lg, 0)
    with pytest.raises(Exception):
        pkg.logits_topk(lg, 1, "bf16")


@pytest.mark.parametrize("M", [1, 4])
def test_lm_head_topk_end_to_end(gpu, pkg, oracle, M):
    """The GEMV's logits meet the 1e-3 bar against fp64, and the ids are the oracle's
    pick over those same logits."""
    say(f"lm_head_topk M={M}")
    rng = np.random.default_rng(M)
    n, kdim, n_valid = 16384, 1024, 16000
    blocks = oracle.baseline_q4_1_blocks(n, kdim, rng)
    w = pkg.pack_q4_1(blocks, gpu)
    x = torch.from_numpy(rng.standard_normal((M, kdim)).astype(np.float32)).to(torch.bfloat16)
    ids, vals, logits = pkg.lm_head_topk(w, x.to(gpu), k=40, mode="sampler", n_valid=n_valid)
    lg = logits.cpu().numpy()
    ref = oracle.gemv_reference(blocks, x.to(torch.float32).numpy())
    assert oracle.maxrel(lg, ref) <= 1e-3
    wi, wv = oracle.topk_reference(lg, 40, 1, n_valid)
    assert np.array_equal(ids.cpu().numpy(), wi) and np.array_equal(vals.cpu().numpy(), wv)
    g1, _, _ = pkg.lm_head_topk(w, x.to(gpu), k=1, mode="sampler", n_valid=n_valid)
    assert np.array_equal(g1.cpu().numpy()[:, 0], wi[:, 0])
