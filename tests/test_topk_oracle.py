"""Pin the oracle of the lm_head's sampling epilogue (oracle.topk_reference /
sampler_view) against library routines and brute force, never its own formula:

* numpy's argmax (first index of the maximum) and descending sort;
* a brute-force tie rule: above the k-th value all ids, at it the lowest ids;
* torch's own f32 -> bf16 rounding, and explicit subnormal / signed-zero / NaN cases
  of the reference's greedy (src/open_qwen36/cli.cpp:103-113, sampler.cpp:355-430).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch


@pytest.mark.parametrize("mode", [0, 1])
def test_argmax_is_numpys_first_maximum(oracle, mode):
    rng = np.random.default_rng(mode)
    lg = rng.standard_normal((8, 5000)).astype(np.float32)
    lg[3, [10, 4000]] = 50.0                    # an exact tie: the lower id
    ids, vals = oracle.topk_reference(lg, 1, mode)
    view = oracle.sampler_view(lg) if mode else lg
    assert np.array_equal(ids[:, 0], np.argmax(view, axis=1))
    assert np.array_equal(vals[:, 0], view.max(axis=1))
    assert ids[3, 0] == 10


@pytest.mark.parametrize("k", [1, 5, 40, 64])
def test_topk_values_and_tie_rule_by_brute_force(oracle, k):
    rng = np.random.default_rng(k)
    lg = (rng.integers(0, 30, (6, 3000)) / 8).astype(np.float32)   # dense ties
    ids, vals = oracle.topk_reference(lg, k, 0)
    for m in range(6):
        row = lg[m]
        assert np.array_equal(vals[m], np.sort(row)[::-1][:k])
        t = vals[m, -1]
        above = np.flatnonzero(row > t)
        at = np.flatnonzero(row == t)[:k - len(above)]
        assert set(ids[m]) == set(above) | set(at)
        # within equal values, ids ascend; values never increase
        for a in range(k - 1):
            assert vals[m, a] > vals[m, a + 1] or (vals[m, a] == vals[m, a + 1] and ids[m, a] < ids[m, a + 1])


def test_sampler_view_is_bf16_rne_with_subnormals_flushed(oracle):
    rng = np.random.default_rng(2)
    v = (rng.standard_normal(20000) * 10.0 ** rng.integers(-3, 4, 20000)).astype(np.float32)
    want = torch.from_numpy(v).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(oracle.sampler_view(v), want)
    sub = np.array([1e-40, -1e-40, 1.1754942e-38, -0.0, 0.0, 1.2e-38], np.float32)
    got = oracle.sampler_view(sub)
    assert got[0] == 0 and got[1] == 0 and got[2] == 0 and not np.signbit(got[0]) and not np.signbit(got[1])
    assert got[5] != 0                              # the smallest normals stay


def test_special_values_order(oracle):
    """-0 ties with +0 (lower id wins), -inf ranks above NaN, an all-NaN row and an
    all -inf row give id 0 (the reference's best_id starts at 0 with strict '>')."""
    nan = np.float32(np.nan)
    lg = np.array([[-0.0, 0.0, -1.0, nan],
                   [nan, -np.inf, nan, -5.0],
                   [nan, nan, nan, nan],
                   [-np.inf, -np.inf, -np.inf, -np.inf]], np.float32)
    ids, _ = oracle.topk_reference(lg, 4, 0)
    assert list(ids[0]) == [0, 1, 2, 3]
    assert list(ids[1]) == [3, 1, 0, 2]
    assert ids[2, 0] == 0 and ids[3, 0] == 0


def test_short_rows_pad(oracle):
    ids, vals = oracle.topk_reference(np.array([[3.0, 1.0, 2.0]], np.float32), 5, 0)
    assert list(ids[0]) == [0, 2, 1, -1, -1] and np.isneginf(vals[0, 3:]).all()


def test_n_valid_skips_padding_rows(oracle):
    lg = np.array([[1.0, 2.0, 3.0, 100.0, 100.0]], np.float32)
    ids, _ = oracle.topk_reference(lg, 2, 1, n_valid=3)
    assert list(ids[0]) == [2, 1]
