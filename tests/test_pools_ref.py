"""The oracle's chunk transcodes against the reference's own C++ (src/open_qwen36/pools.cpp),
on the CPU.

oracle/Makefile compiles the reference's pools.cpp (with manifest.cpp, q4nx_file.cpp,
gguf_file.cpp and open_kernels/harness/stream_patch.hpp, all from /root/reference) behind
oracle/pools_dump.cpp into oracle/_ref/pools_dump, and the reference's own pools_test.cpp
into oracle/_ref/pools_test. Here:
* pools_test runs unchanged and must report "PASS (0 failures)": its FNV-1a goldens are the
  same numbers the reference's Python tests assert (pools_test.cpp:33-53);
* requant_q4_1 (pools.cpp:578-620), q4k_to_q4_1 (:642-663), q4_0_to_q4_1 (:622-640) and the
  exact q8 split (:343-370) are run on random chunks and on edge blocks by both the
  reference binary and the oracle, and the bytes must be identical.
The GPU repacks are held to the same oracle functions bit for bit (tests/test_gpu_q4nx.py,
tests/test_gpu_q8.py, tests/test_gpu_q4k.py), so this pins them to the reference's C++.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
REF = ROOT / "oracle" / "_ref"


def _need(name: str) -> Path:
    p = REF / name
    if not p.is_file():
        pytest.skip(f"oracle/_ref/{name} not built (the reference sources are absent)")
    return p


def _dump(tmp_path, op: str, src: np.ndarray) -> np.ndarray:
    exe = _need("pools_dump")
    fin, fout = tmp_path / f"{op}.in", tmp_path / f"{op}.out"
    np.ascontiguousarray(src, np.uint8).tofile(fin)
    r = subprocess.run([str(exe), op, str(fin), str(fout)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, f"pools_dump {op}: {r.stdout} {r.stderr}"
    return np.fromfile(fout, np.uint8).reshape(-1, 5120)


def test_reference_pools_test_passes():
    exe = _need("pools_test")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, cwd=str(REF))
    assert r.returncode == 0 and "PASS (0 failures)" in r.stdout, r.stdout[-2000:]


def _edge_q8_chunks(oracle, rng) -> np.ndarray:
    """q8 chunks whose blocks hit the requant's edges: constant blocks, all-negative and
    all-positive blocks, the code extremes -128 / 127, zero scales, tiny and large bf16
    scales, and blocks of a single nonzero value."""
    ch = oracle.random_q8_chunks(6, rng)
    code = ch[:, 512:].view(np.int8).reshape(6, 32, 256)           # raster [r][k] per chunk
    code[0] = 5                                                    # constant blocks
    code[1] = rng.integers(-128, -1, code[1].shape)                # all negative
    code[2] = rng.integers(1, 128, code[2].shape)                  # all positive
    code[3, :, ::2] = -128
    code[3, :, 1::2] = 127                                         # extremes
    code[4] = 0
    code[4, :, ::32] = 77                                          # one nonzero per block
    sc = ch[:, :512].view(np.uint16)
    sc[5, :64] = 0                                                 # zero scales
    sc[5, 64:128] = 0x0080                                         # smallest normal bf16
    sc[5, 128:192] = 0x4700                                        # 32768
    sc[5, 192:] = 0x3400 | rng.integers(0, 0x80, 64)
    return ch


def test_requant_matches_the_reference_cpp(tmp_path, oracle):
    rng = np.random.default_rng(31)
    src = np.concatenate([oracle.random_q8_chunks(24, rng), _edge_q8_chunks(oracle, rng),
                          oracle.shared_q8_vector(3)])
    got = oracle.requant_q4_1(src)
    want = _dump(tmp_path, "requant", src)
    bad = np.nonzero((got != want).any(1))[0]
    assert bad.size == 0, f"requant differs from pools.cpp in chunks {bad[:8]}"


@pytest.mark.parametrize("part,op", [(0, "split_hi"), (1, "split_lo")])
def test_q8_split_matches_the_reference_cpp(tmp_path, oracle, part, op):
    rng = np.random.default_rng(32 + part)
    src = np.concatenate([oracle.random_q8_chunks(16, rng), _edge_q8_chunks(oracle, rng)])
    assert np.array_equal(oracle.split_q8_chunks(src, part), _dump(tmp_path, op, src))


def test_q4k_transcode_matches_the_reference_cpp(tmp_path, oracle):
    rng = np.random.default_rng(33)
    src = np.concatenate([oracle.q4k_vector(8), rng.integers(0, 256, (16, 4736), dtype=np.uint8)])
    # random S/M words with finite bf16 values (exponent below 0xFF)
    sm = src[8:, 4608:].view(np.uint16)
    sm &= np.uint16(0xBFFF)
    got = oracle.q4k_chunks_to_pool(src)
    assert np.array_equal(got, _dump(tmp_path, "q4k", src))


def test_signed_q4_0_transcode_matches_the_reference_cpp(tmp_path, oracle):
    rng = np.random.default_rng(34)
    src = oracle.random_signed_pool(16, rng)
    src[0, :512] = 0                                               # zero scales
    assert np.array_equal(oracle.signed_pool_to_q4_1(src), _dump(tmp_path, "q4_0", src))


def test_a_planted_requant_slip_is_caught(tmp_path, oracle):
    """The comparison can fail: rounding d to nearest instead of up changes some bytes."""
    rng = np.random.default_rng(35)
    src = oracle.random_q8_chunks(8, rng)
    want = _dump(tmp_path, "requant", src)
    v = oracle.q8_chunk_values(src)
    m = oracle.bf16_to_f32(oracle._bf16_floor(v.min(-1)))
    d_near = oracle.f32_to_bf16(((v.max(-1) - m).astype(np.float32) / np.float32(15)).astype(np.float32))
    d_up = oracle._bf16_ceil(((v.max(-1) - m).astype(np.float32) / np.float32(15)).astype(np.float32))
    assert (d_near != d_up).any()
    slot = (np.arange(8)[None, :] * 32 + np.arange(32)[:, None]).reshape(-1)
    planted = oracle.requant_q4_1(src)
    meta = np.zeros((8, 256), np.uint16)
    meta[:, slot] = d_near.reshape(8, -1)
    planted[:, :512] = meta.view(np.uint8).reshape(8, 512)
    assert not np.array_equal(planted, want)
