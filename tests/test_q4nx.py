"""The .q4nx container and its chunk formats, on the CPU.

Pins, each independent of the formula it checks:
* the reference's own C++ container reader (src/open_qwen36/q4nx_file.cpp, built into
  oracle/_ref/q4nx_dump by oracle/Makefile): tensor table, chunk sizes, metadata, raw bytes
  and BF16 / F32 decodes, against this build's parser (openflowlm-next_amd/q4nx.py);
* the signed quantiser's transcode: its q4_1 reading equals d * int4(q) read straight off
  the signed bytes, exactly;
* the q8 requant: the reference's own property test (test_qwen35.py:631-654: every value
  within d/2 of its reading, a real quantisation) plus the directed-rounding bounds
  (m <= block min, m + 15 d >= block max) and exactness on constant blocks.
* the reference's FNV-1a goldens over its shared q8 vector (test_qwen35.py:694-703,
  :890-903; pools_test.cpp:33-53): requant_q4_1, the exact split's hi and lo planes and a
  plain transpose, each reproduced by the oracle byte for byte (the reference hashes from
  its own offset basis, 1469598103934665603).
"""
from __future__ import annotations

import importlib
import subprocess
from pathlib import Path

import numpy as np
import pytest

from q4nx_writer import write_q4nx

ROOT = Path(__file__).resolve().parents[1]
Q4NX_DUMP = ROOT / "oracle" / "_ref" / "q4nx_dump"


def q4nx_mod():
    return importlib.import_module("openflowlm-next_amd.q4nx")


def _container(tmp_path, oracle):
    rng = np.random.default_rng(4)
    q41 = oracle.pack_q4_1_pool(oracle.random_q4_1_blocks_ref(128, 512, rng), 1).reshape(-1, 5120)
    tensors = [
        ("model.layers.0.mlp.down_proj.weight", "I8", (q41.shape[0], 5120), q41),
        ("model.layers.0.self_attn.q_proj.weight", "I8", (8, 5120), oracle.random_signed_pool(8, rng)),
        ("model.layers.0.linear_attn.ssm_out_proj.weight", "I8", (8, 8704), oracle.random_q8_chunks(8, rng)),
        ("model.layers.0.mlp.gate_proj.weight", "I8", (4, 4736), oracle.q4k_vector(4)),
        ("model.embed_tokens.weight", "BF16", (16, 64),
         oracle.f32_to_bf16(rng.standard_normal((16, 64)).astype(np.float32))),
        ("model.norm.weight", "F32", (64,), rng.standard_normal(64).astype(np.float32)),
        ("model.layers.0.mlp.up_proj.weight", "I8", (8, 1280), rng.integers(0, 256, (8, 1280), dtype=np.uint8)),
    ]
    p = tmp_path / "m.q4nx"
    write_q4nx(p, tensors, {"format": "q4nx-1.0.2", "adapter": "none"}, pad_header_to=8)
    return p, tensors


def _ref(path, outdir, names, metas=()):
    if not Q4NX_DUMP.is_file():
        pytest.skip("oracle/_ref/q4nx_dump not built (the reference sources are absent)")
    args = [str(Q4NX_DUMP), str(path), str(outdir)]
    for k in metas:
        args += ["--meta", k]
    r = subprocess.run(args + list(names), capture_output=True, text=True, timeout=60)
    return r.returncode, [line.split("\t") for line in r.stdout.splitlines()]


def test_table_and_bytes_match_the_reference_reader(tmp_path, oracle):
    p, tensors = _container(tmp_path, oracle)
    names = [t[0] for t in tensors]
    rc, recs = _ref(p, tmp_path, names, ["format", "adapter", "absent"])
    assert rc == 0, recs
    assert recs[0] == ["count", str(len(tensors))]
    meta = {r[1]: r[2] for r in recs if r[0] == "meta"}
    with q4nx_mod().Q4NXFile(p) as f:
        assert f.metadata == {"format": "q4nx-1.0.2", "adapter": "none"}
        assert meta == {"format": "q4nx-1.0.2", "adapter": "none", "absent": ""}
        for r in (r for r in recs if r[0] == "tensor"):
            _, idx, name, dtype, shape, start, end, cb = r
            t = f.tensors[name]
            assert (t["dtype"], t["shape"], t["start"], t["end"]) == \
                (dtype, tuple(int(s) for s in shape.split(",")), int(start), int(end))
            assert f.chunk_bytes_of(name) == int(cb)
            assert f.raw(name).tobytes() == (tmp_path / f"{idx}.bin").read_bytes()
            if dtype in ("BF16", "F32"):
                ref = np.fromfile(tmp_path / f"{idx}.f32", np.float32)
                assert np.array_equal(f.array(name).reshape(-1), ref)


def test_chunk_formats_are_told_apart(tmp_path, oracle):
    p, _ = _container(tmp_path, oracle)
    with q4nx_mod().Q4NXFile(p) as f:
        assert f.quant_format_of("model.layers.0.mlp.down_proj.weight") == "q4_1"
        assert f.quant_format_of("model.layers.0.self_attn.q_proj.weight") == "q4_0"
        assert f.quant_format_of("model.layers.0.linear_attn.ssm_out_proj.weight") == "q8"
        assert f.quant_format_of("model.layers.0.mlp.gate_proj.weight") == "q4_k"
        assert f.quant_format_of("model.norm.weight") == ""
        with pytest.raises(q4nx_mod().Q4NXError, match="up_proj.*1280.*smaller chunk geometry"):
            f.quant_format_of("model.layers.0.mlp.up_proj.weight")
        with pytest.raises(q4nx_mod().Q4NXError, match="no tensor"):
            f.raw("nope")


def test_declared_format_wins(tmp_path, oracle):
    rng = np.random.default_rng(1)
    sig = oracle.random_signed_pool(2, rng)
    p = tmp_path / "d.q4nx"
    write_q4nx(p, [("w", "I8", (2, 5120), sig)], {"quant_format.w": "q4_1"})
    with q4nx_mod().Q4NXFile(p) as f:
        assert f.quant_format_of("w") == "q4_1"


@pytest.mark.parametrize("cut", [4, 20, -10])
def test_damaged_files_are_refused(tmp_path, oracle, cut):
    p, _ = _container(tmp_path, oracle)
    b = p.read_bytes()
    bad = tmp_path / "bad.q4nx"
    bad.write_bytes(b[:cut])
    with pytest.raises(q4nx_mod().Q4NXError):
        q4nx_mod().Q4NXFile(bad)


def test_signed_transcode_reads_exactly_the_signed_values(oracle):
    rng = np.random.default_rng(2)
    sig = oracle.random_signed_pool(6, rng)
    got = oracle.dq_chunks_q4_1(oracle.signed_pool_to_q4_1(sig)).astype(np.float64)
    assert np.array_equal(got, oracle.signed_pool_values(sig))
    # and read as q4_1 unchanged they would be the one-sided, wrong values
    assert not np.array_equal(oracle.dq_chunks_q4_1(sig).astype(np.float64), oracle.signed_pool_values(sig))


def test_requant_is_within_half_a_step(oracle):
    """test_qwen35.py:631-654, restated: every q8 value within d/2 of its q4_1 reading,
    the nibble in range, and a real quantisation."""
    rng = np.random.default_rng(7)
    src = oracle.random_q8_chunks(12, rng)
    got = oracle.requant_q4_1(src)
    assert got.shape == (12, 5120) and got.dtype == np.uint8
    a = oracle.q8_chunk_values(src).astype(np.float64)
    b = oracle.dq_chunks_q4_1(got).astype(np.float64)
    d = oracle.bf16_to_f32(np.ascontiguousarray(got[:, :512]).view(np.uint16))
    dd = d[:, oracle.CHUNK_META_IDX].reshape(-1, 32, 8, 32).astype(np.float64)
    assert np.all(np.abs(a - b) <= dd / 2 + 1e-30)
    assert 0.0 < np.abs(a - b).max() < dd.max()


def test_requant_directed_rounding_covers_each_block(oracle):
    rng = np.random.default_rng(9)
    src = oracle.random_q8_chunks(6, rng)
    src[0, 512:] = 4                   # chunk 0: every block constant, 4 * scale exact in bf16
    v = oracle.q8_chunk_values(src).astype(np.float64)
    got = oracle.requant_q4_1(src)
    meta = oracle.bf16_to_f32(np.ascontiguousarray(got[:, :1024]).view(np.uint16)).astype(np.float64)
    slot = (np.arange(8)[None, :] * 32 + np.arange(32)[:, None])
    d, m = meta[:, :256][:, slot], meta[:, 256:][:, slot]            # [n, r, block]
    assert (m <= v.min(-1)).all() and (m + 15 * d >= v.max(-1)).all()
    assert np.array_equal(oracle.dq_chunks_q4_1(got[:1]).astype(np.float64), v[:1])


def _fnv(oracle, b):
    return oracle.fnv1a64(bytes(b))


def test_reference_transpose_golden(oracle):
    """test_qwen35.py:700-702: FNV-1a of a plain transpose of (i*37+11) & 0xFF."""
    t = np.frombuffer(bytes(((i * 37 + 11) & 0xFF) for i in range(32 * 64 * 2)), np.uint8)
    td = np.ascontiguousarray(t.reshape(32, 64, 2).transpose(1, 0, 2)).reshape(-1)
    assert _fnv(oracle, td) == 0xB27D0B6F7149FD83


def test_shared_q8_vector_follows_the_lcg(oracle):
    """The vector both reference packers hash, checked by hand against its LCG for the
    first chunk's first scale and code."""
    v = oracle.shared_q8_vector(2)
    s = 0x9E3779B9
    s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
    assert int(v[0, :2].view(np.uint16)[0]) == 0x3B00 | (s >> 24)
    for _ in range(256):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
    assert int(v[0, 512]) == s >> 24
    assert v.shape == (2, 8704)


def test_reference_requant_golden(oracle):
    """test_qwen35.py:698-699 (and pools_test.cpp:37): requant_q4_1 of the shared vector."""
    assert _fnv(oracle, oracle.requant_q4_1(oracle.shared_q8_vector(12))) == 0x4AC3BABAD266DD49


def test_reference_split_goldens(oracle):
    """test_qwen35.py:902-903: the exact q8 split's hi and lo chunks of the shared vector."""
    v = oracle.shared_q8_vector(12)
    assert _fnv(oracle, oracle.split_q8_chunks(v, 0)) == 0x011857DF63D905CE
    assert _fnv(oracle, oracle.split_q8_chunks(v, 1)) == 0x1A95B8AE739769D2


def test_q8_split_planes_sum_to_the_q8_values_exactly(oracle):
    """test_qwen35.py:890-903's property: the hi and lo q4_1 readings add up to every q8
    value exactly (the requant is lossy; this is not), from chunks and from GGUF Q8_0."""
    rng = np.random.default_rng(12)
    n, k = 128, 512
    src = oracle.random_q8_chunks((n // 32) * (k // 256), rng)
    src[0, 512:520] = [0x80, 0x7F, 0xFF, 0x00, 0x01, 0xF0, 0x0F, 0x88]     # -128, 127, -1, 0, 1, -16, 15, -120
    for s16, q in (oracle.q8_chunks_rows(src, n, k, 1), oracle.q8_0_rows(oracle.random_q8_0_blocks(n, k, rng))):
        total = np.zeros((n, k))
        for part in (0, 1):
            d16, m16, codes = oracle.q8_split_parts(s16, q, part)
            assert codes.max() <= 15
            total += oracle.dequant_mx(oracle.pack_mx_from_parts(d16, m16, codes), n, k).astype(np.float64)
        assert np.array_equal(total, oracle.q8_values(s16, q))
    # the chunk reader agrees with the chunk values read straight off the layout
    s16, q = oracle.q8_chunks_rows(src, n, k, 1)
    v = oracle.q8_chunk_values(src).reshape(-1, 32, 256)
    assert np.array_equal(oracle.q8_values(s16, q)[:32, :256], v[0])


@pytest.mark.parametrize("kind", ["q4_1", "q4_0"])
def test_gguf_direct_pool_reads_the_gguf_values_exactly(oracle, kind):
    """gguf_pool.py's self-test (:388+), restated: the direct pool's own f32 reading equals
    the GGUF blocks' fp16-scale dequant bit for bit (the widening is exact), and the
    q8 pool holds every d * q exactly."""
    rng = np.random.default_rng(21)
    n, k = 128, 512
    blocks = oracle.random_q4_1_blocks_ref(n, k, rng) if kind == "q4_1" else oracle.random_q4_0_blocks_ref(n, k, rng)
    for rs in (1, 2):
        pool = oracle.pack_gguf_pool_f32(blocks, rs)
        got = oracle.dequant_gguf_pool_f32(pool, n, k, rs)
        assert got.tobytes() == oracle.dequant_q4_1(blocks, bf16_scales=False).tobytes()
    q8b = oracle.random_q8_0_blocks(n, k, rng)
    pool8 = oracle.pack_gguf_pool_q8_f32(q8b, 1).reshape(-1, 9216)
    d = np.ascontiguousarray(q8b[..., 0:2]).view(np.float16).reshape(n, k // 32).astype(np.float64)
    q = np.ascontiguousarray(q8b[..., 2:]).view(np.int8).reshape(n, k).astype(np.float64)
    want = np.repeat(d, 32, axis=1) * q
    sc = np.ascontiguousarray(pool8[0, :1024]).view(np.float32).astype(np.float64)
    code = np.ascontiguousarray(pool8[0, 1024:]).view(np.int8)[oracle.CHUNK_CODE_IDX].astype(np.float64)
    got8 = (code * sc[oracle.CHUNK_META_IDX]).reshape(32, 8, 32).reshape(32, 256)
    assert np.array_equal(got8, want[:32, :256])


def test_decode_benchmark_harness_rejects_what_it_cannot_read(tmp_path):
    """bench.q4nx_decode_harness: a non-q4_1 tensor and a shape the chunks do not tile are
    refused before any GPU work."""
    import bench
    rng = np.random.default_rng(3)
    write_q4nx(tmp_path / "model.q4nx", [("q8", "I8", (4, 8704), rng.integers(-128, 128, (4, 8704), dtype=np.int8)),
                                         ("q4", "I8", (4, 5120), rng.integers(1, 256, (4, 5120), dtype=np.uint8)),
                                         ("norm", "BF16", (64,), np.zeros(64, np.uint16))])
    with pytest.raises(ValueError, match="q4_1"):
        bench.q4nx_decode_harness(tmp_path, "q8", None)
    with pytest.raises(ValueError, match="q4_1"):
        bench.q4nx_decode_harness(tmp_path, "norm", None)
    with pytest.raises(ValueError, match="do not tile"):
        bench.q4nx_decode_harness(tmp_path, "q4", (128, 512))
