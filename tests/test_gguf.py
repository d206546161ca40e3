"""GGUF in, and the Q4_K source formats, on the CPU.

Pins, each independent of the formula it checks:

* the reference's own C++ GGUF reader (src/gguf/gguf_file.cpp, built into
  oracle/_ref/gguf_dump by oracle/Makefile): tensor table, metadata and its f32 dequant
  of every tensor -- Q4_K, Q4_1, Q4_0, F32, F16, BF16 -- against this build's parser
  (openflowlm-next_amd/gguf.py) and the oracle's Q4_K law;
* an exhaustive encode -> decode of the packed 6-bit (scale, min) pairs, the encoder
  written in the opposite direction (llama.cpp's quantizer packing);
* planted mistakes in the oracle that the reference reader catches;
* for the container Q4_K chunk transcode (recipes/pack.py:266-310), the reference's own
  property checks (test_quant_q4k.py:153-197): within a bf16 half-ulp of the exact value,
  exact nibble de-interleave, no move of the scale index, non-positive mins.
"""
from __future__ import annotations

import importlib
import subprocess
from pathlib import Path

import numpy as np
import pytest

from gguf_writer import ARR, BOOL, F32, F64, I32, STR, U8, U32, U64, write_gguf

ROOT = Path(__file__).resolve().parents[1]
GGUF_DUMP = ROOT / "oracle" / "_ref" / "gguf_dump"


def gguf_mod():
    return importlib.import_module("openflowlm-next_amd.gguf")


def _f16_bytes(a) -> np.ndarray:
    return np.asarray(a, np.float16).view(np.uint8)


def _bf16_bytes(a, oracle) -> np.ndarray:
    return oracle.f32_to_bf16(np.asarray(a, np.float32)).view(np.uint8)


def _model(tmp_path, oracle, alignment=None):
    """A file with one tensor of every type the reader takes, and mixed metadata."""
    rng = np.random.default_rng(11)
    tensors = [
        ("blk.0.ffn_gate.weight", "Q4_K", (128, 512), oracle.random_q4_k_blocks(128, 512, rng)),
        ("blk.0.ffn_up.weight", "Q4_1", (64, 256), oracle.random_q4_1_blocks_ref(64, 256, rng)),
        ("blk.0.ffn_down.weight", "Q4_0", (64, 96), oracle.random_q4_0_blocks_ref(64, 96, rng)),
        ("output_norm.weight", "F32", (96,), rng.standard_normal(96).astype(np.float32)),
        ("blk.0.attn_norm.weight", "F16", (3, 40), _f16_bytes(rng.standard_normal((3, 40)))),
        ("token_embd.weight", "BF16", (5, 64), _bf16_bytes(rng.standard_normal((5, 64)), oracle)),
    ]
    meta = [
        ("general.architecture", STR, "llama"),
        ("llama.block_count", U32, 1),
        ("llama.context_length", U64, 8192),
        ("llama.rope.freq_base", F32, 500000.0),
        ("llama.attention.layer_norm_rms_epsilon", F64, 1e-5),
        ("llama.head_count_kv", ARR, (I32, [8, 0, 8])),
        ("tokenizer.ggml.tokens", ARR, (STR, ["<s>", "</s>", "héllo"])),
        ("general.flag", BOOL, True),
        ("general.small", U8, 7),
    ]
    p = tmp_path / "model.gguf"
    write_gguf(p, tensors, meta, alignment=alignment)
    return p, tensors, meta


def _ref_dump(path, outdir, keys=()):
    if not GGUF_DUMP.is_file():
        pytest.skip("oracle/_ref/gguf_dump not built (the reference sources are absent)")
    r = subprocess.run([str(GGUF_DUMP), str(path), str(outdir), *keys], capture_output=True, text=True,
                       timeout=60)
    recs = [line.split("\t") for line in r.stdout.splitlines()]
    return r.returncode, recs


# --------------------------------------------------------------------------
# the parser against the reference reader
# --------------------------------------------------------------------------

@pytest.mark.parametrize("alignment", [None, 64])
def test_tensor_table_matches_the_reference_reader(tmp_path, oracle, alignment):
    p, tensors, _ = _model(tmp_path, oracle, alignment)
    rc, recs = _ref_dump(p, tmp_path)
    assert rc == 0, recs
    ref = {r[2]: r for r in recs if r[0] == "tensor"}
    with gguf_mod().GGUFFile(p) as f:
        assert set(f.tensors) == set(ref) == {t[0] for t in tensors}
        for name, tname, shape, _ in tensors:
            t = f.tensor(name)
            _, _, _, rtype, rdims, roff = ref[name]
            assert t.type_name == rtype == tname
            assert tuple(int(d) for d in rdims.split(",")) == tuple(reversed(shape)) == tuple(reversed(t.shape))
            assert t.offset == f.data_start + int(roff)
            assert t.offset % (alignment or 32) == 0


def test_every_tensor_dequantizes_as_the_reference_reads_it(tmp_path, oracle):
    """The reference's f32 of each tensor, bit for bit: Q4_K through the oracle's law,
    Q4_1/Q4_0 with their fp16 scales (no bf16 narrowing here: this is the file's value),
    F32/F16/BF16 through the parser's own arrays."""
    p, tensors, _ = _model(tmp_path, oracle)
    rc, recs = _ref_dump(p, tmp_path)
    assert rc == 0, recs
    idx = {r[2]: int(r[1]) for r in recs if r[0] == "tensor"}
    with gguf_mod().GGUFFile(p) as f:
        for name, tname, shape, payload in tensors:
            got_ref = np.fromfile(tmp_path / f"{idx[name]}.f32", np.float32).reshape(shape)
            if tname == "Q4_K":
                mine = oracle.dequant_q4_k(f.blocks(name))
            elif tname in ("Q4_1", "Q4_0"):
                mine = oracle.dequant_q4_1(f.blocks(name), bf16_scales=False)
            else:
                mine = f.array(name)
            assert mine.shape == got_ref.shape, name
            assert mine.tobytes() == got_ref.tobytes(), f"{name} ({tname}) differs from the reference reader"


def test_metadata_matches_the_reference_reader(tmp_path, oracle):
    p, _, meta = _model(tmp_path, oracle)
    keys = [m[0] for m in meta]
    rc, recs = _ref_dump(p, tmp_path, keys)
    assert rc == 0, recs
    ref = {r[1]: r[2] for r in recs if r[0] == "kv"}
    with gguf_mod().GGUFFile(p) as f:
        md = f.metadata
        assert md["general.architecture"] == ref["general.architecture"] == "llama"
        assert md["llama.block_count"] == int(ref["llama.block_count"]) == 1
        assert md["llama.context_length"] == int(ref["llama.context_length"]) == 8192
        assert md["llama.rope.freq_base"] == float(ref["llama.rope.freq_base"]) == 500000.0
        assert abs(md["llama.attention.layer_norm_rms_epsilon"] - 1e-5) < 1e-20
        assert md["llama.head_count_kv"] == [int(v) for v in ref["llama.head_count_kv"].split(",")] == [8, 0, 8]
        assert md["tokenizer.ggml.tokens"] == ref["tokenizer.ggml.tokens"].split(",") == ["<s>", "</s>", "héllo"]
        assert md["general.flag"] is True and ref["general.flag"] == "1"
        assert md["general.small"] == int(ref["general.small"]) == 7


def test_a_planted_q4k_mistake_is_caught_by_the_reference_reader(tmp_path, oracle):
    """Two plausible slips in the Q4_K law -- odd sub-blocks reading the low nibble, and
    the high scale bits taken from byte j instead of j - 4 -- each differ from the
    reference's dequant, so the comparison above has teeth."""
    p, tensors, _ = _model(tmp_path, oracle)
    rc, recs = _ref_dump(p, tmp_path)
    assert rc == 0
    idx = {r[2]: int(r[1]) for r in recs if r[0] == "tensor"}
    name, _, shape, _ = tensors[0]
    ref = np.fromfile(tmp_path / f"{idx[name]}.f32", np.float32).reshape(shape)
    with gguf_mod().GGUFFile(p) as f:
        b = np.array(f.blocks(name))
    D, M, q = oracle.unpack_q4_k_blocks(b)
    # slip 1: every sub-block reads the low nibbles of its 32-byte half
    qs = b[..., 16:144].reshape(b.shape[0], b.shape[1], 4, 32)
    q_low = np.repeat(qs & 0xF, 2, axis=2).reshape(q.shape)
    bad1 = q_low.astype(np.float32) * np.repeat(D, 32, 1) + np.repeat(M, 32, 1)
    assert not np.array_equal(bad1, ref)
    # slip 2: sub-blocks 4..7 take their scale's top bits from byte j
    s = b[..., 4:16].astype(np.int32)
    D2 = D.reshape(b.shape[0], b.shape[1], 8).copy()
    d16 = np.ascontiguousarray(b[..., 0:2]).view(np.float16)[..., 0].astype(np.float32)
    for j in range(4, 8):
        D2[..., j] = d16 * ((s[..., j + 4] & 0xF) | ((s[..., j] >> 6) << 4)).astype(np.float32)
    bad2 = q.astype(np.float32) * np.repeat(D2.reshape(D.shape), 32, 1) + np.repeat(M, 32, 1)
    assert not np.array_equal(bad2, ref)
    # and the right law agrees
    assert np.array_equal(q.astype(np.float32) * np.repeat(D, 32, 1) + np.repeat(M, 32, 1), ref)


# --------------------------------------------------------------------------
# the parser on its own
# --------------------------------------------------------------------------

def test_blocks_are_zero_copy_views_of_the_file(tmp_path, oracle):
    p, tensors, _ = _model(tmp_path, oracle)
    with gguf_mod().GGUFFile(p) as f:
        b = f.blocks("blk.0.ffn_gate.weight")
        assert b.shape == (128, 2, 144) and not b.flags.owndata and not b.flags.writeable
        assert np.array_equal(b, tensors[0][3])
        assert np.array_equal(f.blocks("blk.0.ffn_down.weight"), tensors[2][3])
        assert f.array("output_norm.weight").shape == (96,)
        del b


@pytest.mark.parametrize("mutate,msg", [
    (lambda b: b"GGUX" + b[4:], "bad magic"),
    (lambda b: b[:4] + (1).to_bytes(4, "little") + b[8:], "version 1"),
    (lambda b: b[:40], "truncated|runs past"),
    (lambda b: b"", "not a GGUF"),
])
def test_bad_files_are_refused_with_a_reason(tmp_path, oracle, mutate, msg):
    p, _, _ = _model(tmp_path, oracle)
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(mutate(p.read_bytes()))
    with pytest.raises(gguf_mod().GGUFError, match=msg):
        gguf_mod().GGUFFile(bad)


def test_unknown_type_and_short_data_are_refused(tmp_path, oracle):
    g = gguf_mod()
    p = tmp_path / "k.gguf"
    write_gguf(p, [("w", "Q8_0", (64, 64), np.zeros((64, 2, 34), np.uint8))])
    raw = bytearray(p.read_bytes())
    i = raw.find(b"w") + 1 + 4 + 16          # name, n_dims, two dims -> the type field
    raw[i:i + 4] = (13).to_bytes(4, "little")  # Q5_K: not a type this reader takes
    (tmp_path / "t.gguf").write_bytes(bytes(raw))
    with pytest.raises(g.GGUFError, match="ggml type 13"):
        g.GGUFFile(tmp_path / "t.gguf")
    (tmp_path / "s.gguf").write_bytes(p.read_bytes()[:-100])
    with pytest.raises(g.GGUFError, match="runs past the file"):
        g.GGUFFile(tmp_path / "s.gguf")


def test_packed_refuses_what_the_kernels_cannot_take(tmp_path, oracle):
    p, _, _ = _model(tmp_path, oracle)
    with gguf_mod().GGUFFile(p) as f:
        with pytest.raises(gguf_mod().GGUFError, match="F32"):
            f.packed("output_norm.weight")
        with pytest.raises(gguf_mod().GGUFError, match="no tensor"):
            f.tensor("nope")


# --------------------------------------------------------------------------
# the Q4_K law
# --------------------------------------------------------------------------

def _encode_scale_min(sc, mn) -> np.ndarray:
    """llama.cpp's packing of eight 6-bit (scale, min) pairs into 12 bytes, written in
    the encoding direction: pairs 0-3 whole in bytes j and j+4; pairs 4-7 low nibbles in
    byte j+4, top two bits in the spare bits 6-7 of bytes j-4 (scale) and j (min)."""
    out = np.zeros(12, np.int32)
    for j in range(8):
        if j < 4:
            out[j] |= sc[j]
            out[j + 4] |= mn[j]
        else:
            out[j + 4] = (sc[j] & 0xF) | ((mn[j] & 0xF) << 4)
            out[j - 4] |= (sc[j] >> 4) << 6
            out[j] |= (mn[j] >> 4) << 6
    return out.astype(np.uint8)


def test_scale_min_unpacking_is_the_inverse_of_the_packing(oracle):
    """Every (scale, min) value for every sub-block, through encode then decode."""
    rng = np.random.default_rng(5)
    packed, want_s, want_m = [], [], []
    for v in range(64 * 64):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        sc[v % 8], mn[v % 8] = v // 64, v % 64
        packed.append(_encode_scale_min(sc, mn))
        want_s.append(sc)
        want_m.append(mn)
    packed = np.stack(packed)
    for j in range(8):
        s6, m6 = oracle.q4_k_scale_min(packed, j)
        assert np.array_equal(s6, np.stack(want_s)[:, j]) and np.array_equal(m6, np.stack(want_m)[:, j]), j


def test_a_hand_built_q4k_block_reads_its_closed_form(oracle):
    """One super-block with d = 0.5, dmin = 0.25, sub-block j scale j+1 and min 2j+3, code
    (value index) % 16: value(i) = 0.5 (j+1) (i % 16) - 0.25 (2j+3)."""
    b = np.zeros((1, 1, 144), np.uint8)
    b[0, 0, 0:2] = _f16_bytes([0.5])
    b[0, 0, 2:4] = _f16_bytes([0.25])
    b[0, 0, 4:16] = _encode_scale_min(np.arange(8) + 1, 2 * np.arange(8) + 3)
    codes = np.arange(256) % 16
    for c in range(4):       # byte 32c + l: value 64c + l low, 64c + 32 + l high
        b[0, 0, 16 + 32 * c:48 + 32 * c] = codes[64 * c:64 * c + 32] | (codes[64 * c + 32:64 * c + 64] << 4)
    i = np.arange(256)
    j = i // 32
    want = 0.5 * (j + 1) * (i % 16) - 0.25 * (2 * j + 3)
    assert np.array_equal(oracle.dequant_q4_k(b)[0], want.astype(np.float32))
    D, M, q = oracle.unpack_q4_k_blocks(b)
    assert np.array_equal(q[0], codes) and np.array_equal(D[0], 0.5 * (np.arange(8) + 1))
    assert np.array_equal(M[0], -0.25 * (2 * np.arange(8) + 3))


def test_q4k_to_mx_is_the_bf16_collapse_and_nothing_else(oracle):
    """The mx bytes hold the exact codes and bf16(D), bf16(M); their dequant is within a
    bf16 half-ulp of each term of the file's exact value, and the rounding is exercised."""
    rng = np.random.default_rng(3)
    b = oracle.random_q4_k_blocks(128, 1024, rng)
    D, M, q = oracle.unpack_q4_k_blocks(b)
    packed = oracle.pack_mx_q4_k(b)
    d16, m16, q2 = oracle.unpack_mx(packed, 128, 1024)
    assert np.array_equal(q2, q)
    assert np.array_equal(d16, oracle.f32_to_bf16(D)) and np.array_equal(m16, oracle.f32_to_bf16(M))
    got = oracle.dequant_mx(packed, 128, 1024)
    assert got.tobytes() == oracle.dequant_q4_k_bf16(b).tobytes()
    a = q.astype(np.float64) * np.repeat(D, 32, 1)
    c = np.repeat(M, 32, 1).astype(np.float64)
    err = np.abs(got.astype(np.float64) - (a + c))
    tol = (2.0 ** -8 + 2.0 ** -20) * (np.abs(a) + np.abs(c))
    assert (err <= tol).all() and err.max() > 0


# --------------------------------------------------------------------------
# the container Q4_K chunk transcode (recipes/pack.py:266-310)
# --------------------------------------------------------------------------

def test_container_transcode_is_within_a_bf16_half_ulp(oracle):
    """test_quant_q4k.py:153-180's bound: the transcoded pool chunk read as nib*d + m is
    the container's value to within 2^-8 (+2^-20) of each term, and moves somewhere."""
    src = oracle.q4k_vector(8)
    pool = oracle.q4k_chunks_to_pool(src)
    got = oracle.dq_chunks_q4_1(pool).astype(np.float64).reshape(8, 32, 256)
    S = oracle.bf16_to_f32(np.ascontiguousarray(src[:, 4608:4672]).view(np.uint16)).astype(np.float64)
    Mn = oracle.bf16_to_f32(np.ascontiguousarray(src[:, 4672:4736]).view(np.uint16)).astype(np.float64)
    g = np.arange(256) // 32
    sc = src[:, 0:256].reshape(8, 8, 32).astype(np.float64)[:, g, :].transpose(0, 2, 1)   # [c, r, k]
    mn = src[:, 256:512].reshape(8, 8, 32).astype(np.float64)[:, g, :].transpose(0, 2, 1)
    want = oracle.dequant_q4k_chunks_exact(src)
    c = Mn[:, :, None] * mn                       # the min term
    a = want - c                                  # the scale term (exact in f64)
    assert np.array_equal(a, S[:, :, None] * sc * np.round(a / np.where(sc == 0, 1, S[:, :, None] * sc)))
    tol = (2.0 ** -8 + 2.0 ** -20) * (np.abs(a) + np.abs(c))
    err = np.abs(got - want)
    assert (err <= tol).all() and err.max() > 0


def test_container_nibble_deinterleave_is_exact(oracle):
    """test_quant_q4k.py:183-191: the pool chunk's nibble (r//16)*4096 + 16k + r%16 is the
    container's byte 512 + 16k + r//2 nibble r%2, for every (r, k)."""
    src = oracle.q4k_vector(2)
    pool = oracle.q4k_chunks_to_pool(src)
    for c in range(2):
        nib = np.empty(8192, np.uint8)
        nib[0::2] = pool[c, 1024:] & 0xF
        nib[1::2] = pool[c, 1024:] >> 4
        for r in (0, 1, 14, 15, 16, 17, 30, 31):
            for k in (0, 1, 100, 255):
                byte = src[c, 512 + 16 * k + r // 2]
                want = (byte >> 4) if r % 2 else (byte & 0xF)
                assert nib[(r // 16) * 4096 + 16 * k + r % 16] == want


def test_container_scale_index_does_not_move(oracle):
    """test_quant_q4k.py:194-208: d[32g + r] = S[r] sc[32g + r] to a bf16 half-ulp, m
    likewise, and m is never positive (M is stored negated)."""
    src = oracle.q4k_vector(1)
    pool = oracle.q4k_chunks_to_pool(src)
    d = oracle.bf16_to_f32(np.ascontiguousarray(pool[0, :512]).view(np.uint16)).astype(np.float64)
    m = oracle.bf16_to_f32(np.ascontiguousarray(pool[0, 512:1024]).view(np.uint16)).astype(np.float64)
    S = oracle.bf16_to_f32(np.ascontiguousarray(src[0, 4608:4672]).view(np.uint16)).astype(np.float64)
    Mn = oracle.bf16_to_f32(np.ascontiguousarray(src[0, 4672:4736]).view(np.uint16)).astype(np.float64)
    r = np.arange(256) % 32
    want_d = S[r] * src[0, :256]
    want_m = Mn[r] * src[0, 256:512]
    assert (np.abs(d - want_d) <= 2.0 ** -8 * np.abs(want_d)).all()
    assert (np.abs(m - want_m) <= 2.0 ** -8 * np.abs(want_m)).all()
    assert (m <= 0).all()


def test_container_transcode_vector_and_hash_helpers(oracle):
    """The seeded vector's first bytes follow the LCG by hand, its S/M words carry the
    stated exponents and signs, and the FNV-1a helper meets the published test vectors."""
    v = oracle.q4k_vector(1)
    s = 0x9E3779B9
    first = []
    for _ in range(3):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        first.append(s >> 24)
    assert list(v[0, :3]) == first
    sm = np.ascontiguousarray(v[0, 4608:]).view(np.uint16)
    assert ((sm[:32] >> 8) == 0x3B).all() and ((sm[32:] >> 8) == 0xBB).all()
    # with the textbook offset basis the helper is the published FNV-1a ...
    assert oracle.fnv1a64(b"a", oracle.FNV_BASIS_TEXTBOOK) == 0xAF63DC4C8601EC8C
    assert oracle.fnv1a64(b"foobar", oracle.FNV_BASIS_TEXTBOOK) == 0x85944171F73967E8
    # ... and by default it starts from the reference's basis (test_pack_plan.py:184)
    assert oracle.FNV_BASIS_REF == 1469598103934665603
    assert oracle.fnv1a64(b"") == 1469598103934665603


def test_container_transcode_published_hash(oracle):
    """The reference's golden for q4k_to_q4_1 of its seeded vector (test_quant_q4k.py:52,
    pools_test.cpp:46), reproduced by the oracle's restatement."""
    assert oracle.fnv1a64(oracle.q4k_chunks_to_pool(oracle.q4k_vector(8)).tobytes()) == 0x685DC049EC1CA2D7
