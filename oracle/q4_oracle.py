r"""CPU oracle for the Q4_1 dequant-matmul path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this module, and only as the checker (or the timed CPU baseline).
The product path (``openflowlm-next_amd``) never calls it.

A numpy restatement, written from scratch, of the reference's CPU path for
this hot path (``/root/reference`` is read as text, never imported):

* GGUF Q4_1 / Q4_0 blocks        open_kernels/q4_1_pack.py:1-43, :58-101
* fp16 -> bf16 RNE narrowing      open_kernels/q4_1_pack.py:104-109, :129-130
* bf16 <-> f32 bit helpers        open_kernels/model/q4nx.py:95-102
* the 5120 B pool chunk layout    open_kernels/q4_1_pack.py:16-34, :112-142
* dequant of pool chunks          open_kernels/q4_1_pack.py:155-180,
                                  open_kernels/model/q4nx.py:105-126,
                                  utilities/benchmark-q4-decode.py:19-34
* fp64 GEMV reference             open_kernels/q4_1_pack.py:183-191
* T-token prefill reference       open_kernels/designs/gemm_q4_prefill/make_test.py:82-94
* MoE routing + expert reference  open_kernels/model/replica.py:121-140,
                                  open_kernels/designs/moe_batch/make_test.py:87-98
* Q4_0 -> Q4_1 transcode          open_kernels/recipes/pack.py:606-622
* GGUF Q4_K super-blocks          open_kernels/model/gguf_ref.py:224-250,
                                  src/gguf/gguf_file.cpp:611-635
* container Q4_K -> q4_1 chunks   open_kernels/recipes/pack.py:266-310,
                                  src/open_qwen36/pools.cpp:642-663
* native q8 values (s * q)        open_kernels/recipes/pack.py:94-117 (the split's sum),
                                  open_kernels/designs/gemv_q4/gemv_q8.h
* native Q4_K values              open_kernels/designs/gemm_q4/gemm_q4.h:456-507
  (value d sc nib + mcoef mn of the container chunk; d sc q - dmin min of GGUF)
* the 4608 B Q4_0-native chunk    open_kernels/q4_1_pack.py:145-152 (read with
  m = -8 d by designs/gemv_q4/gemv_q4.h:66-82, :235-238)

``ml_dtypes`` (which the reference uses for its bf16 casts) is absent here; the
bf16 conversions are restated as IEEE round-to-nearest-even on the f32 bits.

Pinning (what fixes each function independently of its own formula) is done in
``tests/test_oracle.py``: the seed-702 scalar-loop known-answer test of
``specs/open-engine/tests/test_q4nx_decode_layout.py:8-30``, the pack->dequant
identity of ``q4_1_pack._selftest`` (:194-209), torch's own fp16->bf16 RNE,
brute-force scalar loops on tiny shapes, one-hot / all-ones activations, and
the exact Q4_0 identity m = -8 d.  The Q4_K functions are pinned in
``tests/test_gguf.py``: against the reference's own C++ GGUF reader, built from
its sources into ``oracle/_ref/gguf_dump`` (bit-exact f32 dequant), by an
exhaustive encode -> decode of the packed 6-bit scales, a closed-form block,
and the reference's property checks of the container transcode.  The chunk
transcodes (``requant_q4_1``, ``q4k_chunks_to_pool``, ``signed_pool_to_q4_1``,
``split_q8_chunks``) are pinned in ``tests/test_pools_ref.py`` byte for byte
against the reference's own C++ (src/open_qwen36/pools.cpp, built from its
sources into ``oracle/_ref/pools_dump``) and by the reference's published FNV-1a
goldens (``fnv1a64`` uses the reference's offset basis).  Functions with no such
check are marked "parity unpinned" in their docstrings (there are none at
present).

The MI355X weight layouts (``pack_mx`` / ``unpack_mx``, and the native Q4_K
``pack_mxk_*`` / ``unpack_mxk``) are this build's own formats, not the
reference's; their oracles are pinned by round trips against the GGUF blocks
and the reference pool and chunk layouts (``dequant_mxk`` of a packed GGUF
matrix equals ``dequant_q4_k``, which the reference's C++ reader pins; of packed
container chunks, the f32 rounding of ``dequant_q4k_chunks_exact``).
"""
from __future__ import annotations

import numpy as np

CH = 5120            # pool chunk bytes: 32 rows x 256 K  (q4_1_pack.py:52)
BLK = 32             # values per GGUF block              (q4_1_pack.py:53)
Q4_1_BYTES = 20      # fp16 d, fp16 m, 16 nibble bytes     (q4_1_pack.py:54)
Q4_0_BYTES = 18      # fp16 d, 16 nibble bytes, min = -8 d (q4_1_pack.py:55)

# MI355X layout geometry (this build's format; see pack_mx)
MX_ROWS = 64                 # output rows per tile (a row group)
MX_TILE = 1280               # bytes per tile: 1024 B codes + 256 B scales
MX_CODES = 1024


# --------------------------------------------------------------------------
# bf16 helpers (q4nx.py:95-102)
# --------------------------------------------------------------------------

def bf16_to_f32(u16) -> np.ndarray:
    """bf16 bit patterns -> f32 (exact widening; q4nx.py:95-96)."""
    return (np.asarray(u16, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f32) -> np.ndarray:
    """f32 -> bf16 bit patterns, round-to-nearest-even (q4nx.py:99-102).

    Finite inputs only (the path never carries NaN/Inf scales)."""
    u = np.ascontiguousarray(np.asarray(f32, dtype=np.float32)).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def bf16_round(f32) -> np.ndarray:
    """f32 -> nearest bf16 value, returned as f32."""
    return bf16_to_f32(f32_to_bf16(f32))


# --------------------------------------------------------------------------
# GGUF blocks (q4_1_pack.py:58-109)
# --------------------------------------------------------------------------

def random_q4_1_blocks_ref(n: int, k: int, rng: np.random.Generator, scale: float = 0.02) -> np.ndarray:
    """The reference's synthetic Q4_1 generator, same draws in the same order
    (q4_1_pack.py:70-81): uint8[n, k//32, 20]."""
    assert k % BLK == 0
    nb = k // BLK
    d = (rng.random((n, nb), np.float32) * scale + 1e-3).astype(np.float16)
    m = ((rng.random((n, nb), np.float32) - 0.5) * scale * 15).astype(np.float16)
    q = rng.integers(0, 16, (n, nb, BLK), dtype=np.uint8)
    return _assemble_q4_1(d, m, q)


def random_q4_0_blocks_ref(n: int, k: int, rng: np.random.Generator, scale: float = 0.02) -> np.ndarray:
    """The reference's synthetic Q4_0 generator (q4_1_pack.py:58-67): uint8[n, k//32, 18]."""
    assert k % BLK == 0
    nb = k // BLK
    d = (rng.random((n, nb), np.float32) * scale + 1e-3).astype(np.float16)
    q = rng.integers(0, 16, (n, nb, BLK), dtype=np.uint8)
    blocks = np.empty((n, nb, Q4_0_BYTES), np.uint8)
    blocks[..., 0:2] = d.view(np.uint8).reshape(n, nb, 2)
    blocks[..., 2:18] = q[..., :16] | (q[..., 16:] << 4)
    return blocks


def baseline_q4_1_blocks(n: int, k: int, rng: np.random.Generator) -> np.ndarray:
    """The benchmark distribution: q ~ U{0..15}, d = fp16(|N(0,1)|*0.002 + 1e-4),
    m = fp16(-8*d*U(0.9,1.1)); uint8[n, k//32, 20].

    Draw order: d, then the U(0.9,1.1) factor, then the codes."""
    assert k % BLK == 0
    nb = k // BLK
    d = (np.abs(rng.standard_normal((n, nb), np.float32)) * np.float32(0.002) + np.float32(1e-4)).astype(np.float16)
    u = rng.uniform(0.9, 1.1, (n, nb)).astype(np.float32)
    m = (np.float32(-8.0) * d.astype(np.float32) * u).astype(np.float16)
    q = rng.integers(0, 16, (n, nb, BLK), dtype=np.uint8)
    return _assemble_q4_1(d, m, q)


def _assemble_q4_1(d16: np.ndarray, m16: np.ndarray, q: np.ndarray) -> np.ndarray:
    n, nb = d16.shape
    blocks = np.empty((n, nb, Q4_1_BYTES), np.uint8)
    blocks[..., 0:2] = np.ascontiguousarray(d16).view(np.uint8).reshape(n, nb, 2)
    blocks[..., 2:4] = np.ascontiguousarray(m16).view(np.uint8).reshape(n, nb, 2)
    blocks[..., 4:20] = q[..., :16] | (q[..., 16:] << 4)   # byte j: value j low, j+16 high
    return blocks


def unpack_q4_1_blocks(blocks: np.ndarray):
    """uint8[n, nb, 20|18] -> (d f32[n,nb], m f32[n,nb], q uint8[n, nb*32]).

    Q4_0 reads as m = -8 d (q4_1_pack.py:84-101)."""
    n, nb, width = blocks.shape
    if width not in (Q4_1_BYTES, Q4_0_BYTES):
        raise ValueError(f"block width {width} is neither Q4_1 (20) nor Q4_0 (18)")
    d = np.ascontiguousarray(blocks[..., 0:2]).view(np.float16).reshape(n, nb).astype(np.float32)
    if width == Q4_1_BYTES:
        m = np.ascontiguousarray(blocks[..., 2:4]).view(np.float16).reshape(n, nb).astype(np.float32)
        qs = blocks[..., 4:20]
    else:
        m = np.float32(-8.0) * d
        qs = blocks[..., 2:18]
    q = np.concatenate([qs & 0xF, qs >> 4], axis=-1).reshape(n, nb * BLK)
    return d, m, q


def dequant_q4_1(blocks: np.ndarray, bf16_scales: bool = True) -> np.ndarray:
    """GGUF blocks -> f32[n, k] = fl32(q*d + m) (q4_1_pack.py:104-109).

    ``bf16_scales=True`` narrows d and m to bf16 first: what the kernels see."""
    d, m, q = unpack_q4_1_blocks(blocks)
    if bf16_scales:
        d, m = bf16_round(d), bf16_round(m)
    return q.astype(np.float32) * np.repeat(d, BLK, axis=1) + np.repeat(m, BLK, axis=1)


def q4_0_to_q4_1(blocks: np.ndarray) -> np.ndarray:
    """Exact Q4_0 (18 B) -> Q4_1 (20 B) transcode: m = -8 d, same codes
    (recipes/pack.py:606-622 states it for the signed container form; for GGUF
    offset-binary codes the nibbles are kept as they are)."""
    n, nb, width = blocks.shape
    assert width == Q4_0_BYTES
    d16 = np.ascontiguousarray(blocks[..., 0:2]).view(np.float16).reshape(n, nb)
    m16 = (np.float32(-8.0) * d16.astype(np.float32)).astype(np.float16)
    out = np.empty((n, nb, Q4_1_BYTES), np.uint8)
    out[..., 0:2] = blocks[..., 0:2]
    out[..., 2:4] = m16.view(np.uint8).reshape(n, nb, 2)
    out[..., 4:20] = blocks[..., 2:18]
    return out


# --------------------------------------------------------------------------
# Reference pool layout (q4_1_pack.py:16-34, :112-191)
# --------------------------------------------------------------------------

def chunk_geometry(n: int, k: int, rs: int):
    """(nch, per_band, rows0[nch], cols0[nch]) for the pool order (q4_1_pack.py:112-121)."""
    assert k % 256 == 0 and n % (32 * rs) == 0
    per_band = rs * k // 256
    nch = n * k // (32 * 256)
    c = np.arange(nch)
    band, ci = np.divmod(c, per_band)
    rows0 = 32 * rs * band + 32 * (ci % rs)
    cols0 = 256 * (ci // rs)
    return nch, per_band, rows0, cols0


def pack_q4_1_pool(blocks: np.ndarray, rs: int) -> np.ndarray:
    """GGUF blocks -> pool-order chunk bytes uint8[nch*5120] (q4_1_pack.py:124-142).

    Chunk: d bf16[256] @0 (index kb*32+r), m bf16[256] @512, nibbles @1024 with
    nibble p = (r//16)*4096 + k*16 + r%16, even p in the low half of byte p//2."""
    n, nb, _ = blocks.shape
    k = nb * BLK
    d, m, q = unpack_q4_1_blocks(blocks)
    d16, m16 = f32_to_bf16(d), f32_to_bf16(m)
    nch, _, rows0, cols0 = chunk_geometry(n, k, rs)
    # gather every chunk's [32 r, 256 k] window at once
    r_idx = rows0[:, None] + np.arange(32)[None, :]                      # [nch, 32]
    kb_idx = (cols0 // BLK)[:, None] + np.arange(8)[None, :]              # [nch, 8]
    dd = d16[r_idx[:, :, None], kb_idx[:, None, :]]                       # [nch, 32 r, 8 kb]
    mm = m16[r_idx[:, :, None], kb_idx[:, None, :]]
    k_idx = cols0[:, None] + np.arange(256)[None, :]                      # [nch, 256]
    qq = q[r_idx[:, :, None], k_idx[:, None, :]]                          # [nch, 32 r, 256 k]
    qq = qq.reshape(nch, 2, 16, 256).transpose(0, 1, 3, 2).reshape(nch, 8192)  # [rb, k, r16]
    out = np.empty((nch, CH), np.uint8)
    out[:, 0:512] = np.ascontiguousarray(dd.transpose(0, 2, 1)).reshape(nch, 256).view(np.uint8)
    out[:, 512:1024] = np.ascontiguousarray(mm.transpose(0, 2, 1)).reshape(nch, 256).view(np.uint8)
    out[:, 1024:] = qq[:, 0::2] | (qq[:, 1::2] << 4)
    return out.reshape(-1)


def dequant_chunk(b: np.ndarray) -> np.ndarray:
    """One 5120 B pool chunk -> f32[32 rows, 256 k] (q4_1_pack.py:155-170)."""
    d = bf16_to_f32(np.ascontiguousarray(b[0:512]).view(np.uint16))
    m = bf16_to_f32(np.ascontiguousarray(b[512:1024]).view(np.uint16))
    qb = b[1024:CH]
    nib = np.empty(8192, np.uint8)
    nib[0::2] = qb & 0xF
    nib[1::2] = qb >> 4
    n3 = nib.reshape(2, 256, 16)                       # [rb, k, r16]
    codes = n3.transpose(0, 2, 1).reshape(32, 256).astype(np.float32)   # [r, k]
    j = (np.arange(256) // BLK)[None, :] * 32 + np.arange(32)[:, None]  # kb*32 + r
    return codes * d[j] + m[j]


def dequant_pool(pool: np.ndarray, n: int, k: int, rs: int) -> np.ndarray:
    """Pool-order chunk bytes -> f32[n, k] (q4_1_pack.py:173-180)."""
    nch, _, rows0, cols0 = chunk_geometry(n, k, rs)
    chunks = np.asarray(pool, np.uint8).reshape(nch, CH)
    tiles = dq_chunks_q4_1(chunks).reshape(nch, 32, 256)
    w = np.empty((n, k), np.float32)
    for c in range(nch):
        w[rows0[c]:rows0[c] + 32, cols0[c]:cols0[c] + 256] = tiles[c]
    return w


def dq_chunks_q4_1(chunks: np.ndarray) -> np.ndarray:
    """[n, 5120] chunk bytes -> [n, 32 row, 8 block, 32 lane] f32 (q4nx.py:105-126).

    Value at (row, block, lane) = nib[p]*d[j] + m[j] with
    p = (row//16)*4096 + block*512 + lane*16 + row%16 and j = block*32 + row."""
    chunks = np.asarray(chunks, np.uint8)
    nch = chunks.shape[0]
    meta = bf16_to_f32(np.ascontiguousarray(chunks[:, :1024]).view(np.uint16))
    d, mn = meta[:, :256], meta[:, 256:]
    q = chunks[:, 1024:]
    nib = np.empty((nch, 8192), dtype=np.float32)
    nib[:, 0::2] = q & 0xF
    nib[:, 1::2] = q >> 4
    r = np.arange(32)[:, None, None]
    bc = np.arange(8)[None, :, None]
    i = np.arange(32)[None, None, :]
    p = ((r // 16) * 4096 + bc * 512 + i * 16 + (r % 16)).reshape(-1)
    j = np.broadcast_to(bc * 32 + r, (32, 8, 32)).reshape(-1)
    shape = (nch, 32, 8, 32)
    return (np.take(nib, p, axis=1).reshape(shape) * np.take(d, j, axis=1).reshape(shape)
            + np.take(mn, j, axis=1).reshape(shape))


def legacy_decode(chunks: np.ndarray) -> np.ndarray:
    """The benchmark harness's strided-indexing dequant (benchmark-q4-decode.py:19-34);
    byte-identical to dq_chunks_q4_1 by construction of the same fp32 operations."""
    nch = chunks.shape[0]
    meta = bf16_to_f32(np.ascontiguousarray(chunks[:, :1024]).view(np.uint16))
    d, mn = meta[:, :256], meta[:, 256:]
    q = chunks[:, 1024:]
    n = np.empty((nch, 8192), dtype=np.float32)
    n[:, 0::2] = q & 0xF
    n[:, 1::2] = q >> 4
    r = np.arange(32)[:, None, None]
    bc = np.arange(8)[None, :, None]
    i = np.arange(32)[None, None, :]
    p = ((r // 16) * 4096 + bc * 512 + i * 16 + (r % 16)).reshape(-1)
    j = (bc * 32 + r + 0 * i).reshape(-1)
    s = (nch, 32, 8, 32)
    return n[:, p].reshape(s) * d[:, j].reshape(s) + mn[:, j].reshape(s)


def pool_reference(pool: np.ndarray, x: np.ndarray, n: int, k: int, rs: int) -> np.ndarray:
    """y = W @ x accumulated in fp64 from the pool bytes, returned f32[n]
    (q4_1_pack.py:183-191)."""
    w = dequant_pool(pool, n, k, rs).astype(np.float64)
    return (w @ np.asarray(x, np.float64)).astype(np.float32)


# --------------------------------------------------------------------------
# References for the kernels' outputs
# --------------------------------------------------------------------------

def gemv_reference(blocks: np.ndarray, x: np.ndarray) -> np.ndarray:
    """Y[M, N] = X[M, K] @ W^T in fp64 from the bf16-scale dequant of the blocks
    (pool_reference semantics, q4_1_pack.py:183-191; batched rows as in
    designs/gemm_q4/make_test.py: every token row is an independent GEMV)."""
    w = dequant_q4_1(blocks, bf16_scales=True).astype(np.float64)
    xx = np.atleast_2d(np.asarray(x, np.float64))
    return (xx @ w.T).astype(np.float32)


def prefill_reference(blocks: np.ndarray, x_tk: np.ndarray) -> np.ndarray:
    """Y[T, N] for T distinct token activations, fp64 from the same weights
    (gemm_q4_prefill/make_test.py:82-94, returned token-major: the engine's
    layout after host::transpose, core.cpp:2960)."""
    return gemv_reference(blocks, x_tk)


def maxrel(got: np.ndarray, ref: np.ndarray) -> float:
    """max|got-ref| / max|ref| in fp64 (designs/gemv_q4/compare.py:13)."""
    g = np.asarray(got, np.float64).reshape(-1)
    r = np.asarray(ref, np.float64).reshape(-1)
    return float(np.abs(g - r).max() / (np.abs(r).max() + 1e-30)) if r.size else 0.0


def rel_fro(got: np.ndarray, ref: np.ndarray) -> float:
    """||got-ref||_F / ||ref||_F (gemm_q4_prefill/compare.py:33)."""
    g = np.asarray(got, np.float64).reshape(-1)
    r = np.asarray(ref, np.float64).reshape(-1)
    return float(np.linalg.norm(g - r) / (np.linalg.norm(r) + 1e-30))


def softmax_topk(logits: np.ndarray, topk: int):
    """Per token: p = softmax(logits); ids = argsort(-p, stable)[:topk];
    w = p[ids] / sum(p[ids])  (replica.py:121-128 route, :135 renormalise).

    Returns (ids int32[T, topk], w f32[T, topk])."""
    lg = np.atleast_2d(np.asarray(logits, np.float64))
    p = np.exp(lg - lg.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :topk]
    pw = np.take_along_axis(p, ids, axis=1)
    w = pw / pw.sum(axis=1, keepdims=True)
    return ids.astype(np.int32), w.astype(np.float32)


def silu(v: np.ndarray) -> np.ndarray:
    return v / (1.0 + np.exp(-v))


def moe_reference(gate_w, up_w, down_w, x: np.ndarray, ids: np.ndarray, wts: np.ndarray,
                  h_bf16: bool = False) -> np.ndarray:
    """out[t] = sum_j wts[t,j] * down_e( silu(gate_e x_t) * (up_e x_t) ), e = ids[t,j],
    in fp64 (replica.py:131-140 moe_decode without the shared expert; the
    per-expert product is moe_batch/make_test.py:91-98).

    ``gate_w/up_w/down_w`` are callables e -> f32 dequantized [rows, cols]
    (or arrays indexed by e). ``h_bf16`` rounds h to bf16 as the reference's
    moe_batch kernel does (make_test.py:96); the default keeps it in fp64 as
    the replica does."""
    get = (lambda a: (lambda e: a[e])) if not callable(gate_w) else None
    g_of = get(gate_w) if get else gate_w
    u_of = get(up_w) if get else up_w
    d_of = get(down_w) if get else down_w
    xx = np.atleast_2d(np.asarray(x, np.float64))
    T = xx.shape[0]
    out = np.zeros((T, np.asarray(d_of(int(ids[0, 0]))).shape[0]), np.float64)
    for e in np.unique(ids):
        toks, slots = np.nonzero(ids == e)
        xe = xx[toks]
        g = xe @ np.asarray(g_of(int(e)), np.float64).T
        u = xe @ np.asarray(u_of(int(e)), np.float64).T
        h = silu(g) * u
        if h_bf16:
            h = bf16_round(h.astype(np.float32)).astype(np.float64)
        y = h @ np.asarray(d_of(int(e)), np.float64).T
        out[toks] += np.asarray(wts, np.float64)[toks, slots][:, None] * y
    return out.astype(np.float32)


# --------------------------------------------------------------------------
# The MI355X layout (this build's own format)
# --------------------------------------------------------------------------
#
# An [N, K] matrix (N % 64 == 0, K % 32 == 0) is a grid of tiles (g, kb):
# row group g = n // 64, block kb = k // 32; tile (g, kb) sits at byte
# (g * K/32 + kb) * 1280, so one row group streams contiguously along K.
#
#   codes  [0, 1024): dword (lane, r) at byte lane*16 + r*4, lane 0..63, r 0..3:
#           row n = 64 g + 16 r + lane % 16,  k = 32 kb + 8 (lane // 16) + e,
#           e = 0..7, nibble e at bit 16*(e % 2) + 4*(e // 2).
#   scales [1024, 1280): dword at 1024 + (lane % 16)*16 + r*4 for the same row:
#           bits 31..16 = bf16 d, bits 15..0 = bf16 m.
#
# A 16x16x32 bf16 MFMA's B operand is exactly one codes dword per lane (the
# eight k of row lane%16 in k-group lane//16), so one 128-bit load per lane
# feeds four MFMAs (r = 0..3) and a wave streams 1 KB per load.


def moe_fin_reference(moe_out: np.ndarray, residual, shared, x: np.ndarray, sgw_bf16_bits) -> np.ndarray:
    """The MoE block's finish in fp64: out = xres + acc + sigmoid(xm . sgw) * shared
    (designs/moe_combine/moe_fin.py:1-4; designs/moe_experts/moe_fin.cc), acc the routed
    sum (moe_reference), xm the block's input rows, sgw the shared-expert gate vector as
    bf16 bits [H]. ``residual`` / ``shared`` may be None (that term left out)."""
    out = np.asarray(moe_out, np.float64).copy()
    if residual is not None:
        out += np.asarray(residual, np.float64)
    if shared is not None:
        sgw = (np.asarray(sgw_bf16_bits, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        g = 1.0 / (1.0 + np.exp(-(np.atleast_2d(np.asarray(x, np.float64)) @ sgw)))
        out += g[:, None] * np.asarray(shared, np.float64)
    return out

def mx_bytes(n: int, k: int) -> int:
    assert n % MX_ROWS == 0 and k % BLK == 0
    return (n // MX_ROWS) * (k // BLK) * MX_TILE


_E = np.arange(8)
_NIB_SHIFT = 16 * (_E % 2) + 4 * (_E // 2)        # bit position of element e


def pack_mx(blocks: np.ndarray, fp16_scales: bool = False) -> np.ndarray:
    """GGUF Q4_1/Q4_0 blocks [N, K/32, 20|18] -> the MI355X layout bytes
    (d and m narrowed to bf16 by RNE, as q4_1_pack.py:129-130 does). ``fp16_scales``
    (Q4_1 blocks): the scale word carries GGUF's own fp16 d and m bits unchanged, the
    exact-scale mode (the GGUF-direct pool keeps them, gguf_pool/gguf_pool.py:1-17)."""
    d, m, q = unpack_q4_1_blocks(blocks)
    if fp16_scales:
        if blocks.shape[2] != Q4_1_BYTES:
            raise ValueError("fp16 scale words are a Q4_1 mode")
        n, nb = d.shape
        d16 = np.ascontiguousarray(blocks[..., 0:2]).view(np.uint16).reshape(n, nb)
        m16 = np.ascontiguousarray(blocks[..., 2:4]).view(np.uint16).reshape(n, nb)
        return pack_mx_from_parts(d16, m16, q)
    return pack_mx_from_parts(f32_to_bf16(d), f32_to_bf16(m), q)


def unpack_mx(packed: np.ndarray, n: int, k: int):
    """MI355X layout bytes -> (d16 uint16[n,kb], m16 uint16[n,kb], q uint8[n,k])."""
    nb = k // BLK
    G = n // MX_ROWS
    t = np.asarray(packed, np.uint8).reshape(G, nb, MX_TILE)
    codes = np.ascontiguousarray(t[:, :, :MX_CODES]).view(np.uint32).reshape(G, nb, 4, 16, 4)  # [G,kb,kg,i,r]
    sc = np.ascontiguousarray(t[:, :, MX_CODES:]).view(np.uint32).reshape(G, nb, 16, 4)        # [G,kb,i,r]
    dw = codes.transpose(0, 4, 3, 1, 2).reshape(n, nb, 4)                                       # [n, kb, kg]
    q = np.empty((n, nb, 4, 8), np.uint8)
    for e in range(8):
        q[..., e] = (dw >> np.uint32(_NIB_SHIFT[e])) & np.uint32(0xF)
    s = sc.transpose(0, 3, 2, 1).reshape(n, nb)
    return (s >> np.uint32(16)).astype(np.uint16), (s & np.uint32(0xFFFF)).astype(np.uint16), q.reshape(n, k)


def dequant_mx(packed: np.ndarray, n: int, k: int, fp16_scales: bool = False) -> np.ndarray:
    """MI355X layout -> f32[n, k] = fl32(q*d + m) with the stored bf16 d, m (or, with
    ``fp16_scales``, the stored fp16 d, m of the exact-scale mode)."""
    d16, m16, q = unpack_mx(packed, n, k)
    conv = (lambda b: b.view(np.float16).astype(np.float32)) if fp16_scales else bf16_to_f32
    d = np.repeat(conv(d16), BLK, axis=1)
    m = np.repeat(conv(m16), BLK, axis=1)
    return q.astype(np.float32) * d + m


def pool_to_blocks(pool: np.ndarray, n: int, k: int, rs: int):
    """Invert pack_q4_1_pool to (d16, m16, q): bf16 scales [n, k/32], codes [n, k]."""
    nch, _, rows0, cols0 = chunk_geometry(n, k, rs)
    ch = np.asarray(pool, np.uint8).reshape(nch, CH)
    d16 = np.empty((n, k // BLK), np.uint16)
    m16 = np.empty((n, k // BLK), np.uint16)
    q = np.empty((n, k), np.uint8)
    dd = np.ascontiguousarray(ch[:, 0:512]).view(np.uint16).reshape(nch, 8, 32)
    mm = np.ascontiguousarray(ch[:, 512:1024]).view(np.uint16).reshape(nch, 8, 32)
    nib = np.empty((nch, 8192), np.uint8)
    nib[:, 0::2] = ch[:, 1024:] & 0xF
    nib[:, 1::2] = ch[:, 1024:] >> 4
    qq = nib.reshape(nch, 2, 256, 16).transpose(0, 1, 3, 2).reshape(nch, 32, 256)
    for c in range(nch):
        r0, c0 = int(rows0[c]), int(cols0[c])
        d16[r0:r0 + 32, c0 // BLK:c0 // BLK + 8] = dd[c].T
        m16[r0:r0 + 32, c0 // BLK:c0 // BLK + 8] = mm[c].T
        q[r0:r0 + 32, c0:c0 + 256] = qq[c]
    return d16, m16, q


def pack_mx_from_parts(d16: np.ndarray, m16: np.ndarray, q: np.ndarray) -> np.ndarray:
    """(bf16 d bits [N, K/32], bf16 m bits, codes uint8[N, K]) -> MI355X layout bytes."""
    n, nb = d16.shape
    assert n % MX_ROWS == 0 and q.shape == (n, nb * BLK)
    G = n // MX_ROWS
    q5 = q.reshape(n, nb, 4, 8).astype(np.uint32)
    dw = np.zeros((n, nb, 4), np.uint32)                                # [n, kb, kg]
    for e in range(8):
        dw |= q5[..., e] << np.uint32(_NIB_SHIFT[e])
    sc = (d16.astype(np.uint32) << np.uint32(16)) | m16.astype(np.uint32)   # [n, kb]
    # n = 64 G + 16 r + i;  codes dword index within a tile = (kg*16 + i)*4 + r
    codes = dw.reshape(G, 4, 16, nb, 4).transpose(0, 3, 4, 2, 1)          # [G, kb, kg, i, r]
    sc = sc.reshape(G, 4, 16, nb).transpose(0, 3, 2, 1)                   # [G, kb, i, r]
    out = np.empty((G, nb, MX_TILE), np.uint8)
    out[:, :, :MX_CODES] = np.ascontiguousarray(codes).reshape(G, nb, 256).view(np.uint8).reshape(G, nb, MX_CODES)
    out[:, :, MX_CODES:] = np.ascontiguousarray(sc).reshape(G, nb, 64).view(np.uint8).reshape(G, nb, 256)
    return out.reshape(-1)


# --------------------------------------------------------------------------
# Q4_0-native: the reference's 4608 B chunk and the MI355X mx0 tile
# --------------------------------------------------------------------------
# mx0 tile (g, kb), 1152 B: the mx codes [0, 1024), then bf16 d of row 16 r + i at
# 1024 + 8 i + 2 r. Q4_0 stores no min: weight = fl32(q d + m), m = -8 d (exact).
CH_Q4_0 = 4608
MX0_TILE = 1152


def pack_q4_0_native_pool(blocks: np.ndarray, rs: int) -> np.ndarray:
    """GGUF Q4_0 blocks -> 4608 B Q4_0-native chunks in pool order: the 5120 B chunk of
    pack_q4_1_pool with its m plane [512, 1024) left out (q4_1_pack.py:145-152)."""
    assert blocks.shape[2] == Q4_0_BYTES, "a Q4_0-native pool holds Q4_0 blocks only"
    full = pack_q4_1_pool(blocks, rs).reshape(-1, CH)
    return np.concatenate([full[:, :512], full[:, 1024:]], axis=1).reshape(-1)


def mx0_bytes(n: int, k: int) -> int:
    assert n % MX_ROWS == 0 and k % BLK == 0
    return (n // MX_ROWS) * (k // BLK) * MX0_TILE


def pack_mx0(blocks: np.ndarray) -> np.ndarray:
    """GGUF Q4_0 blocks [N, K/32, 18] -> mx0 bytes: pack_mx's codes with the bf16 d alone."""
    assert blocks.shape[2] == Q4_0_BYTES
    d, _, q = unpack_q4_1_blocks(blocks)
    n, nb = d.shape
    G = n // MX_ROWS
    full = pack_mx_from_parts(f32_to_bf16(d), np.zeros_like(f32_to_bf16(d)), q).reshape(G, nb, MX_TILE)
    dd = f32_to_bf16(d).reshape(G, 4, 16, nb).transpose(0, 3, 2, 1)          # [G, kb, i, r]
    out = np.empty((G, nb, MX0_TILE), np.uint8)
    out[:, :, :MX_CODES] = full[:, :, :MX_CODES]
    out[:, :, MX_CODES:] = np.ascontiguousarray(dd).view(np.uint8).reshape(G, nb, 128)
    return out.reshape(-1)


def unpack_mx0(packed: np.ndarray, n: int, k: int):
    """mx0 bytes -> (d16 uint16[n, k/32], codes uint8[n, k])."""
    nb, G = k // BLK, n // MX_ROWS
    t = np.asarray(packed, np.uint8).reshape(G, nb, MX0_TILE)
    as_mx = np.zeros((G, nb, MX_TILE), np.uint8)
    as_mx[:, :, :MX_CODES] = t[:, :, :MX_CODES]
    _, _, q = unpack_mx(as_mx.reshape(-1), n, k)
    d16 = np.ascontiguousarray(t[:, :, MX_CODES:]).view(np.uint16).reshape(G, nb, 16, 4).transpose(0, 3, 2, 1)
    return d16.reshape(n, nb), q


def dequant_mx0(packed: np.ndarray, n: int, k: int) -> np.ndarray:
    """mx0 -> f32[n, k] = fl32(q d + m), m = -8 d from the stored bf16 d."""
    d16, q = unpack_mx0(packed, n, k)
    d = np.repeat(bf16_to_f32(d16), BLK, axis=1)
    return (q.astype(np.float32) * d + np.float32(-8.0) * d).astype(np.float32)


# --------------------------------------------------------------------------
# Q4_K: GGUF super-blocks and the reference container's 4736 B chunks
# --------------------------------------------------------------------------
# GGUF Q4_K super-block, 144 B for 256 values along K (llama.cpp's block_q4_K, read by
# open_kernels/model/gguf_ref.py:236-250 and src/gguf/gguf_file.cpp:611-635):
#   [0, 2) fp16 d   [2, 4) fp16 dmin   [4, 16) eight packed 6-bit (scale, min) pairs
#   [16, 144) codes: byte 32 c + l holds value 64 c + l (low nibble) and 64 c + 32 + l (high)
# Sub-block j (values 32 j .. 32 j + 31) reads  d * sc_j * q - dmin * min_j.

Q4_K_BYTES = 144
Q4K_CHUNK = 4736     # container Q4_K chunk: 32 rows x 256 K (recipes/pack.py:272-283)


def q4_k_scale_min(scales: np.ndarray, j: int):
    """6-bit (sc_j, min_j) of sub-block j from the 12 packed bytes [..., 12]
    (gguf_ref.py:224-233; get_scale_min_k4 in src/gguf/gguf_file.cpp). Sub-blocks 0-3
    keep their pair in the low six bits of bytes j and j + 4; 4-7 keep the low four
    bits in byte j + 4 (scale low nibble, min high nibble) and the top two bits in the
    spare top bits of bytes j - 4 (scale) and j (min)."""
    s = np.asarray(scales).astype(np.int32)
    if j < 4:
        return s[..., j] & 63, s[..., j + 4] & 63
    return ((s[..., j + 4] & 0xF) | ((s[..., j - 4] >> 6) << 4),
            (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4))


def unpack_q4_k_blocks(blocks: np.ndarray):
    """uint8[n, K/256, 144] -> (d f32[n, K/32], m f32[n, K/32], q uint8[n, K]): each
    sub-block as a Q4_1 block reading q*d + m, with d = fp16 d * sc_j and
    m = -(fp16 dmin * min_j). Both products are exact in f32 (11-bit x 6-bit
    significands), so this is a change of form, not of value (gguf_ref.py:236-250)."""
    b = np.asarray(blocks, np.uint8)
    n, ns, width = b.shape
    if width != Q4_K_BYTES:
        raise ValueError(f"block width {width} is not Q4_K ({Q4_K_BYTES})")
    d = np.ascontiguousarray(b[..., 0:2]).view(np.float16).reshape(n, ns).astype(np.float32)
    dmin = np.ascontiguousarray(b[..., 2:4]).view(np.float16).reshape(n, ns).astype(np.float32)
    sc = b[..., 4:16]
    qs = b[..., 16:144]
    D = np.empty((n, ns, 8), np.float32)
    M = np.empty((n, ns, 8), np.float32)
    q = np.empty((n, ns, 8, BLK), np.uint8)
    for j in range(8):
        s6, m6 = q4_k_scale_min(sc, j)
        D[..., j] = d * s6.astype(np.float32)
        M[..., j] = -(dmin * m6.astype(np.float32))
        half = qs[..., 32 * (j // 2):32 * (j // 2) + 32]
        q[..., j, :] = (half >> 4) if j % 2 else (half & 0xF)
    return D.reshape(n, ns * 8), M.reshape(n, ns * 8), q.reshape(n, ns * 256)


def dequant_q4_k(blocks: np.ndarray) -> np.ndarray:
    """GGUF Q4_K -> f32[n, K] as the reference reads it: fl32(d sc q - dmin min)
    (gguf_file.cpp:627-630). d sc q is exact, so this equals fl32(q*D + M)."""
    D, M, q = unpack_q4_k_blocks(blocks)
    return q.astype(np.float32) * np.repeat(D, BLK, axis=1) + np.repeat(M, BLK, axis=1)


def dequant_q4_k_bf16(blocks: np.ndarray) -> np.ndarray:
    """What the kernels see of a Q4_K weight: D and M narrowed to bf16 (RNE), then
    fl32(q*d + m) -- the reference's Q4_K -> q4_1 collapse (recipes/pack.py:266-310)."""
    D, M, q = unpack_q4_k_blocks(blocks)
    return q.astype(np.float32) * np.repeat(bf16_round(D), BLK, axis=1) + np.repeat(bf16_round(M), BLK, axis=1)


def pack_mx_q4_k(blocks: np.ndarray) -> np.ndarray:
    """GGUF Q4_K [N, K/256, 144] -> the MI355X layout bytes (D, M rounded to bf16)."""
    D, M, q = unpack_q4_k_blocks(blocks)
    return pack_mx_from_parts(f32_to_bf16(D), f32_to_bf16(M), q)


def random_q4_k_blocks(n: int, k: int, rng: np.random.Generator, scale: float = 0.02) -> np.ndarray:
    """Seeded GGUF Q4_K super-blocks: every packed scale/min byte and code uniform, fp16 d
    and dmin positive and sized so d*sc*15 is about ``scale`` (llama.cpp's quantizer
    makes d = max_j(scale_j)/63 and dmin = max_j(min_j)/63)."""
    assert k % 256 == 0
    ns = k // 256
    b = rng.integers(0, 256, (n, ns, Q4_K_BYTES), dtype=np.uint8)
    d = (rng.uniform(0.5, 1.5, (n, ns)) * scale / (15 * 40)).astype(np.float16)
    dmin = (rng.uniform(0.5, 1.5, (n, ns)) * scale / 40).astype(np.float16)
    b[..., 0:2] = d.view(np.uint8).reshape(n, ns, 2)
    b[..., 2:4] = dmin.view(np.uint8).reshape(n, ns, 2)
    return b


def q4k_chunks_to_pool(chunks: np.ndarray) -> np.ndarray:
    """Container Q4_K chunks [n, 4736] -> pool q4_1 chunks [n, 5120], same order
    (recipes/pack.py:266-310; test_quant_q4k.py:7-13 gives the layout):

      Q4_K chunk: scales u8[8 g][32 r] @0, mins u8 @256, codes @512 with row r of
      column k at byte 512 + 16 k + r//2 (even r low nibble), S bf16[32 r] @4608,
      M bf16[32 r] @4672 (stored negated); value S sc nib + M min.

    Pool d = bf16_rne(S[r] sc[g][r]) and m = bf16_rne(M[r] min[g][r]) at index 32 g + r
    (the f32 products are exact: 8-bit x 8-bit significands). Codes: pool byte
    2048 h + 8 k + i = chunk byte 512 + 16 k + 8 h + i (rows 16 h .. 16 h + 15)."""
    src = np.asarray(chunks, np.uint8).reshape(-1, Q4K_CHUNK)
    n = src.shape[0]
    S = bf16_to_f32(np.ascontiguousarray(src[:, 4608:4672]).view(np.uint16))   # [n, 32 r]
    Mn = bf16_to_f32(np.ascontiguousarray(src[:, 4672:4736]).view(np.uint16))
    sc = src[:, 0:256].reshape(n, 8, 32).astype(np.float32)                     # [n, g, r]
    mn = src[:, 256:512].reshape(n, 8, 32).astype(np.float32)
    d16 = f32_to_bf16(S[:, None, :] * sc).reshape(n, 256)
    m16 = f32_to_bf16(Mn[:, None, :] * mn).reshape(n, 256)
    out = np.empty((n, CH), np.uint8)
    out[:, 0:512] = d16.view(np.uint8).reshape(n, 512)
    out[:, 512:1024] = m16.view(np.uint8).reshape(n, 512)
    codes = src[:, 512:4608].reshape(n, 256, 2, 8)                               # [k, h, i]
    out[:, 1024:] = np.ascontiguousarray(codes.transpose(0, 2, 1, 3)).reshape(n, 4096)
    return out


def dequant_q4k_chunks_exact(chunks: np.ndarray) -> np.ndarray:
    """Container Q4_K chunks -> f64 [n, 32 r, 256 k], the value the layout states, with no
    bf16 collapse (test_quant_q4k.py:100-112's reading)."""
    src = np.asarray(chunks, np.uint8).reshape(-1, Q4K_CHUNK)
    n = src.shape[0]
    S = bf16_to_f32(np.ascontiguousarray(src[:, 4608:4672]).view(np.uint16)).astype(np.float64)
    Mn = bf16_to_f32(np.ascontiguousarray(src[:, 4672:4736]).view(np.uint16)).astype(np.float64)
    sc = src[:, 0:256].reshape(n, 8, 32).astype(np.float64)
    mn = src[:, 256:512].reshape(n, 8, 32).astype(np.float64)
    cb = src[:, 512:4608].reshape(n, 256, 16)                                   # [k, r//2]
    r = np.arange(32)
    nib = np.where(r % 2 == 0, cb[:, :, r // 2] & 0xF, cb[:, :, r // 2] >> 4)  # [n, k, r]
    nib = nib.transpose(0, 2, 1).astype(np.float64)                             # [n, r, k]
    g = np.arange(256) // 32
    scale = S[:, :, None] * sc[:, g, :].transpose(0, 2, 1)                      # [n, r, k]
    off = Mn[:, :, None] * mn[:, g, :].transpose(0, 2, 1)
    return scale * nib + off


def q4k_vector(nch: int) -> np.ndarray:
    """The reference's seeded container Q4_K chunks (test_quant_q4k.py:60-80): per chunk
    c an LCG (x <- 1664525 x + 1013904223 mod 2^32, byte = x >> 24) seeded with
    0x9E3779B9 (c + 1); 4608 plain bytes, then 32 bf16 S = 0x3B00 | byte and 32 bf16
    M = 0xBB00 | byte (negative)."""
    M32 = 0xFFFFFFFF
    out = np.zeros((nch, Q4K_CHUNK), np.uint8)
    for c in range(nch):
        s = (0x9E3779B9 * (c + 1)) & M32
        stream = np.empty(4672, np.uint32)
        for i in range(4672):
            s = (s * 1664525 + 1013904223) & M32
            stream[i] = s >> 24
        out[c, :4608] = stream[:4608]
        sm = np.concatenate([0x3B00 | stream[4608:4640], 0xBB00 | stream[4640:4672]]).astype(np.uint16)
        out[c, 4608:] = sm.view(np.uint8)
    return out


# --------------------------------------------------------------------------
# The native Q4_K layout ("mxk", this build's own format)
# --------------------------------------------------------------------------
#
# An [N, K] matrix (N % 64 == 0, K % 256 == 0) is a grid of tiles (g, sb): row group
# g = n // 64, super-block sb = k // 256, 9728 bytes at (g * K/256 + sb) * 9728:
#   codes [0, 8192): sub-block j = 0..7 at j * 1024 in the mx code layout above;
#   sc/mn [8192, 9216): row 16 r + i at 8192 + i * 64 + r * 16: sc[0..7] of its 8
#         sub-blocks, then mn[0..7];
#   d     [9216, 9472): f32 of row 16 r + i at 9216 + i * 16 + r * 4;  m at 9472 + ...
# weight = fl32(q * (d sc) + m mn); d sc and m mn are exact in f32.

MXK_TILE = 9728


def mxk_bytes(n: int, k: int) -> int:
    assert n % MX_ROWS == 0 and k % 256 == 0
    return (n // MX_ROWS) * (k // 256) * MXK_TILE


def pack_mxk_from_parts(d: np.ndarray, m: np.ndarray, sc: np.ndarray, mn: np.ndarray, q: np.ndarray) -> np.ndarray:
    """(f32 d [N, K/256], f32 m [N, K/256], uint8 sc [N, K/256, 8], uint8 mn, codes uint8[N, K])
    -> native Q4_K layout bytes."""
    n, SB = d.shape
    assert n % MX_ROWS == 0 and q.shape == (n, SB * 256) and sc.shape == (n, SB, 8) == mn.shape
    G = n // MX_ROWS
    nb = SB * 8
    q5 = q.reshape(n, nb, 4, 8).astype(np.uint32)
    dw = np.zeros((n, nb, 4), np.uint32)                                   # [n, kb, kg]
    for e in range(8):
        dw |= q5[..., e] << np.uint32(_NIB_SHIFT[e])
    codes = dw.reshape(G, 4, 16, SB, 8, 4).transpose(0, 3, 4, 5, 2, 1)    # [G, sb, j, kg, i, r]
    pair = np.concatenate([sc, mn], axis=2).astype(np.uint8)              # [n, sb, 16]
    pair = pair.reshape(G, 4, 16, SB, 16).transpose(0, 3, 2, 1, 4)        # [G, sb, i, r, 16]
    dd = np.asarray(d, np.float32).reshape(G, 4, 16, SB).transpose(0, 3, 2, 1)   # [G, sb, i, r]
    mm = np.asarray(m, np.float32).reshape(G, 4, 16, SB).transpose(0, 3, 2, 1)
    out = np.empty((G, SB, MXK_TILE), np.uint8)
    out[:, :, :8192] = np.ascontiguousarray(codes).view(np.uint8).reshape(G, SB, 8192)
    out[:, :, 8192:9216] = np.ascontiguousarray(pair).view(np.uint8).reshape(G, SB, 1024)
    out[:, :, 9216:9472] = np.ascontiguousarray(dd).view(np.uint8).reshape(G, SB, 256)
    out[:, :, 9472:] = np.ascontiguousarray(mm).view(np.uint8).reshape(G, SB, 256)
    return out.reshape(-1)


def unpack_mxk(packed: np.ndarray, n: int, k: int):
    """Native Q4_K layout bytes -> (d f32[n, k/256], m f32, sc uint8[n, k/256, 8], mn, q uint8[n, k])."""
    G, SB = n // MX_ROWS, k // 256
    t = np.asarray(packed, np.uint8).reshape(G, SB, MXK_TILE)
    codes = np.ascontiguousarray(t[:, :, :8192]).view(np.uint32).reshape(G, SB, 8, 4, 16, 4)  # [G,sb,j,kg,i,r]
    dw = codes.transpose(0, 5, 4, 1, 2, 3).reshape(n, SB * 8, 4)                              # [n, kb, kg]
    q = np.empty((n, SB * 8, 4, 8), np.uint8)
    for e in range(8):
        q[..., e] = (dw >> np.uint32(_NIB_SHIFT[e])) & np.uint32(0xF)
    pair = t[:, :, 8192:9216].reshape(G, SB, 16, 4, 16).transpose(0, 3, 2, 1, 4).reshape(n, SB, 16)  # [n,sb,16]
    d = np.ascontiguousarray(t[:, :, 9216:9472]).view(np.float32).reshape(G, SB, 16, 4).transpose(0, 3, 2, 1)
    m = np.ascontiguousarray(t[:, :, 9472:]).view(np.float32).reshape(G, SB, 16, 4).transpose(0, 3, 2, 1)
    return (d.reshape(n, SB), m.reshape(n, SB), np.ascontiguousarray(pair[:, :, :8]),
            np.ascontiguousarray(pair[:, :, 8:]), q.reshape(n, k))


def dequant_mxk(packed: np.ndarray, n: int, k: int) -> np.ndarray:
    """Native Q4_K layout -> f32[n, k] = fl32(q * (d sc) + m mn), d sc and m mn exact in f32."""
    d, m, sc, mn, q = unpack_mxk(packed, n, k)
    D = (d[:, :, None] * sc.astype(np.float32)).reshape(n, -1)
    M = (m[:, :, None] * mn.astype(np.float32)).reshape(n, -1)
    return q.astype(np.float32) * np.repeat(D, BLK, axis=1) + np.repeat(M, BLK, axis=1)


def q4_k_native_parts(blocks: np.ndarray):
    """GGUF Q4_K [N, K/256, 144] -> the native layout's parts: d = fp16 d, m = -fp16 dmin,
    (sc_j, mn_j) = the packed 6-bit pairs (gguf_ref.py:224-250; get_scale_min_k4), codes."""
    b = np.asarray(blocks, np.uint8)
    n, ns, width = b.shape
    if width != Q4_K_BYTES:
        raise ValueError(f"block width {width} is not Q4_K ({Q4_K_BYTES})")
    d = np.ascontiguousarray(b[..., 0:2]).view(np.float16).reshape(n, ns).astype(np.float32)
    dmin = np.ascontiguousarray(b[..., 2:4]).view(np.float16).reshape(n, ns).astype(np.float32)
    sc = np.empty((n, ns, 8), np.uint8)
    mn = np.empty((n, ns, 8), np.uint8)
    q = np.empty((n, ns, 8, BLK), np.uint8)
    for j in range(8):
        s6, m6 = q4_k_scale_min(b[..., 4:16], j)
        sc[..., j], mn[..., j] = s6, m6
        half = b[..., 16 + 32 * (j // 2):16 + 32 * (j // 2) + 32]
        q[..., j, :] = (half >> 4) if j % 2 else (half & 0xF)
    return d, -dmin, sc, mn, q.reshape(n, ns * 256)


def pack_mxk_q4_k(blocks: np.ndarray) -> np.ndarray:
    """GGUF Q4_K super-blocks -> native Q4_K layout bytes (no rounding of any value)."""
    return pack_mxk_from_parts(*q4_k_native_parts(blocks))


def q4k_chunks_native_parts(chunks: np.ndarray, n: int, k: int, rs: int):
    """Container Q4_K chunks (4736 B, band order with row split rs) -> the native layout's
    parts in [n, k] order: d = bf16 S[r], m = bf16 M[r] (stored negated), (sc, mn) =
    (scales[g][r], mins[g][r]), codes (row r of column kk at byte 512 + 16 kk + r // 2,
    even r low nibble) -- the chunk's own value S sc nib + M mn (gemm_q4.h:456-507)."""
    nch, _, rows0, cols0 = chunk_geometry(n, k, rs)
    src = np.asarray(chunks, np.uint8).reshape(nch, Q4K_CHUNK)
    SB = k // 256
    d = np.empty((n, SB), np.float32)
    m = np.empty((n, SB), np.float32)
    sc = np.empty((n, SB, 8), np.uint8)
    mn = np.empty((n, SB, 8), np.uint8)
    q = np.empty((n, k), np.uint8)
    r = np.arange(32)
    for c in range(nch):
        r0, c0 = int(rows0[c]), int(cols0[c])
        sb = c0 // 256
        ch = src[c]
        d[r0:r0 + 32, sb] = bf16_to_f32(np.ascontiguousarray(ch[4608:4672]).view(np.uint16))
        m[r0:r0 + 32, sb] = bf16_to_f32(np.ascontiguousarray(ch[4672:4736]).view(np.uint16))
        sc[r0:r0 + 32, sb, :] = ch[0:256].reshape(8, 32).T
        mn[r0:r0 + 32, sb, :] = ch[256:512].reshape(8, 32).T
        cb = ch[512:4608].reshape(256, 16)                                     # [kk, r // 2]
        nib = np.where(r % 2 == 0, cb[:, r // 2] & 0xF, cb[:, r // 2] >> 4)    # [kk, r]
        q[r0:r0 + 32, c0:c0 + 256] = nib.T
    return d, m, sc, mn, q


def pack_mxk_q4k_chunks(chunks: np.ndarray, n: int, k: int, rs: int) -> np.ndarray:
    """Container Q4_K chunks -> native Q4_K layout bytes (no rounding of any value)."""
    return pack_mxk_from_parts(*q4k_chunks_native_parts(chunks, n, k, rs))


# The offset basis the reference's hash starts from: 1469598103934665603
# (specs/open-engine/tests/test_pack_plan.py:184, src/open_qwen36/pools_test.cpp:84). It is
# the textbook FNV-1a basis 14695981039346656037 with its last digit dropped, so the
# reference's goldens are hashes under this basis, not under the textbook one.
FNV_BASIS_REF = 1469598103934665603
FNV_BASIS_TEXTBOOK = 0xCBF29CE484222325
FNV_PRIME = 0x100000001B3          # 1099511628211, the same in both


def fnv1a64(data, basis: int = FNV_BASIS_REF) -> int:
    """FNV-1a 64-bit hash of a byte string as the reference computes it
    (test_pack_plan.py:183-187, pools_test.cpp:83-90): its own offset basis by default;
    ``basis=FNV_BASIS_TEXTBOOK`` gives the published FNV-1a."""
    b = np.frombuffer(bytes(data), np.uint8)
    h = basis
    # byte loop in chunks of numpy-free Python ints (the hash is sequential)
    for x in b.tolist():
        h = ((h ^ x) * FNV_PRIME) & 0xFFFFFFFFFFFFFFFF
    return h


def shared_q8_vector(nch: int) -> np.ndarray:
    """The q8 chunks both reference packers hash (test_qwen35.py:668-684,
    src/open_qwen36/pools_test.cpp:60-80): per chunk an LCG seeded 0x9E3779B9 * (c + 1),
    256 bf16 scales 0x3B00 | (s >> 24), then 8192 code bytes s >> 24."""
    M32 = 0xFFFFFFFF
    out = np.zeros((nch, Q8_CHUNK), np.uint8)
    for c in range(nch):
        s = (0x9E3779B9 * (c + 1)) & M32
        stream = np.empty(256 + 8192, np.uint32)
        for i in range(256 + 8192):
            s = (s * 1664525 + 1013904223) & M32
            stream[i] = s >> 24
        out[c, :512] = (np.uint32(0x3B00) | stream[:256]).astype(np.uint16).view(np.uint8)
        out[c, 512:] = stream[256:].astype(np.uint8)
    return out


# --------------------------------------------------------------------------
# The lm_head's sampling epilogue
# --------------------------------------------------------------------------

def sampler_view(logits: np.ndarray) -> np.ndarray:
    """What the reference's sampler ranks: each f32 logit rounded to bf16 by the plain RNE
    formula (src/open_qwen36/q4nx_file.hpp:97-101; Engine::logits_view,
    src/open_qwen36/engine.cpp:125-131), an f32 subnormal read as +0
    (argmax_bf16, src/open_qwen36/cli.cpp:103-113)."""
    v = np.ascontiguousarray(logits, np.float32)
    u = v.view(np.uint32)
    r = bf16_to_f32(f32_to_bf16(v))
    return np.where((u & np.uint32(0x7F800000)) == 0, np.float32(0.0), r).astype(np.float32)


def topk_reference(logits: np.ndarray, k: int, mode: int = 1, n_valid: int | None = None):
    """(ids int32[M, k], vals f32[M, k]): per row, the k largest of the first n_valid
    values -- value descending, the lower id first on a tie (sampler.cpp:230-241's
    comparator), -0 equal to +0, NaN below every number. mode 1 ranks sampler_view of
    the logits, mode 0 the logits. Rows with fewer than k values pad with -1 / -inf."""
    lg = np.atleast_2d(np.asarray(logits, np.float32))
    M, N = lg.shape
    n = N if n_valid is None else int(n_valid)
    v = lg[:, :n]
    if mode == 1:
        v = sampler_view(v)
    ids = np.full((M, k), -1, np.int32)
    vals = np.full((M, k), -np.inf, np.float32)
    idx = np.arange(n)
    for m in range(M):
        row = v[m]
        nan = np.isnan(row)
        order = np.lexsort((idx, -np.where(nan, 0.0, row).astype(np.float64), nan))[:k]
        ids[m, :len(order)] = order
        vals[m, :len(order)] = row[order]
    return ids, vals


# --------------------------------------------------------------------------
# Epilogues either side of the GEMV
# --------------------------------------------------------------------------

def swiglu_reference(gate_blocks: np.ndarray, up_blocks: np.ndarray, x: np.ndarray) -> np.ndarray:
    """h[M, F] = silu(X G^T) * (X U^T) in fp64 from the bf16-scale dequant of both
    matrices (designs/silu_mul/make_test.py:18-21's h, before its bf16 rounding;
    model/replica.py:140's silu(gate x) * (up x))."""
    xx = np.atleast_2d(np.asarray(x, np.float64))
    g = xx @ dequant_q4_1(gate_blocks, bf16_scales=True).astype(np.float64).T
    u = xx @ dequant_q4_1(up_blocks, bf16_scales=True).astype(np.float64).T
    return silu(g) * u


def rmsnorm_add_reference(x: np.ndarray, add, w: np.ndarray, eps: float = 1e-6):
    """(y f32, xn f64): y = x + add in f32, xn = y / sqrt(mean(y^2) + eps) * w in fp64 per
    row (designs/ln/make_test.py:44-50; model/replica.py:33-35's rms)."""
    x = np.atleast_2d(np.asarray(x, np.float32))
    y = x + np.atleast_2d(np.asarray(add, np.float32)) if add is not None else x.copy()
    y64 = y.astype(np.float64)
    xn = y64 / np.sqrt((y64 ** 2).mean(-1, keepdims=True) + eps) * np.asarray(w, np.float64)
    return y, xn


# --------------------------------------------------------------------------
# .q4nx chunk formats: the signed quantiser and q8, read as q4_1
# --------------------------------------------------------------------------
Q8_CHUNK = 8704      # bf16 scales[256] (index kb*32 + r) then int8 codes[8192] (q4nx.py)

_R = np.arange(BLK)[:, None, None]
_BC = np.arange(8)[None, :, None]
_I = np.arange(BLK)[None, None, :]
CHUNK_CODE_IDX = ((_R // 16) * 4096 + _BC * 512 + _I * 16 + (_R % 16)).reshape(-1)   # (r, block, lane)
CHUNK_META_IDX = (_BC * 32 + _R + 0 * _I).reshape(-1)


def signed_pool_to_q4_1(chunks: np.ndarray) -> np.ndarray:
    """5120 B chunks of the signed quantiser (w = d * int4(q), mins 0) -> q4_1 chunks:
    nibble q ^ 8, m = bf16(-8 d) (recipes/pack.py:606-622). Exact both ways."""
    src = np.asarray(chunks, np.uint8).reshape(-1, CH)
    out = src.copy()
    d = bf16_to_f32(np.ascontiguousarray(src[:, :512]).view(np.uint16))
    out[:, 512:1024] = f32_to_bf16(np.float32(-8.0) * d).view(np.uint8).reshape(-1, 512)
    out[:, 1024:] = src[:, 1024:] ^ 0x88
    return out


def signed_pool_values(chunks: np.ndarray) -> np.ndarray:
    """[n, 32 r, 8 block, 32 lane] f64 values d * int4(q) straight from the signed bytes."""
    src = np.asarray(chunks, np.uint8).reshape(-1, CH)
    nib = np.empty((src.shape[0], 8192), np.int64)
    nib[:, 0::2] = src[:, 1024:] & 0xF
    nib[:, 1::2] = src[:, 1024:] >> 4
    q = np.where(nib >= 8, nib - 16, nib)[:, CHUNK_CODE_IDX]
    d = bf16_to_f32(np.ascontiguousarray(src[:, :512]).view(np.uint16)).astype(np.float64)[:, CHUNK_META_IDX]
    return (q * d).reshape(-1, 32, 8, 32)


def q8_chunk_values(chunks: np.ndarray) -> np.ndarray:
    """[n, 32 r, 8 block, 32 lane] f32 code * scale of q8 chunks (exact in f32)."""
    src = np.asarray(chunks, np.uint8).reshape(-1, Q8_CHUNK)
    sc = bf16_to_f32(np.ascontiguousarray(src[:, :512]).view(np.uint16))
    code = np.ascontiguousarray(src[:, 512:]).view(np.int8)
    return (code[:, CHUNK_CODE_IDX].astype(np.float32) * sc[:, CHUNK_META_IDX]).reshape(-1, 32, 8, 32)


def _bf16_floor(x) -> np.ndarray:
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return np.where(u >> 31, (u + np.uint32(0xFFFF)) >> 16, u >> 16).astype(np.uint16)


def _bf16_ceil(x) -> np.ndarray:
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return np.where(u >> 31, u >> 16, (u + np.uint32(0xFFFF)) >> 16).astype(np.uint16)


def requant_q4_1(chunks: np.ndarray) -> np.ndarray:
    """q8 chunks [n, 8704] -> q4_1 chunks [n, 5120], block for block (recipes/pack.py:
    224-263): m = block min rounded down to bf16; d = f32((max - m) / 15) rounded up to
    bf16; nibble = clip(trunc(f32(f32(v - m) * f32(1 / d)) + 0.5), 0, 15), each f32
    operation rounded on its own. The block's min and max are taken as the reference's
    C++ scans them (pools.cpp:591-601: start at lane 0, replace only on a strict < or >),
    i.e. the first lane holding the extreme value keeps its sign: a -0 (a negative code
    under a zero scale) that comes first makes m = bf16 -0 (0x8000)."""
    v = q8_chunk_values(chunks)                                  # [n, r, block, lane]
    n = v.shape[0]
    first_min = np.argmax(v == v.min(-1, keepdims=True), axis=-1)[..., None]
    m_u = _bf16_floor(np.take_along_axis(v, first_min, -1)[..., 0])
    m = bf16_to_f32(m_u)
    first_max = np.argmax(v == v.max(-1, keepdims=True), axis=-1)[..., None]
    mx = np.take_along_axis(v, first_max, -1)[..., 0]
    d_u = _bf16_ceil(((mx - m).astype(np.float32) / np.float32(15)).astype(np.float32))
    d = bf16_to_f32(d_u)
    inv = np.where(d > 0, np.float32(1) / np.where(d > 0, d, np.float32(1)), np.float32(0)).astype(np.float32)
    t = ((v - m[..., None]).astype(np.float32) * inv[..., None]).astype(np.float32) + np.float32(0.5)
    nib = np.clip(t.astype(np.int32), 0, 15).astype(np.uint8)
    out = np.zeros((n, CH), np.uint8)
    meta_d = np.zeros((n, 256), np.uint16)
    meta_m = np.zeros((n, 256), np.uint16)
    slot = (np.arange(8)[None, :] * 32 + np.arange(32)[:, None]).reshape(-1)   # (r, block) -> block*32 + r
    meta_d[:, slot] = d_u.reshape(n, -1)
    meta_m[:, slot] = m_u.reshape(n, -1)
    out[:, :512] = meta_d.view(np.uint8).reshape(n, 512)
    out[:, 512:1024] = meta_m.view(np.uint8).reshape(n, 512)
    flat = np.zeros((n, 8192), np.uint8)
    flat[:, CHUNK_CODE_IDX] = nib.reshape(n, -1)
    out[:, 1024:] = flat[:, 0::2] | (flat[:, 1::2] << 4)
    return out


def random_q8_chunks(nch: int, rng: np.random.Generator) -> np.ndarray:
    """Synthetic q8 chunks as the reference's tests draw them (test_qwen35.py:621-628):
    bf16 scales U(0, 0.02) + 1e-3 (RNE), int8 codes uniform."""
    out = np.zeros((nch, Q8_CHUNK), np.uint8)
    sc = (rng.random((nch, 256), np.float32) * np.float32(0.02) + np.float32(1e-3)).astype(np.float32)
    out[:, :512] = f32_to_bf16(sc).view(np.uint8).reshape(nch, 512)
    out[:, 512:] = rng.integers(-128, 128, (nch, 8192), dtype=np.int8).view(np.uint8)
    return out


def random_signed_pool(nch: int, rng: np.random.Generator) -> np.ndarray:
    """Synthetic chunks of the signed quantiser: positive bf16 d, mins 0, random nibbles."""
    out = rng.integers(0, 256, (nch, CH), dtype=np.uint8)
    d = (rng.random((nch, 256), np.float32) * np.float32(0.02) + np.float32(1e-3)).astype(np.float32)
    out[:, :512] = f32_to_bf16(d).view(np.uint8).reshape(nch, 512)
    out[:, 512:1024] = 0
    return out


# --------------------------------------------------------------------------
# q8 held exactly as two q4_1 planes (recipes/pack.py:94-117, split_q8_q4_1)
# --------------------------------------------------------------------------

def q8_chunks_rows(chunks: np.ndarray, n: int, k: int, rs: int):
    """q8 chunks in band order -> (scale bits uint16[n, k/32], codes int8[n, k])."""
    nch, _, rows0, cols0 = chunk_geometry(n, k, rs)
    src = np.asarray(chunks, np.uint8).reshape(nch, Q8_CHUNK)
    s16 = np.empty((n, k // BLK), np.uint16)
    q = np.empty((n, k), np.int8)
    sc = np.ascontiguousarray(src[:, :512]).view(np.uint16)                       # [c, block*32 + r]
    code = np.ascontiguousarray(src[:, 512:]).view(np.int8)[:, CHUNK_CODE_IDX].reshape(nch, 32, 8, 32)
    for c in range(nch):
        r0, c0 = int(rows0[c]), int(cols0[c])
        s16[r0:r0 + 32, c0 // BLK:c0 // BLK + 8] = sc[c].reshape(8, 32).T
        q[r0:r0 + 32, c0:c0 + 256] = code[c].reshape(32, 256)
    return s16, q


def q8_0_rows(blocks: np.ndarray):
    """GGUF Q8_0 blocks uint8[n, k/32, 34] -> (bf16 scale bits [n, k/32], codes int8[n, k])."""
    b = np.asarray(blocks, np.uint8)
    n, nb, _ = b.shape
    d = np.ascontiguousarray(b[..., 0:2]).view(np.float16).reshape(n, nb).astype(np.float32)
    return f32_to_bf16(d), np.ascontiguousarray(b[..., 2:34]).view(np.int8).reshape(n, nb * BLK)


def q8_split_parts(s16: np.ndarray, q: np.ndarray, part: int):
    """(d16, m16, codes) of plane `part` (0 hi: d = 16 s, m = -128 s, code (q >> 4) + 8;
    1 lo: d = s, m = 0, code q & 15), for pack_mx_from_parts."""
    s = bf16_to_f32(s16)
    q = np.asarray(q, np.int8).astype(np.int32)
    if part == 0:
        return f32_to_bf16(np.float32(16) * s), f32_to_bf16(np.float32(-128) * s), ((q >> 4) + 8).astype(np.uint8)
    return s16.copy(), np.zeros_like(s16), (q & 15).astype(np.uint8)


def split_q8_chunks(chunks: np.ndarray, part: int) -> np.ndarray:
    """q8 chunks [n, 8704] -> 5120 B q4_1 chunks of one plane of the exact split, in the
    same chunk order (split_q8_q4_1, recipes/pack.py:94-117; pools.cpp split_q4_1_chunks):
    the scales at the same meta index, built by q8_split_parts; code i of the q8 chunk is
    nibble i of the q4_1 chunk (even i low), since the two formats share the code raster."""
    src = np.asarray(chunks, np.uint8).reshape(-1, Q8_CHUNK)
    n = src.shape[0]
    s16 = np.ascontiguousarray(src[:, :512]).view(np.uint16)
    code = np.ascontiguousarray(src[:, 512:]).view(np.int8)
    d16, m16, q = q8_split_parts(s16, code, part)
    out = np.zeros((n, CH), np.uint8)
    out[:, :512] = np.ascontiguousarray(d16, np.uint16).view(np.uint8).reshape(n, 512)
    out[:, 512:1024] = np.ascontiguousarray(m16, np.uint16).view(np.uint8).reshape(n, 512)
    out[:, 1024:] = q[:, 0::2] | (q[:, 1::2] << 4)
    return out


def q8_values(s16: np.ndarray, q: np.ndarray) -> np.ndarray:
    """s * q in f64 per weight (exact)."""
    return np.repeat(bf16_to_f32(s16).astype(np.float64), BLK, axis=1) * np.asarray(q, np.float64)


# The native q8 layout ("mx8", this build's own format): tile (g, kb) = 64 rows x 32 K,
# 2176 bytes at (g * K/32 + kb) * 2176. Codes [0, 2048): lane l = kg * 16 + i holds at
# (r // 2) * 1024 + l * 16 + (r % 2) * 8 the 8 codes of row 16 r + i, k = 32 kb + 8 kg +
# 0..7, as b = q + 128, each dword's bytes in the k order (0, 2, 1, 3); scale
# [2048, 2176): bf16 of row 16 r + i at 2048 + i * 8 + r * 2. Weight s * q.

MX8_TILE = 2176
_MX8_ORDER = np.array([0, 2, 1, 3, 4, 6, 5, 7])     # byte j of an 8-byte group holds k = _MX8_ORDER[j]


def mx8_bytes(n: int, k: int) -> int:
    assert n % MX_ROWS == 0 and k % BLK == 0
    return (n // MX_ROWS) * (k // BLK) * MX8_TILE


def pack_mx8_from_parts(s16: np.ndarray, q: np.ndarray) -> np.ndarray:
    """(bf16 scale bits [N, K/32], int8 codes [N, K]) -> native q8 layout bytes."""
    n, nb = s16.shape
    assert n % MX_ROWS == 0 and q.shape == (n, nb * BLK)
    G = n // MX_ROWS
    b = (np.asarray(q, np.int8).view(np.uint8) ^ 0x80).reshape(n, nb, 4, 8)[..., _MX8_ORDER]   # [n, kb, kg, 8]
    codes = b.reshape(G, 2, 2, 16, nb, 4, 8).transpose(0, 4, 1, 5, 3, 2, 6)               # [G, kb, r//2, kg, i, r%2, 8]
    sc = np.asarray(s16, np.uint16).reshape(G, 4, 16, nb).transpose(0, 3, 2, 1)             # [G, kb, i, r]
    out = np.empty((G, nb, MX8_TILE), np.uint8)
    out[:, :, :2048] = np.ascontiguousarray(codes).reshape(G, nb, 2048)
    out[:, :, 2048:] = np.ascontiguousarray(sc).view(np.uint8).reshape(G, nb, 128)
    return out.reshape(-1)


def unpack_mx8(packed: np.ndarray, n: int, k: int):
    """Native q8 layout bytes -> (bf16 scale bits uint16[n, k/32], codes int8[n, k])."""
    nb, G = k // BLK, n // MX_ROWS
    t = np.asarray(packed, np.uint8).reshape(G, nb, MX8_TILE)
    codes = t[:, :, :2048].reshape(G, nb, 2, 4, 16, 2, 8).transpose(0, 2, 5, 4, 1, 3, 6).reshape(n, nb, 4, 8)
    q = np.empty_like(codes)
    q[..., _MX8_ORDER] = codes
    sc = np.ascontiguousarray(t[:, :, 2048:]).view(np.uint16).reshape(G, nb, 16, 4).transpose(0, 3, 2, 1)
    return sc.reshape(n, nb), (q.reshape(n, k) ^ 0x80).view(np.int8)


def dequant_mx8(packed: np.ndarray, n: int, k: int) -> np.ndarray:
    """Native q8 layout -> f32[n, k] = s * q (exact)."""
    s16, q = unpack_mx8(packed, n, k)
    return (np.repeat(bf16_to_f32(s16), BLK, axis=1) * q.astype(np.float32)).astype(np.float32)


def random_q8_0_blocks(n: int, k: int, rng: np.random.Generator) -> np.ndarray:
    """Seeded GGUF Q8_0 blocks: fp16 d = |N(0,1)| * 0.002 + 1e-4, int8 codes uniform."""
    nb = k // BLK
    b = np.empty((n, nb, 34), np.uint8)
    d = (np.abs(rng.standard_normal((n, nb))) * 0.002 + 1e-4).astype(np.float16)
    b[..., 0:2] = d.view(np.uint8).reshape(n, nb, 2)
    b[..., 2:] = rng.integers(-128, 128, (n, nb, 32), dtype=np.int8).view(np.uint8)
    return b


# --------------------------------------------------------------------------
# The GGUF-direct pool: f32 scales (open_kernels/gguf_pool/gguf_pool.py)
# --------------------------------------------------------------------------
CH_F32 = 6144        # q4 chunk with f32 d[256], f32 m[256], codes[4096]   (gguf_pool.py:19-27)
CH_Q8_F32 = 9216     # q8 chunk with f32 scales[256], int8 codes[8192]    (gguf_pool.py:28)


def pack_gguf_pool_f32(blocks: np.ndarray, rs: int) -> np.ndarray:
    """GGUF Q4_1 / Q4_0 blocks -> the direct pool's 6144 B chunks in band order: fp16 d, m
    widened exactly to f32 (Q4_0: m = -8 d), index kb*32 + r; codes in the pool raster
    (gguf_pool.py:191-213)."""
    n, nb, _ = blocks.shape
    k = nb * BLK
    d, m, q = unpack_q4_1_blocks(blocks)                       # f32, exact widenings
    nch, _, rows0, cols0 = chunk_geometry(n, k, rs)
    out = np.empty((nch, CH_F32), np.uint8)
    for c in range(nch):
        r0, c0 = int(rows0[c]), int(cols0[c])
        kb0 = c0 // BLK
        out[c, 0:1024] = np.ascontiguousarray(d[r0:r0 + 32, kb0:kb0 + 8].T).reshape(-1).view(np.uint8)
        out[c, 1024:2048] = np.ascontiguousarray(m[r0:r0 + 32, kb0:kb0 + 8].T).reshape(-1).view(np.uint8)
        qq = q[r0:r0 + 32, c0:c0 + 256].reshape(2, 16, 256).transpose(0, 2, 1).reshape(-1)
        out[c, 2048:] = qq[0::2] | (qq[1::2] << 4)
    return out.reshape(-1)


def dequant_gguf_pool_f32(pool: np.ndarray, n: int, k: int, rs: int) -> np.ndarray:
    """The direct pool's own f32 reading fl32(q * d + m) -> f32[n, k] (gguf_pool.py:269-320)."""
    nch, _, rows0, cols0 = chunk_geometry(n, k, rs)
    ch = np.asarray(pool, np.uint8).reshape(nch, CH_F32)
    w = np.empty((n, k), np.float32)
    for c in range(nch):
        d = np.ascontiguousarray(ch[c, 0:1024]).view(np.float32).reshape(8, 32)
        m = np.ascontiguousarray(ch[c, 1024:2048]).view(np.float32).reshape(8, 32)
        nib = np.empty(8192, np.uint8)
        nib[0::2] = ch[c, 2048:] & 0xF
        nib[1::2] = ch[c, 2048:] >> 4
        q = nib.reshape(2, 256, 16).transpose(0, 2, 1).reshape(32, 256).astype(np.float32)
        g = np.arange(256) // 32
        r0, c0 = int(rows0[c]), int(cols0[c])
        w[r0:r0 + 32, c0:c0 + 256] = q * d[g, :].T + m[g, :].T
    return w


def pack_gguf_pool_q8_f32(blocks: np.ndarray, rs: int) -> np.ndarray:
    """GGUF Q8_0 blocks -> the direct pool's 9216 B q8 chunks (gguf_pool.py:182-189, 216-227)."""
    b = np.asarray(blocks, np.uint8)
    n, nb, _ = b.shape
    k = nb * BLK
    d = np.ascontiguousarray(b[..., 0:2]).view(np.float16).reshape(n, nb).astype(np.float32)
    q = np.ascontiguousarray(b[..., 2:34]).view(np.int8).reshape(n, k)
    nch, _, rows0, cols0 = chunk_geometry(n, k, rs)
    out = np.empty((nch, CH_Q8_F32), np.uint8)
    for c in range(nch):
        r0, c0 = int(rows0[c]), int(cols0[c])
        out[c, 0:1024] = np.ascontiguousarray(d[r0:r0 + 32, c0 // BLK:c0 // BLK + 8].T).reshape(-1).view(np.uint8)
        out[c, 1024:] = q[r0:r0 + 32, c0:c0 + 256].reshape(2, 16, 256).transpose(0, 2, 1).reshape(-1).view(np.uint8)
    return out.reshape(-1)
