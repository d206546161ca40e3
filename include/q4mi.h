/*
 * q4mi.h -- C ABI of the MI355X (gfx950) Q4_1 dequant-matmul kernels.
 *
 * Plain C: device pointers, sizes and an opaque HIP stream (`void*`, a
 * hipStream_t; NULL = the default stream). No HIP or torch types appear in
 * these signatures, so ctypes / cgo / JNI bind them without HIP headers.
 *
 * Every function returns Q4MI_OK (0) or a negative Q4MI_E* code. All device
 * memory belongs to the caller; the library never allocates. Packed weights,
 * activations, outputs and workspaces must be 16-byte aligned (Q4MI_E_ARG
 * otherwise; the descriptors of q4_gemv_grouped are the caller's to check). Work is enqueued
 * on `stream` and is asynchronous to the host; the functions are re-entrant
 * and keep no global state (calls that share one caller-owned workspace must
 * be ordered on one stream), except q4_gemv_noalloc, whose scratch is one
 * static device array per device (see there).
 *
 * No entry point takes byte counts for its buffers: each pointer must cover the
 * whole region its shape arguments name, in the dtype its enum names -- an
 * activation X of M rows x K is M*K*4 bytes for Q4MI_F32 and M*K*2 for Q4MI_BF16,
 * an f32 output Y[M][N] is M*N*4 bytes, a packed matrix q4_packed_bytes(N, K).
 * A dtype enum that disagrees with the buffer reads or writes past its end (an
 * f32 enum on a bf16 X reads 2*M*K bytes beyond it). The Python layer derives
 * every enum from the tensor and checks every buffer before it calls in.
 *
 * Weights live in the "mx" layout (see q4_packed_bytes): an [N, K] matrix,
 * N % 64 == 0, K % 32 == 0, cut into tiles of 64 rows x 32 K (one GGUF block
 * column) of 1280 bytes: 1024 B of 4-bit codes laid out as the B operand of a
 * 16x16x32 bf16 MFMA, then 256 B of (bf16 d << 16 | bf16 m) scale words.
 * Tiles of one 64-row group are contiguous along K.
 *
 * Reference interfaces replaced (paths under the reference repository):
 *   pack_q4_1_pool / pool layout  open_kernels/q4_1_pack.py:124-142
 *   dequant_pool / dq_chunks_q4_1 open_kernels/q4_1_pack.py:173-180,
 *                                 open_kernels/model/q4nx.py:105-126
 *   gemv_q4 design + kernel       open_kernels/designs/gemv_q4/gemv_q4.py:118-194,
 *                                 designs/gemv_q4/gemv_q4.h:320-341
 *   gemm_q4 (batched decode)      open_kernels/designs/gemm_q4/gemm_q4.py:164-197,
 *                                 designs/gemm_q4/gemm_q4.h:208-226
 *   gemm_q4_prefill               open_kernels/designs/gemm_q4_prefill/gemm_q4_prefill.py:171-177
 *   moe_batch / moe_experts       open_kernels/designs/moe_batch/moe_batch.py:145-146,
 *                                 open_kernels/designs/moe_experts/moe_experts.py:1-43
 */
#ifndef Q4MI_H
#define Q4MI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define Q4MI_OK            0
#define Q4MI_E_SHAPE      -1   /* a dimension is not a multiple the layout needs, or <= 0 */
#define Q4MI_E_ARG        -2   /* NULL or misaligned pointer, bad enum, bad block width */
#define Q4MI_E_WORKSPACE  -3   /* workspace missing or too small */
#define Q4MI_E_LAUNCH     -4   /* the HIP launch itself failed */
#define Q4MI_E_RANGE      -5   /* M or another count out of the supported range */

/* activation dtypes */
#define Q4MI_F32   0
#define Q4MI_BF16  1

/* Library version, e.g. 100 for 0.1.0. */
int q4mi_version(void);

/* Human-readable text for a status code (static storage). */
const char* q4mi_strerror(int status);

/* Bytes of the mx layout for an [N, K] matrix (N % 64 == 0, K % 32 == 0),
 * or Q4MI_E_SHAPE. Same 0.625 B/weight as GGUF Q4_1 (1280 B per 2048 weights).
 * Replaces the size rule of pack_q4_1_pool (q4_1_pack.py:112-121, 5120 B per
 * 32x256 chunk). */
int64_t q4_packed_bytes(int64_t N, int64_t K);

/* GGUF blocks -> mx layout, on the device.
 * `gguf_blocks`: uint8[N][K/32][block_bytes], block_bytes 20 (Q4_1: fp16 d,
 * fp16 m, 16 code bytes) or 18 (Q4_0: fp16 d, codes; its min is -8 d).
 * scale_mode 0: d and m narrowed fp16 -> bf16 round-to-nearest-even, the
 * reference's pool semantics (q4_1_pack.py:104-109, :129-130).
 * scale_mode 1 (opt in, Q4_1 blocks only): GGUF's fp16 d and m kept exactly, the scale
 * word fp16 d << 16 | fp16 m, as the reference's GGUF-direct pool keeps them
 * (open_kernels/gguf_pool/gguf_pool.py:1-17, designs/gemv_q4/gemv_q4.h:54-65). Same tile
 * size; such a matrix is read by the _fp16s entry points (q4_dequant_fp16s, q4_gemv_fp16s,
 * q4_gemv_grouped_fp16s) and by no other.
 * Replaces pack_q4_1_pool (q4_1_pack.py:124-142) as the packer. */
int q4_repack(const uint8_t* gguf_blocks, int block_bytes, uint8_t* packed,
              int64_t N, int64_t K, int scale_mode, void* stream);

/* Reference pool chunks -> mx layout, on the device: the 5120-byte
 * 32-row x 256-K chunks in band order with row split `rs`
 * (q4_1_pack.py:16-34, :112-121; K % 256 == 0, N % (32*rs) == 0). The bytes
 * carry over exactly (bf16 scales, same codes). */
int q4_repack_pool(const uint8_t* pool, int rs, uint8_t* packed,
                   int64_t N, int64_t K, void* stream);

/* The GGUF-direct pool's chunks -> mx layout, on the device: 6144-byte 32-row x 256-K
 * chunks with f32 d[256] @0 and f32 m[256] @1024 (index kb*32 + r, exact widenings of
 * GGUF's fp16 scales; Q4_0's m = -8 d) and the codes @2048 in the pool raster
 * (open_kernels/gguf_pool/gguf_pool.py:19-33, pack_q4_pool :191-213), band order with
 * row split rs. d and m are narrowed to bf16 by RNE, as that pool's kernel does in
 * flight (gguf_pool.py:10-16): the result equals q4_repack of the same GGUF blocks. */
int q4_repack_pool_f32(const uint8_t* pool, int rs, uint8_t* packed,
                       int64_t N, int64_t K, void* stream);

/* GGUF Q4_K super-blocks -> mx layout, on the device. `q4k_blocks`:
 * uint8[N][K/256][144] (fp16 d, fp16 dmin, 12 bytes of packed 6-bit sub-block
 * scales/mins, 128 code bytes; llama.cpp's block_q4_K). Each 32-value sub-block
 * is a Q4_1 block with d' = d * sc, m' = -dmin * min: both products are exact in
 * f32 and are narrowed to bf16 (RNE), the arithmetic of the reference's Q4_K
 * transcode (recipes/pack.py:266-310, q4k_to_q4_1) on GGUF's own block layout
 * (model/gguf_ref.py:224-250). N % 64 == 0, K % 256 == 0. */
int q4_repack_q4k(const uint8_t* q4k_blocks, uint8_t* packed, int64_t N, int64_t K, void* stream);

/* The reference container's Q4_K chunks -> mx layout, on the device. `chunks`:
 * 4736-byte 32-row x 256-K chunks in band order with row split `rs` (rs = 1 is
 * the file's raster order): uint8 scales[8][32] @0 and mins @256 (index
 * g*32 + r), codes @512 (row r of column k in byte 512 + 16k + r/2, even r in
 * the low nibble), bf16 S[32] @4608, bf16 M[32] @4672 (negated). Each (row,
 * 32-K block) becomes d = bf16_rne(S[r] * scales), m = bf16_rne(M[r] * mins),
 * the reference's q4k_to_q4_1 (recipes/pack.py:266-310;
 * src/open_qwen36/pools.cpp:642-663). K % 256 == 0, N % 64 == 0,
 * N % (32*rs) == 0. */
int q4_repack_q4k_chunks(const uint8_t* chunks, int rs, uint8_t* packed,
                         int64_t N, int64_t K, void* stream);

/* Native Q4_K ("mxk" layout): the super-block's own integers, no bf16 collapse. A
 * 64-row x 256-K tile (one super-block per row) is 9728 bytes: the 8 sub-blocks'
 * codes in the mx code layout, per row and sub-block the 8-bit multipliers (sc, mn),
 * per row the f32 bases d and m. Weight = fl32(d sc q + m mn), with d sc and m mn exact
 * in f32: the value the reference's Q4_K GEMM reads (open_kernels/designs/gemm_q4/
 * gemm_q4.h:456-507, gemm_q4k_tile4 :555: value = d sc nib + mcoef mn) and, for GGUF
 * blocks, the GGUF reader's dequant (src/gguf/gguf_file.cpp:611-635). 0.594 bytes per
 * weight against the mx layout's 0.625. Bytes of an [N, K] matrix (N % 64 == 0,
 * K % 256 == 0), or -1: */
int64_t q4_q4k_packed_bytes(int64_t N, int64_t K);

/* GGUF Q4_K super-blocks (uint8[N][K/256][144], as q4_repack_q4k) -> mxk, on the
 * device: d = fp16 d, m = -fp16 dmin, (sc_j, mn_j) the packed 6-bit pairs. */
int q4_repack_q4k_native(const uint8_t* q4k_blocks, uint8_t* packed, int64_t N, int64_t K, void* stream);

/* The reference container's Q4_K chunks (as q4_repack_q4k_chunks) -> mxk, on the
 * device: d = bf16 S[r], m = bf16 M[r], (sc, mn) = (scales[g][r], mins[g][r]). */
int q4_repack_q4k_chunks_native(const uint8_t* chunks, int rs, uint8_t* packed,
                                int64_t N, int64_t K, void* stream);

/* mxk -> f32 [N][K] row-major, w = fl32(q (d sc) + m mn), bit-exact with the values
 * above (the mxk twin of q4_dequant). */
int q4_dequant_q4k(const uint8_t* packed, float* w, int64_t N, int64_t K, void* stream);

/* Workspace bytes q4_gemv_q4k needs (0 if none). */
size_t q4_gemv_q4k_workspace_bytes(int M, int64_t N, int64_t K);

/* Y[M][N] = X[M][K] . W^T over an mxk matrix, 1 <= M <= 16, fp32 accumulate, plus
 * residual (f32 [M][N], may be y) when not NULL: the Q4_K-native skinny GEMM, the
 * counterpart of the reference's gemm_q4k_tile4 (gemm_q4.h:555). Per 32-K block the
 * kernel applies the exact f32 scale d sc and offset m mn to the MFMA's sum of q x.
 * K is split (on whole super-blocks) for matrices of few row groups, as q4_gemv. */
int q4_gemv_q4k(const uint8_t* packed, const void* x, int x_dtype, const float* residual, float* y,
                int M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes, void* stream);

/* Pool chunks of the SIGNED quantiser -> mx layout: 5120-byte chunks laid out as
 * q4_1's, holding w = d * int4(q) with every min 0 (recipes/pack.py:583-603 tells them
 * apart by those zero mins). Read the q4_1 way, exactly: code q ^ 8, m = -8 d
 * (q4_0_to_q4_1, recipes/pack.py:606-622). Band order with row split rs, as
 * q4_repack_pool. */
int q4_repack_pool_signed(const uint8_t* pool, int rs, uint8_t* packed,
                          int64_t N, int64_t K, void* stream);

/* q8 chunks -> mx layout, re-quantised to q4_1 block for block as the reference's
 * requant_q4_1 does (recipes/pack.py:224-263): 8704-byte 32-row x 256-K chunks (bf16
 * scales[256] index kb*32 + r, then int8 codes in the q4_1 code raster), band order
 * with row split rs. Per block: m = min rounded down to bf16, d = (max - m) / 15
 * rounded up to bf16, nibble = clamp(trunc((v - m) * (1/d) + 0.5), 0, 15), each f32
 * operation rounded on its own. Every value lands within d/2 of its reading. */
int q4_repack_q8_chunks(const uint8_t* chunks, int rs, uint8_t* packed,
                        int64_t N, int64_t K, void* stream);

/* One plane of a q8 matrix held exactly as two q4_1 mx matrices (part 0 "hi":
 * d = 16 s, m = -128 s, code (q >> 4) + 8; part 1 "lo": d = s, m = 0, code q & 15;
 * hi + lo = s q exactly -- split_q8_q4_1, recipes/pack.py:94-117). src_format 0:
 * 8704-byte q8 chunks in band order with row split rs (N % (32 rs) == 0, K % 256 == 0);
 * 1: GGUF Q8_0 blocks uint8[N][K/32][34] (fp16 d narrowed to bf16 by RNE, K % 32 == 0);
 * 2: the GGUF-direct pool's 9216-byte q8 chunks (f32 scales @0, codes @1024; scales
 * narrowed to bf16 by RNE; gguf_pool.py:28-33), band order with row split rs. */
int q4_repack_q8_split(const uint8_t* src, int src_format, int rs, int part, uint8_t* packed,
                       int64_t N, int64_t K, void* stream);

/* mx layout -> f32 W[N][K] row-major, w = fl32(q * d + m), bit-exact with
 * dequant_pool / dq_chunks_q4_1 (q4_1_pack.py:155-180, q4nx.py:105-126). */
int q4_dequant(const uint8_t* packed, float* w, int64_t N, int64_t K, void* stream);

/* q4_dequant of a matrix packed with scale_mode 1: w = fl32(q * d + m) with GGUF's fp16 d
 * and m, bit-exact with the reference's f32-scale unpack (q4_1_pack.py:104-109 with
 * scale_dtype float32; q*d has 4 + 11 significant bits, exact in f32). */
int q4_dequant_fp16s(const uint8_t* packed, float* w, int64_t N, int64_t K, void* stream);

/* Workspace bytes q4_gemv needs for (M, N, K); 0 when it needs none (enough
 * 64-row groups to fill the GPU). A short matrix is split along K: the
 * workspace holds the per-split partial sums, which a second launch adds in
 * split order. No initial contents are needed; calls sharing one workspace
 * must be ordered on one stream. The bytes a split call writes (the query's
 * count from the workspace pointer on) must not overlap x, y or, for the _acc
 * forms, res, the partial planes or x_out: workgroups store their partials
 * while others still read those (Q4MI_E_ARG, before any launch). */
size_t q4_gemv_workspace_bytes(int M, int64_t N, int64_t K);

/* Decode GEMV / skinny GEMM: Y[M][N] = X[M][K] . W[N][K]^T, fp32 accumulate,
 * fp32 out. 1 <= M <= 24 (17..24: two 16-token blocks share each weight tile's loads).
 * x_dtype Q4MI_F32 or Q4MI_BF16, X row-major [M][K].
 * Replaces gemv_q4 (M = 1; gemv_q4.py:118-123: pool in, bf16 x in, f32 y out)
 * and gemm_q4 (M = 1..24; gemm_q4.py:9-13, :164-197); Y is the logical [M][N] order
 * (the reference's device order is core-interleaved, check.py:59-79). */
int q4_gemv(const uint8_t* packed, const void* x, int x_dtype, float* y,
            int M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
            void* stream);

/* Bytes of the device array q4_gemv_noalloc keeps its K-split partial sums in (8 MiB per
 * device that runs it, held until the process ends). */
#define Q4MI_NOALLOC_SCRATCH_BYTES (8u << 20)

/* q4_gemv with no workspace argument and no allocation of any kind: its K-split partial
 * sums go to a file-scope device array of Q4MI_NOALLOC_SCRATCH_BYTES, whose per-device
 * address the library looks up on its first call on that device. Same kernels, split
 * order and bits as q4_gemv, for 1 <= M <= 16 (Q4MI_E_RANGE above). Q4MI_E_WORKSPACE when
 * a shape's partials would not fit (none does under the current split policy: at most
 * 8,380,416 bytes for M <= 16). Every
 * call on one device shares that device's array: calls that overlap on one device (other
 * streams or host threads) race, so order them on one stream. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). */
int q4_gemv_noalloc(const uint8_t* packed, const void* x, int x_dtype, float* y,
                    int M, int64_t N, int64_t K, void* stream);

/* Workspace bytes for q4_gemv_rmsnorm / q4_gemv_rmsnorm_acc: q4_gemv_workspace_bytes, and for
 * vocabulary-sized matrices (N / 64 row groups x the split count >= 1024, e.g. an lm_head) room
 * after the split partials for the normalised rows (bf16 [M][K], at the partials' size rounded
 * up to 256 bytes). With that room the rows are normalised once by q4_rmsnorm_add's kernel and
 * the plain GEMV reads them (one more launch, same bits); with less, every workgroup
 * normalises per position as before. The rows' room must not overlap x, x_out or y. */
size_t q4_gemv_rmsnorm_workspace_bytes(int M, int64_t N, int64_t K);

/* The GEMV with its RMSNorm inside: Y = X . W^T with X = bf16(RMSNorm(x) * norm_w), formed per
 * tile from the f32 residual stream x [M][K] (1 <= M <= 16, K <= 16384, norm_w [K] bf16 or
 * f32). Same bits as q4_rmsnorm_add (bf16 out, no add) then q4_gemv: every workgroup first
 * computes the rows' 1/rms with q4_rmsnorm_add's arithmetic. Saves the norm's launch and its
 * bf16 copy in a decode step (the reference's ln design ahead of a projection,
 * designs/ln/ln.py:1-6). Workspace: q4_gemv_rmsnorm_workspace_bytes (q4_gemv's suffices). */
int q4_gemv_rmsnorm(const uint8_t* packed, const float* x, const void* norm_w, int norm_w_dtype, float eps,
                    float* y, int M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
                    void* stream);

/* q4_gemv plus the residual: y = residual + X . W^T (residual f32 [M][N]; it may
 * be y itself, which then accumulates in place). Same workspace as q4_gemv. The
 * residual adds the reference makes after a projection: x_res + o_proj / down
 * (open_kernels/model/replica.py:81, :144; designs/moe_combine/moe_fin.py:1-4). */
int q4_gemv_residual(const uint8_t* packed, const void* x, int x_dtype, const float* residual,
                     float* y, int M, int64_t N, int64_t K, void* workspace,
                     size_t workspace_bytes, void* stream);

/* The q8 GEMV (the reference's gemv_q8 sibling, designs/gemv_q4's q8 twin): Y[M][N] =
 * X . (HI + LO)^T for a q8 matrix split by q4_repack_q8_split, exact in the weights;
 * both planes stream in one launch with shared activation fragments. residual (f32
 * [M][N], may be y) is added when not NULL. Same shapes (1 <= M <= 16) and workspace as
 * q4_gemv. */
int q4_gemv_q8(const uint8_t* hi, const uint8_t* lo, const void* x, int x_dtype,
               const float* residual, float* y, int M, int64_t N, int64_t K,
               void* workspace, size_t workspace_bytes, void* stream);

/* Native q8 ("mx8" layout): a 64-row x 32-K tile is 2176 bytes, the 8-bit codes as
 * b = q + 128 plus one bf16 scale per row (1.0625 bytes per weight, GGUF Q8_0's density,
 * against the split pair's 1.25). Weight = s * q, exact: the same values as the split's
 * hi + lo planes. The counterpart of the reference's q8 GEMV (designs/gemv_q4/gemv_q8.h,
 * designs/lm_head_q8). Bytes of an [N, K] matrix (N % 64 == 0, K % 32 == 0), or -1: */
int64_t q4_q8_native_packed_bytes(int64_t N, int64_t K);

/* q8 weights -> mx8, on the device; src_format and rs as q4_repack_q8_split (0: 8704-byte
 * chunks, 1: GGUF Q8_0 blocks, 2: the GGUF-direct pool's 9216-byte chunks), scales
 * narrowed to bf16 as there. */
int q4_repack_q8_native(const uint8_t* src, int src_format, int rs, uint8_t* packed,
                        int64_t N, int64_t K, void* stream);

/* mx8 -> f32 [N][K] row-major, w = s * q (exact). */
int q4_dequant_q8_native(const uint8_t* packed, float* w, int64_t N, int64_t K, void* stream);

/* Q4_0-native ("mx0" layout): Q4_0 stores no min, so the 64-row x 32-K tile is the mx
 * codes plus one bf16 d per row, 1152 bytes (0.5625 bytes per weight against the widened
 * Q4_1's 0.625). Weight = fl32(q d + m) with m = -8 d, exact: the same values as q4_repack of
 * the same 18-byte blocks. The counterpart of the reference's Q4_0-native chunk
 * (open_kernels/q4_1_pack.py:145-152, 4608 B: the d plane and the codes, no m plane) and of
 * its GEMV build that reads it (designs/gemv_q4/gemv_q4.h:66-82, GEMV_Q4_0_NATIVE, m = -8 d).
 * Bytes of an [N, K] matrix (N % 64 == 0, K % 32 == 0), or -1: */
int64_t q4_q40_packed_bytes(int64_t N, int64_t K);

/* Q4_0 -> mx0, on the device. src_format 0: GGUF Q4_0 blocks (18 B, row-major [N][K/32]),
 * d narrowed fp16 -> bf16 by RNE as pack_q4_1_pool narrows it (q4_1_pack.py:129-130);
 * 1: the reference's 4608 B Q4_0-native chunks in pool order with row split rs
 * (pack_q4_0_native_pool, q4_1_pack.py:148-152; K % 256 == 0, N % (32 rs) == 0), bytes
 * carried over. */
int q4_repack_q40(const uint8_t* src, int src_format, int rs, uint8_t* packed, int64_t N, int64_t K,
                  void* stream);

/* mx0 -> f32 [N][K] row-major, w = fl32(q d - 8 d) (bit-exact with the reference's
 * dequant_chunk of the same Q4_0 values, q4_1_pack.py:155-170). */
int q4_dequant_q40(const uint8_t* packed, float* w, int64_t N, int64_t K, void* stream);

/* Y[M][N] = X[M][K] . W^T over an mx0 matrix, 1 <= M <= 16, plus residual (f32 [M][N], may
 * be y) when not NULL. q4_gemv's work items, split plan and workspace
 * (q4_gemv_workspace_bytes); bit-identical to q4_gemv over q4_repack of the same Q4_0
 * blocks. Replaces gemv_q4 built with GEMV_Q4_0_NATIVE (gemv_q4.h:66-82, :235-238). */
int q4_gemv_q40(const uint8_t* packed, const void* x, int x_dtype, const float* residual, float* y,
                int M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes q4_gemv_q8_native needs (0 if none; the same as q4_gemv's). */
size_t q4_gemv_q8_native_workspace_bytes(int M, int64_t N, int64_t K);

/* Y[M][N] = X[M][K] . W^T over an mx8 matrix, 1 <= M <= 16, fp32 accumulate, plus
 * residual (f32 [M][N], may be y) when not NULL. Per 64 x 32 tile one code load feeds two
 * MFMAs per row tile on the code's nibble planes; acc += s (16 P_hi + P_lo) - 128 s sum x. */
int q4_gemv_q8_native(const uint8_t* packed, const void* x, int x_dtype, const float* residual, float* y,
                      int M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes q4_gemv_swiglu needs for (M, F, K); 0 when it needs none. */
size_t q4_gemv_swiglu_workspace_bytes(int M, int64_t F, int64_t K);

/* The FFN's first half with SwiGLU fused: h[M][F] = silu(X . G^T) * (X . U^T), gate G
 * and up U two mx matrices [F, K] (e.g. the two halves of one fused gate/up buffer),
 * fp32 accumulate; h stored f32 or bf16 (RNE, h_dtype), ready for the down GEMV.
 * silu(g) = g / (1 + exp(-g)). 1 <= M <= 16, F % 64 == 0. Replaces the gate/up GEMVs
 * plus the silu_mul design (open_kernels/designs/silu_mul/silu_mul.cc: h = bf16(silu(g)
 * * u)); the MoE kernel's own mb_silu_tile step (moe_batch.h:181-202) is q4_moe_gemv's. */
int q4_gemv_swiglu(const uint8_t* gate, const uint8_t* up, const void* x, int x_dtype,
                   void* h, int h_dtype, int M, int64_t F, int64_t K,
                   void* workspace, size_t workspace_bytes, void* stream);

/* q4_gemv_swiglu with its RMSNorm inside, as q4_gemv_rmsnorm (x the f32 residual stream,
 * 1 <= M <= 16, K <= 16384): the bits of q4_rmsnorm_add then q4_gemv_swiglu. */
int q4_gemv_swiglu_rmsnorm(const uint8_t* gate, const uint8_t* up, const float* x, const void* norm_w,
                           int norm_w_dtype, float eps, void* h, int h_dtype, int M, int64_t F, int64_t K,
                           void* workspace, size_t workspace_bytes, void* stream);

/* The K-split reduction deferred into the next norm-fused GEMV (a decode step's o and down
 * projections feed the residual stream that the next RMSNorm reads). In the reference the
 * split GEMV's partials are summed by the kernel's own reduction (split_reduce in the
 * gemv design, open_kernels/designs/gemv_q4/gemv_q4.py) and the residual add and norm
 * follow as separate steps (model/replica.py:81, :144; designs/ln/ln.py:1-6); here the
 * three become the prelude of the GEMV that consumes the norm. */

/* The split count q4_gemv plans for an N x K matrix (1: unsplit; 0: invalid shape). */
int q4_gemv_split_count(int64_t N, int64_t K);

/* The partial sums of a K-split GEMV, left unreduced: part[s][M][N] (f32) is X . W^T over
 * the s-th of S contiguous K ranges (1 <= S <= 16, S <= K / 32, 1 <= M <= 16). With S =
 * q4_gemv_split_count(N, K) the planes added in split order are q4_gemv's Y bit for bit. */
int q4_gemv_partials(const uint8_t* packed, const void* x, int x_dtype, float* part, int S, int M,
                     int64_t N, int64_t K, void* stream);

/* q4_gemv_rmsnorm of x = res + ((0 + part[0]) + part[1] + ...) (S planes of [M][K], in
 * split order; S = 0: x = res; S = 1: res + part[0]), which is also stored to x_out [M][K]
 * (the residual stream's next value: q4_gemv_residual's bits for the GEMV that made the
 * planes). x_out must not overlap res, part or y. M = 1 with K <= 4096 and a grid of at most
 * one workgroup per CU reduces inside the GEMV's workgroups; other shapes add one reduce
 * launch first (vocabulary-sized matrices given q4_gemv_rmsnorm_workspace_bytes: one launch
 * that reduces and normalises, K <= 4096). Workspace as q4_gemv_rmsnorm; where the GEMV itself is split (e.g. 4096 x 4096 at
 * M = 1), its partials must not overlap res, part, x_out or y (Q4MI_E_ARG): a workspace
 * shared with the planes of q4_gemv_partials is carved apart from them. */
int q4_gemv_rmsnorm_acc(const uint8_t* packed, const float* res, const float* part, int S,
                        const void* norm_w, int norm_w_dtype, float eps, float* x_out, float* y, int M,
                        int64_t N, int64_t K, void* workspace, size_t workspace_bytes, void* stream);

/* q4_gemv_swiglu_rmsnorm of the same x = res + partials, stored to x_out, as
 * q4_gemv_rmsnorm_acc. */
int q4_gemv_swiglu_rmsnorm_acc(const uint8_t* gate, const uint8_t* up, const float* res, const float* part,
                               int S, const void* norm_w, int norm_w_dtype, float eps, float* x_out, void* h,
                               int h_dtype, int M, int64_t F, int64_t K, void* workspace,
                               size_t workspace_bytes, void* stream);

/* The decoder layer's GEMV chain between two attentions at M = 1, as one persistent launch
 * (one workgroup per CU, phases handed over by device-scope counters in the workspace; the
 * reference's whole-layer dispatch, open_kernels/designs/dense/dx.py:1-5, with attention
 * left out):
 *   x_mid  = x + o . attn                                   (attn bf16 [H])
 *   h      = bf16(silu(gate . n1) * (up . n1)),  n1 = bf16(RMSNorm(x_mid) * nw_post)
 *   down_planes[s] = the s-th K split of down . h, s < Sd  (f32 [Sd][H])
 *   x_next = x_mid + ((0 + down_planes[0]) + down_planes[1] + ...)
 *   qkv_planes[s]  = the s-th K split of qkv . n2, s < Sq  (f32 [Sq][NQ]),
 *                    n2 = bf16(RMSNorm(x_next) * nw_next)
 * o [H, H], gate and up [F, H], down [H, F], qkv [NQ, H] in the mx layout (bf16 scale words);
 * norm weights f32 or bf16 (nw_dtype); RMSNorm as q4_rmsnorm_add. qkv NULL (the last layer):
 * the chain ends with down_planes (nw_next, x_next, qkv_planes unused), which the next norm
 * GEMV adds (q4_gemv_rmsnorm_acc). Split counts: q4_decode_segment_splits. The sums of
 * the planes in split order are the projections' outputs.
 * Shapes: H, F, NQ multiples of 64, H <= 4096, H and F >= 256. x_next may be x; x_mid,
 * the planes and the workspace must not overlap each other or x, attn and x_next
 * (Q4MI_E_ARG). The workspace (q4_decode_segment_workspace_bytes) starts with the
 * hand-over counters: its first 12800 bytes must be zero before the first call on it; each
 * call leaves them ready for the next (not all zero). The 32-bit word at byte 12544 becomes
 * nonzero if a hand-over timed out (about a second: the grid could not be resident); the
 * outputs are then not valid and the counters must be zeroed again. Calls sharing one
 * workspace must not overlap in time. */
size_t q4_decode_segment_workspace_bytes(int64_t H, int64_t F, int64_t NQ);
int q4_decode_segment_splits(int64_t H, int64_t F, int64_t NQ, int* splits /* [3]: So, Sd, Sq */);
int q4_decode_segment(const uint8_t* o, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                      const uint8_t* qkv, const void* attn, const float* x, const void* nw_post,
                      const void* nw_next, int nw_dtype, float eps, float* x_mid, float* x_next,
                      float* down_planes, float* qkv_planes, int64_t H, int64_t F, int64_t NQ,
                      void* workspace, size_t workspace_bytes, void* stream);

/* The activation producer: per row m < M of N values,
 *   y = x + add (add may be NULL; y may be NULL, or x itself when N <= 16384),
 *   xn = (y * r) * w, r = 1 / sqrt(mean(y^2) + eps) with the sum in fp64,
 * w f32 or bf16 [N] (w_dtype), xn stored f32 or bf16 (RNE, xn_dtype). The reference's
 * ln design (open_kernels/designs/ln/ln.py:1-6) and rms_vec
 * (src/open_qwen36/block_host.cpp:42-47). */
int q4_rmsnorm_add(const float* x, const float* add, const void* w, int w_dtype, float* y,
                   void* xn, int xn_dtype, int M, int64_t N, float eps, void* stream);

/* One matrix of a grouped GEMV launch (device-resident array of these). */
typedef struct q4_gemv_desc {
    const uint8_t* packed;   /* mx layout, [N, K] */
    const void* x;           /* [M][K] activations (dtype of the launch) */
    float* y;                /* [M][N] output */
    int64_t N;
    int64_t K;
    int64_t item_begin;      /* sum of N/64 over the descriptors before this one */
} q4_gemv_desc;

/* Many independent GEMVs in ONE launch: descriptor i covers work items
 * [item_begin_i, item_begin_i + N_i/64). `descs` is a DEVICE pointer to
 * `count` descriptors sorted by item_begin; total_items = sum of N_i/64.
 * Same M and x dtype for all. The counterpart of the reference's fused
 * multi-projection dispatches (one xclbin running several gemv_q4 bands,
 * gemv_q4.py:46-53 YOFF/YTOT; designs/dense, designs/moe_experts). */
int q4_gemv_grouped(const q4_gemv_desc* descs, int count, int64_t total_items,
                    int M, int x_dtype, void* stream);

/* q4_gemv_residual and q4_gemv_grouped over matrices packed with scale_mode 1 (fp16 d and m
 * in the scale words): the same work items, plans, workspaces and arithmetic, d and m
 * converted from fp16 (1 <= M <= 16). The GGUF-direct pool's exact-scale GEMV
 * (designs/gemv_q4/gemv_q4.h:54-65). */
int q4_gemv_fp16s(const uint8_t* packed, const void* x, int x_dtype, const float* residual, float* y,
                  int M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes, void* stream);
int q4_gemv_grouped_fp16s(const q4_gemv_desc* descs, int count, int64_t total_items,
                          int M, int x_dtype, void* stream);

/* Workspace bytes q4_logits_topk needs for M rows of n logits and k (0 if none). */
size_t q4_topk_workspace_bytes(int M, int64_t n, int k);

/* The sampling epilogue: for each of M rows of f32 logits (row stride ld >= n),
 * the k largest of logits[m][0..n) (1 <= k <= 64), value descending and the
 * lower id first on a tie, into ids int32[M][k] and (if not NULL) vals
 * f32[M][k]. k = 1 is the greedy argmax. mode 1 ranks what the sampler sees:
 * each logit rounded to bf16 (RNE), an f32 subnormal read as 0 -- the greedy
 * pick of Sampler::sample_greedy over Engine::logits_view's bf16 logits
 * (src/common/modules/sampler.cpp:355-430, src/open_qwen36/engine.cpp:125-131;
 * stated as argmax_bf16, src/open_qwen36/cli.cpp:103-113), and the order of
 * Sampler::sampler_topk_apply (sampler.cpp:222-245). mode 0 ranks the f32
 * logits themselves. Both read -0 as +0 and NaN below every number; vals are
 * the ranked values (bf16-rounded in mode 1). A row with fewer than k entries
 * pads with id -1, value -inf. */
int q4_logits_topk(const float* logits, int64_t ld, int M, int64_t n, int k, int mode,
                   int32_t* ids, float* vals, void* workspace, size_t workspace_bytes,
                   void* stream);

/* Workspace bytes q4_lm_head_topk needs (0 if none). */
size_t q4_lm_head_workspace_bytes(int M, int64_t N, int64_t K, int k);

/* lm_head at vocabulary scale with its sampling epilogue: logits[M][N] =
 * q4_gemv(packed [N, K], x [M][K]) (1 <= M <= 16), then q4_logits_topk over the
 * first n_valid <= N rows of each token (rows past the tokenizer's vocabulary
 * are padding, read as -inf by Engine::logits_view, engine.cpp:129-130).
 * Replaces the lm_head_q4 design (designs/lm_head_q4/lm_head_q4.py: pool W,
 * bf16 x, f32 logits) plus the host's greedy / top-k pass over its logits. */
int q4_lm_head_topk(const uint8_t* packed, const void* x, int x_dtype, float* logits,
                    int M, int64_t N, int64_t K, int64_t n_valid, int k, int mode,
                    int32_t* ids, float* vals, void* workspace, size_t workspace_bytes,
                    void* stream);

/* Workspace bytes q4_gemm_prefill needs (0 if none). */
size_t q4_gemm_prefill_workspace_bytes(int T, int64_t N, int64_t K);

/* Prefill GEMM: Y[T][N] = X[T][K] . W[N][K]^T with W dequantized into LDS
 * tiles feeding MFMA, fp32 accumulate, fp32 out. Any T >= 0, N % 64 == 0,
 * K % 32 == 0. precision 0 (default): each weight row and each token row is
 * scaled by a power of two into fp16's range (the weights' exponents and fp16
 * scale words are the matrix's prefill scales, see q4_prefill_scales, computed
 * into the workspace on every call), each weight is rounded once to fp16
 * (11-bit significand; bf16 X converts exactly; f32 X goes through twice, as
 * its fp16 rounding and the fp16 remainder) and fed to the fp16 MFMA, whose
 * dense peak equals bf16's on CDNA4; the outputs are scaled back exactly.
 * precision 1: the reference's own tile, RNE_bf16(fl32(q*d+m)), into the
 * bf16 MFMA (gemm_q4_dequant.h:283-286; its rel_fro bar is 5e-3).
 * Replaces gemm_q4_prefill (gemm_q4_prefill.py:171-177: pool W, bf16 X,
 * f32 Y[N][T]); Y here is token-major [T][N], the engine's order after
 * host::transpose (core.cpp:2955-2963). */
int q4_gemm_prefill(const uint8_t* packed, const void* x, int x_dtype, float* y,
                    int T, int64_t N, int64_t K, int precision,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of an [N, K] matrix's prefill scales (0 for a shape the layout rejects). */
size_t q4_prefill_scales_bytes(int64_t N, int64_t K);

/* The prefill scales of an mx matrix, which precision 0 of the prefill GEMM reads instead of
 * the tiles' bf16 scale words: per row n an exponent e_n with max over its 32-K blocks of
 * (15 |d| + |m|) * 2^-e_n in [2^14, 2^15) (int32 [N]), and every block's (d, m) again as
 * fp16(d 2^-e_n) << 16 | fp16(m 2^-e_n), in the tiles' scale-block word order (4 bytes per
 * row and block). Every weight q d + m then fits fp16 with its 11-bit significand whatever
 * its row's magnitude; the GEMM multiplies row n's outputs by 2^e_n back, exactly. `scales`
 * (q4_prefill_scales_bytes) is caller-owned; weights are static, so compute it once per
 * matrix. No counterpart in the reference, whose prefill tile is bf16
 * (gemm_q4_dequant.h:283-286): it makes the fp16 tile exact in range. */
int q4_prefill_scales(const uint8_t* packed, int64_t N, int64_t K, void* scales, size_t scales_bytes,
                      void* stream);

/* Workspace bytes q4_gemm_prefill_scaled needs (0 if none). */
size_t q4_gemm_prefill_scaled_workspace_bytes(int T, int64_t N, int64_t K);

/* q4_gemm_prefill at precision 0 with the matrix's prefill scales given (q4_prefill_scales),
 * so a call does not compute them again. Same shapes, bits and bar. */
int q4_gemm_prefill_scaled(const uint8_t* packed, const void* scales, const void* x, int x_dtype, float* y,
                           int T, int64_t N, int64_t K, void* workspace, size_t workspace_bytes, void* stream);

/* Prepared activations: q4_gemm_prefill's activation pre-pass on its own, so one producer
 * output is converted once and read by several projections (gate and up of an FFN; Q, K
 * and V), or written in this layout by the producer itself. The buffer holds the GEMM's
 * 16-bit activation planes (one; two for f32 x in precision 0: value and fp16 remainder) in
 * the pipelined kernel's tiled image (K % 64 == 0; rows [T][K] otherwise), then the
 * per-token exponents (precision 0). The reference's prefill design likewise takes X
 * pre-tiled for its B operand, the tiling being the host's job (gemm_q4_prefill.py:19-22,
 * :68-70). Bytes, or 0 for bad arguments: */
size_t q4_prefill_prepared_bytes(int T, int64_t K, int x_dtype, int precision);
int q4_prefill_prepare(const void* x, int x_dtype, int T, int64_t K, int precision,
                       void* prepared, size_t prepared_bytes, void* stream);

/* The RMSNorm producer writing prepared activations directly (one launch): per token row
 *   y  = x + add (f32 [T][K]; add and y optional; y may be x, no other overlap), where add
 *        is add_planes planes [add_planes][T][K] summed in q4_gemm_prefill's split-reduce
 *        order (((p0 + p1) + p2) ...): a K-split projection's unreduced partials
 *        (q4_gemm_prefill_prepared_partials) land here with no reduce launch; add_planes 0
 *        with add NULL, 1 for a plain addend, at most 64,
 *   xn = bf16((y * r) * w), r = 1 / sqrt(mean(y^2) + eps) as q4_rmsnorm_add forms it,
 * and `prepared` = q4_prefill_prepare of xn as bf16 (q4_prefill_prepared_bytes(T, K,
 * Q4MI_BF16, precision) bytes): the same bits as q4_rmsnorm_add (bf16 xn) followed by
 * q4_prefill_prepare, without the bf16 row in memory or the pre-pass launch. K % 32 == 0,
 * K <= 16384; w [K] f32 or bf16 (w_dtype). Replaces the ln design in front of a prefill
 * projection (designs/ln/ln.py:1-6, xn = bf16(y * rsqrt(mean(y^2) + eps) * w)) together with
 * the host's pre-tiling of the GEMM's X (block_host.cpp:228-244). */
int q4_rmsnorm_prepare(const float* x, const float* add, int add_planes, const void* w, int w_dtype, float* y, int T,
                       int64_t K, float eps, int precision, void* prepared, size_t prepared_bytes, void* stream);

/* The K splits the prefill GEMM's plan takes for (T, N, K) (1: unsplit), 0 for bad shapes. */
int q4_prefill_split_count(int T, int64_t N, int64_t K);

/* q4_gemm_prefill_prepared without the split reduce: plane s of the plan's S K-splits at
 * part + s T N (f32 [S][T][N]; S = q4_prefill_split_count; the whole product when S = 1). The
 * planes summed in order are the prepared GEMM's Y bit for bit; q4_rmsnorm_prepare takes them
 * as its addend. One activation pass only (bf16 x, or precision 1). part_bytes is part's size:
 * below S T N 4 for this process's plan the call returns Q4MI_E_WORKSPACE before any launch
 * (the plan follows the device's CU count, so query q4_prefill_split_count on the device that
 * runs the call). Replaces the reference's down K-pieces summed on the host
 * (ironutil.py:98-115) with the sum folded into the next layer's norm. */
int q4_gemm_prefill_prepared_partials(const uint8_t* packed, const void* scales, const void* prepared, int x_dtype,
                                      float* part, size_t part_bytes, int T, int64_t N, int64_t K, int precision,
                                      void* stream);

/* The SwiGLU producer writing the down projection's prepared activations (one launch): per
 * token row h[f] = bf16(silu(g[t][f]) * u[t][f]), silu(g) = g / (1 + exp(-g)), from f32 rows
 * g and u with row strides ldg / ldu in elements (a fused [T][2F] gate/up output: u = g + F,
 * ldg = ldu = 2F), and `prepared` = q4_prefill_prepare of h as bf16
 * (q4_prefill_prepared_bytes(T, F, Q4MI_BF16, precision) bytes). h [T][F] bf16 is also
 * stored when not NULL. F % 32 == 0, F <= 16384, strides % 4 == 0. Replaces the reference's
 * bf16 SwiGLU between the FFN's GEMMs (moe_batch.h:181-202, mb_silu_tile) and the host's X
 * tiling (block_host.cpp:228-244). */
int q4_swiglu_prepare(const float* g, const float* u, int64_t ldg, int64_t ldu, int T, int64_t F, int precision,
                      void* h, void* prepared, size_t prepared_bytes, void* stream);

/* The FFN's gate/up prefill GEMM with SwiGLU in its epilogue: h[T][F] bf16 =
 * bf16(silu(X . G^T) * (X . U^T)) from prepared activations (one activation pass: bf16 x, or
 * precision 1), over gate_up, an mx matrix [2F, K] whose 64-row groups alternate gate / up
 * (the q4_moe_gemv expert layout), with its prefill scales for precision 0 (q4_prefill_scales
 * of that matrix). Each h is what q4_swiglu_prepare forms from the plain GEMM's f32 gate and
 * up outputs (the same GEMM bits where that GEMM's plan is unsplit), without the f32 output
 * in memory. 256-row tiles, no K split. F % 128 == 0, K % 64 == 0. Replaces the reference's
 * gate/up prefill dispatches and the bf16 SwiGLU after them (moe_batch.h:181-202). */
int q4_gemm_prefill_swiglu(const uint8_t* gate_up, const void* scales, const void* prepared, int x_dtype, void* h,
                           int T, int64_t F, int64_t K, int precision, void* stream);

/* Workspace of q4_gemm_prefill_prepared: the K-split partials only (0 when unsplit). */
size_t q4_gemm_prefill_prepared_workspace_bytes(int T, int64_t N, int64_t K);

/* q4_gemm_prefill over prepared activations (x_dtype and precision as prepared; precision 0
 * takes the matrix's prefill scales). Same bits as q4_gemm_prefill / _scaled on the same X. */
int q4_gemm_prefill_prepared(const uint8_t* packed, const void* scales, const void* prepared, int x_dtype,
                             float* y, int T, int64_t N, int64_t K, int precision, void* workspace,
                             size_t workspace_bytes, void* stream);

/* Workspace bytes q4_moe_gemv needs. */
size_t q4_moe_workspace_bytes(int T, int E, int topk, int H, int F);

/* Routed MoE expert block for T decode tokens:
 *   out[t] = sum_j topk_w[t][j] * down_e( silu(gate_e . x_t) * (up_e . x_t) ),
 *   e = topk_ids[t][j],
 * fp32 h, fp32 accumulate, fp32 out[T][H].
 * gate_up: E experts, each an mx matrix [2F, H] whose row groups alternate
 *   gate / up (64 gate rows, then the same 64 rows of up, ...);
 * down: E experts, each an mx matrix [H, F];
 * x: [T][H] in x_dtype; topk_ids int32 [T][topk] in [0, E); topk_w f32.
 * H % 64 == 0, F % 64 == 0, 1 <= T*topk <= 4096, topk <= 16, E <= 8192; ids outside
 * [0, E) contribute nothing.
 * Replaces moe_batch (moe_batch.py:145-281, per-slot
 * y = down(silu(gate x) * (up x))) with the host gather/scatter of
 * Core::moe_block (core.cpp:5150-5245) moved onto the device. */
int q4_moe_gemv(const uint8_t* gate_up, const uint8_t* down, const void* x, int x_dtype,
                const int32_t* topk_ids, const float* topk_w, float* out,
                int T, int E, int topk, int64_t H, int64_t F,
                void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes q4_moe_prefill needs (sized for any routing of T tokens x topk). */
size_t q4_moe_prefill_workspace_bytes(int T, int E, int topk, int H, int F);

/* The routed MoE block at prefill scale (any T; the same formula and operand layouts as
 * q4_moe_gemv): the pairs routed to each expert are batched into 256-token tiles on the
 * device and every expert's gate/up and down run as tiles of the prefill GEMM, one launch
 * each over all experts; then out[t] = sum_j topk_w[t][j] y[t][j] in slot order j.
 * precision 0: fp16 tiles with power-of-two scaling as q4_gemm_prefill precision 0, with
 * gate_up_scales / down_scales = q4_prefill_scales of the stacked matrices ([E 2F, H] and
 * [E H, F]); f32 x and h go in two passes (value and remainder). precision 1: the reference's
 * bf16 tile RNE(q d + m), x and h rounded to bf16 (scales may be NULL). precision 2: the fp16
 * tile of precision 0 with h rounded to bf16 as the reference's kernel rounds it, so down
 * takes one pass (scales as precision 0).
 * H % 256 == 0, F % 128 == 0, 1 <= topk <= 16, T * topk <= 2^22, E <= 8192.
 * Replaces the host loop over expert dispatches of 256 slots (Core::moe_block,
 * core.cpp:5163-5178; moe_batch.h:98-172 mb_step_parity / mb_step_tile, h in bf16 as
 * moe_batch.h:181-202). */
int q4_moe_prefill(const uint8_t* gate_up, const uint8_t* down, const void* gate_up_scales,
                   const void* down_scales, const void* x, int x_dtype, const int32_t* topk_ids,
                   const float* topk_w, float* out, int T, int E, int topk, int64_t H, int64_t F,
                   int precision, void* workspace, size_t workspace_bytes, void* stream);

/* The same block with the residual and a gated shared expert folded into the combine:
 *   out[t] = (residual[t] + sum_j topk_w[t][j] * y[t][j]) + sigmoid(x[t] . sgw) * shared[t],
 * residual f32 [T][H] (may be NULL, may alias out), shared f32 [T][H] (the shared expert's
 * output) and shared_gate_w bf16 [H] (sgw), both NULL or both given. The gate's dot product
 * runs in fp32. Replaces the routed-weight combine plus residual of moe_fin
 * (designs/moe_combine/moe_fin.py:1-4, designs/moe_experts/moe_fin.cc; moe_acc.cc's sum). */
int q4_moe_gemv_fin(const uint8_t* gate_up, const uint8_t* down, const void* x, int x_dtype,
                    const int32_t* topk_ids, const float* topk_w, const float* residual,
                    const float* shared, const uint16_t* shared_gate_w, float* out,
                    int T, int E, int topk, int64_t H, int64_t F,
                    void* workspace, size_t workspace_bytes, void* stream);

/* The whole decode MoE block with its shared expert inside the same launches (one
 * dispatch chain: the expert kernels, then the finish):
 *   out[t] = (residual[t] + sum_j topk_w[t][j] y[t][j]) + sigmoid(x[t] . sgw) * y_s[t],
 *   y_s[t] = down_s(silu(gate_s x[t]) * (up_s x[t])), h_s in fp32,
 * the routed y as q4_moe_gemv. The shared expert's gate/up is shared_gate_up [2 Fs, H]
 * (gate and up 64-row groups interleaved, as an expert of gate_up) and its down shared_down
 * [H, Fs], Fs % 64 == 0; its workgroups lead the expert kernels' grids, every token taking
 * it with weight sigmoid(x . sgw) (shared_gate_w bf16 [H], the dot product in fp32).
 * residual may be NULL or alias out; out must not overlap the workspace
 * (q4_moe_shared_workspace_bytes: q4_moe_gemv's, then h_s [T][Fs] and y_s [T][H] f32).
 * Replaces the reference's one-dispatch block, 8 routed experts plus the shared expert as a
 * 9th streamed the same way and the combine (designs/moe_experts/moe_experts.py:1-13,
 * moe_fin.cc), and the replica's moe_decode (model/replica.py:131-144). */
size_t q4_moe_shared_workspace_bytes(int T, int E, int topk, int H, int F, int Fs);
int q4_moe_gemv_shared(const uint8_t* gate_up, const uint8_t* down, const uint8_t* shared_gate_up,
                       const uint8_t* shared_down, int64_t Fs, const uint16_t* shared_gate_w,
                       const void* x, int x_dtype, const int32_t* topk_ids, const float* topk_w,
                       const float* residual, float* out, int T, int E, int topk, int64_t H, int64_t F,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Measurement probes (no counterpart in the reference: on-box reference points for the
 * roofline fractions the benchmark reports).
 * q4_probe_stream_read: `workgroups` workgroups of 256 threads read `bytes` (a multiple of
 * 16) of buf once, in contiguous shares, with 16-byte non-temporal loads; the xor of the
 * words lands in out (q4_probe_stream_read_out_bytes(workgroups) bytes). Bytes / time is
 * the HBM read rate a plain stream sustains (buf beyond the 256 MB MALL).
 * q4_probe_mfma: `workgroups` workgroups of 4 waves each run iters rounds of independent
 * v_mfma_f32_16x16x32_f16 (16 * 16 * 32 * 2 flops each) on register operands, 8 per round
 * with operands NULL (the same constant A and B every time), 64 per round otherwise: each lane
 * then loads 8 A and 8 B fragments (operands = fp16 [64 lanes][16][8], 16 KB, 16-byte
 * aligned) and consecutive MFMAs pair different sets, so the multipliers toggle as on real
 * data. One float per thread goes to out (workgroups * 256 floats). Flops / time is the dense
 * fp16 MFMA rate with no operand traffic; workgroups = k x CUs runs k waves per SIMD. */
size_t q4_probe_stream_read_out_bytes(int workgroups);
int q4_probe_stream_read(const void* buf, size_t bytes, int workgroups, uint32_t* out, void* stream);
int q4_probe_mfma(int workgroups, int iters, const void* operands, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* Q4MI_H */
