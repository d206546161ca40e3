// repack.hip -- GGUF blocks / reference pool chunks -> mx layout, and the
// bit-exact dequant of the mx layout. One thread per (row, 32-K block).
//
// Reference semantics followed:
//   GGUF Q4_1 block: fp16 d | fp16 m | 16 bytes, byte j = value j (low nibble)
//     and value j+16 (high nibble); Q4_0 has no m and reads as m = -8 d
//     (open_kernels/q4_1_pack.py:1-9, :84-101).
//   d, m narrowed fp16 -> bf16 by round-to-nearest-even (q4_1_pack.py:104-109,
//     :129-130): the only change to the GGUF bytes.
//   pool chunk: 32 rows x 256 K, d bf16[256] @0 index kb*32 + r, m @512, code
//     nibble p = (r/16)*4096 + k*16 + r%16 @1024 (even p = low half), chunks
//     in band order with row split rs (q4_1_pack.py:16-34, :112-142).
//   dequant: w = fl32(q * d + m) (q4_1_pack.py:155-170, q4nx.py:105-126);
//     q*d is exact in f32 (4-bit x 8-bit significands), so one fma equals the
//     reference's multiply-then-add bit for bit.
//   scale_mode 1 (opt in): GGUF's fp16 d and m kept exactly in the scale word
//     (fp16 d << 16 | fp16 m), as the GGUF-direct pool keeps them (gguf_pool.py:1-17,
//     gemv_q4.h:54-65); then q*d has 4 + 11 significant bits, still exact in f32.
#include "q4mi_device.h"
#include "q4mi_internal.h"

using namespace q4mi;

namespace {

__device__ __forceinline__ void mx_write_block(uint8_t* packed, int64_t KB, int64_t n, int64_t kb,
                                               const uint8_t code[32], uint32_t scale_word) {
    const int64_t g = n >> 6;
    const int i = (int)(n & 63);
    const int r = i >> 4, i16 = i & 15;
    uint8_t* tile = packed + (g * KB + kb) * kTileBytes;
#pragma unroll
    for (int kg = 0; kg < 4; ++kg) {
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            w |= (uint32_t)code[8 * kg + e] << (16 * (e & 1) + 4 * (e >> 1));
        *(uint32_t*)(tile + (kg * 16 + i16) * 16 + r * 4) = w;
    }
    *(uint32_t*)(tile + kCodeBytes + i16 * 16 + r * 4) = scale_word;
}

__global__ __launch_bounds__(256) void repack_gguf_kernel(const uint8_t* __restrict__ src, int bw,
                                                          uint8_t* __restrict__ packed, int64_t N, int64_t KB,
                                                          int f16s) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= N * KB) return;
    // idx -> (tile, row): 64 consecutive threads fill one tile
    const int64_t tile = idx >> 6;
    const int64_t n = (tile / KB) * 64 + (idx & 63);
    const int64_t kb = tile % KB;
    const uint8_t* b = src + (n * KB + kb) * bw;
    uint32_t dbits = (uint32_t)b[0] | ((uint32_t)b[1] << 8), mbits;
    float d = f16_bits_to_f32(dbits), m;
    const uint8_t* qs;
    if (bw == 20) {
        mbits = (uint32_t)b[2] | ((uint32_t)b[3] << 8);
        m = f16_bits_to_f32(mbits);
        qs = b + 4;
    } else {
        m = -8.0f * d;   // Q4_0 written the Q4_1 way; exact
        mbits = 0;       // (scale_mode 1 takes Q4_1 blocks only)
        qs = b + 2;
    }
    uint8_t code[32];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        uint8_t v = qs[j];
        code[j] = v & 0xF;
        code[j + 16] = v >> 4;
    }
    const uint32_t word = f16s ? (dbits << 16) | mbits : (f32_to_bf16_rne(d) << 16) | f32_to_bf16_rne(m);
    mx_write_block(packed, KB, n, kb, code, word);
}

// f32_scales: the GGUF-direct pool's 6144 B chunks (open_kernels/gguf_pool/gguf_pool.py:
// 19-33: f32 d[256] @0, f32 m[256] @1024, codes @2048), narrowed to bf16 by RNE as that
// pool's kernel does in flight; else the 5120 B chunks, bytes carried over.
__global__ __launch_bounds__(256) void repack_pool_kernel(const uint8_t* __restrict__ pool, int rs, int f32_scales,
                                                          uint8_t* __restrict__ packed, int64_t N, int64_t KB) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= N * KB) return;
    const int64_t tile = idx >> 6;
    const int64_t n = (tile / KB) * 64 + (idx & 63);
    const int64_t kb = tile % KB;
    const int64_t K = KB * 32;
    const int64_t per_band = (int64_t)rs * K / 256;
    const int64_t band = n / (32 * rs);
    const int64_t ci = (kb / 8) * rs + (n % (32 * rs)) / 32;
    const int64_t chb = f32_scales ? 6144 : 5120;
    const uint8_t* ch = pool + (band * per_band + ci) * chb;
    const int r = (int)(n & 31);
    const int kbl = (int)(kb & 7);
    uint32_t d16, m16;
    if (f32_scales) {
        const float* sc = (const float*)ch;
        d16 = f32_to_bf16_rne(sc[kbl * 32 + r]);
        m16 = f32_to_bf16_rne(sc[256 + kbl * 32 + r]);
    } else {
        const uint16_t* sc = (const uint16_t*)ch;
        d16 = sc[kbl * 32 + r];
        m16 = sc[256 + kbl * 32 + r];
    }
    uint8_t code[32];
    const uint8_t* nib = ch + (chb - 4096) + (r >> 4) * 2048 + (r & 15) / 2;
    const int sh = 4 * (r & 1);
#pragma unroll
    for (int v = 0; v < 32; ++v) code[v] = (nib[(32 * kbl + v) * 8] >> sh) & 0xF;
    mx_write_block(packed, KB, n, kb, code, (d16 << 16) | m16);
}

// GGUF Q4_K super-blocks (256 values, 144 B: fp16 d | fp16 dmin | 12 B of packed 6-bit
// sub-block scales and mins | 128 B of codes) -> mx layout. Sub-block j (32 values) reads
// d sc_j q - dmin m_j (llama.cpp's dequantize_row_q4_K; restated in the reference's
// open_kernels/model/gguf_ref.py:224-250), i.e. a Q4_1 block with d' = d sc_j and
// m' = -dmin m_j. Both products are exact in f32 (11-bit x 6-bit significands); they are
// rounded to bf16 (RNE) as the reference's Q4_K transcode does (recipes/pack.py:266-310).
// Codes: chunk c = j / 2 holds 32 bytes; sub-block 2c takes the low nibbles, 2c+1 the high.
__global__ __launch_bounds__(256) void repack_q4k_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ packed,
                                                         int64_t N, int64_t KB) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= N * KB) return;
    const int64_t tile = idx >> 6;
    const int64_t n = (tile / KB) * 64 + (idx & 63);
    const int64_t kb = tile % KB;
    const uint8_t* b = src + (n * (KB / 8) + kb / 8) * 144;
    const int j = (int)(kb & 7);
    const float d = f16_bits_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    const float dmin = f16_bits_to_f32((uint32_t)b[2] | ((uint32_t)b[3] << 8));
    const uint8_t* sc = b + 4;
    int s6, m6;
    if (j < 4) {
        s6 = sc[j] & 63;
        m6 = sc[j + 4] & 63;
    } else {
        s6 = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4);
        m6 = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
    const float dd = d * (float)s6, mm = -(dmin * (float)m6);      // exact
    const uint8_t* qs = b + 16 + 32 * (j >> 1);
    const int sh = 4 * (j & 1);
    uint8_t code[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) code[e] = (qs[e] >> sh) & 0xF;
    mx_write_block(packed, KB, n, kb, code, (f32_to_bf16_rne(dd) << 16) | f32_to_bf16_rne(mm));
}

// The reference container's Q4_K chunks (4736 B, 32 rows x 256 K, in the pool's band
// order with row split rs) -> mx layout (recipes/pack.py:266-310). Chunk: uint8
// scales[8 g][32 r] @0, mins @256, codes @512 with row r of column k at byte
// 512 + 16 k + r/2 (even r low nibble), bf16 S[32 r] @4608, bf16 M[32 r] @4672 (negated).
// d = bf16_rne(S[r] * scales[g][r]), m = bf16_rne(M[r] * mins[g][r]); both f32 products
// are exact (8-bit x 8-bit significands), so the one rounding is the reference's.
__global__ __launch_bounds__(256) void repack_q4k_chunk_kernel(const uint8_t* __restrict__ chunks, int rs,
                                                               uint8_t* __restrict__ packed, int64_t N, int64_t KB) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= N * KB) return;
    const int64_t tile = idx >> 6;
    const int64_t n = (tile / KB) * 64 + (idx & 63);
    const int64_t kb = tile % KB;
    const int64_t K = KB * 32;
    const int64_t per_band = (int64_t)rs * K / 256;
    const int64_t band = n / (32 * rs);
    const int64_t ci = (kb / 8) * rs + (n % (32 * rs)) / 32;
    const uint8_t* ch = chunks + (band * per_band + ci) * 4736;
    const int r = (int)(n & 31);
    const int g = (int)(kb & 7);
    const float S = bf16_hi_to_f32(((uint32_t)ch[4608 + 2 * r] | ((uint32_t)ch[4609 + 2 * r] << 8)) << 16);
    const float M = bf16_hi_to_f32(((uint32_t)ch[4672 + 2 * r] | ((uint32_t)ch[4673 + 2 * r] << 8)) << 16);
    const float d = S * (float)ch[g * 32 + r], m = M * (float)ch[256 + g * 32 + r];   // exact
    const uint8_t* codes = ch + 512 + (32 * g) * 16 + (r >> 1);
    const int sh = 4 * (r & 1);
    uint8_t code[32];
#pragma unroll
    for (int v = 0; v < 32; ++v) code[v] = (codes[v * 16] >> sh) & 0xF;
    mx_write_block(packed, KB, n, kb, code, (f32_to_bf16_rne(d) << 16) | f32_to_bf16_rne(m));
}

// --- native Q4_K ("mxk", q4mi_device.h): the super-block's own integers, no collapse ---

// Row n's share of mxk tile (n / 64, sb): 8 sub-blocks of 32 codes, their (sc, mn) bytes
// and the f32 bases d, m.
__device__ __forceinline__ void mxk_write_row(uint8_t* packed, int64_t SB, int64_t n, int64_t sb,
                                              const uint8_t (&code)[8][32], const uint8_t (&sc)[8],
                                              const uint8_t (&mn)[8], float d, float m) {
    const int i = (int)(n & 63);
    const int r = i >> 4, i16 = i & 15;
    uint8_t* tile = packed + ((n >> 6) * SB + sb) * kKTileBytes;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
        for (int kg = 0; kg < 4; ++kg) {
            uint32_t w = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e) w |= (uint32_t)code[j][8 * kg + e] << (16 * (e & 1) + 4 * (e >> 1));
            *(uint32_t*)(tile + j * 1024 + (kg * 16 + i16) * 16 + r * 4) = w;
        }
        tile[kKScOff + i16 * 64 + r * 16 + j] = sc[j];
        tile[kKScOff + i16 * 64 + r * 16 + 8 + j] = mn[j];
    }
    *(float*)(tile + kKDOff + i16 * 16 + r * 4) = d;
    *(float*)(tile + kKMOff + i16 * 16 + r * 4) = m;
}

// GGUF Q4_K super-block (144 B: fp16 d | fp16 dmin | 12 B of packed 6-bit (sc, min) |
// 128 B of codes) -> mxk, one thread per (row, super-block): d = fp16 d, m = -fp16 dmin,
// (sc_j, mn_j) = llama.cpp's get_scale_min_k4 pairs; weight d sc q - dmin min exactly as
// the GGUF reader dequantizes it (src/gguf/gguf_file.cpp:611-635).
__global__ __launch_bounds__(256) void repack_mxk_gguf_kernel(const uint8_t* __restrict__ src,
                                                              uint8_t* __restrict__ packed, int64_t N, int64_t SB) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= N * SB) return;
    const int64_t tile = idx >> 6;
    const int64_t n = (tile / SB) * 64 + (idx & 63);
    const int64_t sb = tile % SB;
    const uint8_t* b = src + (n * SB + sb) * 144;
    const float d = f16_bits_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    const float dmin = f16_bits_to_f32((uint32_t)b[2] | ((uint32_t)b[3] << 8));
    const uint8_t* q6 = b + 4;
    uint8_t sc[8], mn[8], code[8][32];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if (j < 4) {
            sc[j] = q6[j] & 63;
            mn[j] = q6[j + 4] & 63;
        } else {
            sc[j] = (q6[j + 4] & 0xF) | ((q6[j - 4] >> 6) << 4);
            mn[j] = (q6[j + 4] >> 4) | ((q6[j] >> 6) << 4);
        }
        const uint8_t* qs = b + 16 + 32 * (j >> 1);
#pragma unroll
        for (int e = 0; e < 32; ++e) code[j][e] = (qs[e] >> (4 * (j & 1))) & 0xF;
    }
    mxk_write_row(packed, SB, n, sb, code, sc, mn, d, -dmin);
}

// The reference container's Q4_K chunks (4736 B, 32 rows x 256 K, band order with row
// split rs) -> mxk: d = bf16 S[r], m = bf16 M[r] (stored negated), (sc, mn) =
// (scales[g][r], mins[g][r]); weight S sc nib + M mn as the reference's Q4_K kernel reads
// the chunk (open_kernels/designs/gemm_q4/gemm_q4.h:456-507).
__global__ __launch_bounds__(256) void repack_mxk_chunk_kernel(const uint8_t* __restrict__ chunks, int rs,
                                                               uint8_t* __restrict__ packed, int64_t N, int64_t SB) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= N * SB) return;
    const int64_t tile = idx >> 6;
    const int64_t n = (tile / SB) * 64 + (idx & 63);
    const int64_t sb = tile % SB;
    const int64_t per_band = (int64_t)rs * SB;
    const uint8_t* ch = chunks + ((n / (32 * rs)) * per_band + sb * rs + (n % (32 * rs)) / 32) * 4736;
    const int r = (int)(n & 31);
    const float d = bf16_hi_to_f32(((uint32_t)ch[4608 + 2 * r] | ((uint32_t)ch[4609 + 2 * r] << 8)) << 16);
    const float m = bf16_hi_to_f32(((uint32_t)ch[4672 + 2 * r] | ((uint32_t)ch[4673 + 2 * r] << 8)) << 16);
    const int sh = 4 * (r & 1);
    uint8_t sc[8], mn[8], code[8][32];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        sc[j] = ch[j * 32 + r];
        mn[j] = ch[256 + j * 32 + r];
        const uint8_t* cb = ch + 512 + (32 * j) * 16 + (r >> 1);
#pragma unroll
        for (int e = 0; e < 32; ++e) code[j][e] = (cb[e * 16] >> sh) & 0xF;
    }
    mxk_write_row(packed, SB, n, sb, code, sc, mn, d, m);
}

// mxk -> f32: w = fl32(q * (d sc) + m mn); q (d sc) is exact, so one fma is the
// reference's multiply-then-add bit for bit. One thread per 8 consecutive k of a row.
__global__ __launch_bounds__(256) void dequant_mxk_kernel(const uint8_t* __restrict__ packed, float* __restrict__ w,
                                                          int64_t N, int64_t K) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t K8 = K >> 3;
    if (idx >= N * K8) return;
    const int64_t n = idx / K8, k8 = idx % K8;
    const int64_t kb = k8 >> 2, sb = kb >> 3;
    const int j = (int)(kb & 7), kg = (int)(k8 & 3);
    const int i = (int)(n & 63), r = i >> 4, i16 = i & 15;
    const uint8_t* tile = packed + ((n >> 6) * (K >> 8) + sb) * kKTileBytes;
    const uint32_t c = *(const uint32_t*)(tile + j * 1024 + (kg * 16 + i16) * 16 + r * 4);
    const uint8_t* sm = tile + kKScOff + i16 * 64 + r * 16;
    const float D = *(const float*)(tile + kKDOff + i16 * 16 + r * 4) * (float)sm[j];
    const float M = *(const float*)(tile + kKMOff + i16 * 16 + r * 4) * (float)sm[8 + j];
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = __builtin_fmaf((float)((c >> (16 * (e & 1) + 4 * (e >> 1))) & 0xF), D, M);
    f32x4* dst = (f32x4*)(w + n * K + k8 * 8);
    dst[0] = f32x4{o[0], o[1], o[2], o[3]};
    dst[1] = f32x4{o[4], o[5], o[6], o[7]};
}

// Chunk of row n, 32-K block kb in the pool's band order with row split rs (q4_1_pack.py:
// 112-121; rs = 1 is the .q4nx file's raster, chunk = (n / 32) * K / 256 + kb / 8).
__device__ __forceinline__ int64_t band_chunk(int64_t n, int64_t kb, int rs, int64_t K) {
    const int64_t per_band = (int64_t)rs * K / 256;
    return (n / (32 * rs)) * per_band + (kb / 8) * rs + (n % (32 * rs)) / 32;
}

// 5120 B chunks of the SIGNED quantiser (w = d * int4(q), every min stored as 0) -> mx
// layout read the q4_1 way: int4(q) = (q ^ 8) - 8, so the code is q ^ 8 and m = -8 d,
// both exact (recipes/pack.py:606-622).
__global__ __launch_bounds__(256) void repack_pool_signed_kernel(const uint8_t* __restrict__ pool, int rs,
                                                                 uint8_t* __restrict__ packed, int64_t N,
                                                                 int64_t KB) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= N * KB) return;
    const int64_t tile = idx >> 6;
    const int64_t n = (tile / KB) * 64 + (idx & 63);
    const int64_t kb = tile % KB;
    const uint8_t* ch = pool + band_chunk(n, kb, rs, KB * 32) * 5120;
    const int r = (int)(n & 31), kbl = (int)(kb & 7);
    const uint32_t d16 = ((const uint16_t*)ch)[kbl * 32 + r];
    const float d = bf16_hi_to_f32(d16 << 16);
    const uint32_t m16 = f32_to_bf16_rne(-8.0f * d);
    uint8_t code[32];
    const uint8_t* nib = ch + 1024 + (r >> 4) * 2048 + (r & 15) / 2;
    const int sh = 4 * (r & 1);
#pragma unroll
    for (int v = 0; v < 32; ++v) code[v] = ((nib[(32 * kbl + v) * 8] >> sh) & 0xF) ^ 0x8;
    mx_write_block(packed, KB, n, kb, code, (d16 << 16) | m16);
}

__device__ __forceinline__ uint32_t bf16_floor_bits(float x) {          // toward -inf
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    return (u >> 31) ? (u + 0xFFFFu) >> 16 : u >> 16;
}
__device__ __forceinline__ uint32_t bf16_ceil_bits(float x) {           // toward +inf
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    return (u >> 31) ? u >> 16 : (u + 0xFFFFu) >> 16;
}

// 8704 B q8 chunks (bf16 scales[256] @0 index kb*32 + r; int8 codes @512, code (r, kb,
// i) at (r/16)*4096 + kb*512 + i*16 + r%16) re-quantised to q4_1 block for block, the
// reference's requant_q4_1 (recipes/pack.py:224-263) step for step in f32 with every
// operation rounded on its own (no fused multiply-add): v = code * scale (exact); m = the
// block minimum rounded down to bf16; d = (max - m) / 15 rounded up to bf16, so
// [m, m + 15 d] covers the block; nibble = clamp(trunc((v - m) * (1 / d) + 0.5), 0, 15).
// The block's min and max are scanned as the reference's C++ does (pools.cpp:591-601):
// start at lane 0 and replace only on a strict < or >, so the first lane holding the
// extreme keeps its sign (a leading -0, a negative code under a zero scale, gives m = -0).
__global__ __launch_bounds__(256) void repack_q8_chunk_kernel(const uint8_t* __restrict__ chunks, int rs,
                                                              uint8_t* __restrict__ packed, int64_t N,
                                                              int64_t KB) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= N * KB) return;
    const int64_t tile = idx >> 6;
    const int64_t n = (tile / KB) * 64 + (idx & 63);
    const int64_t kb = tile % KB;
    const uint8_t* ch = chunks + band_chunk(n, kb, rs, KB * 32) * 8704;
    const int r = (int)(n & 31), kbl = (int)(kb & 7);
    const float sc = bf16_hi_to_f32((uint32_t)((const uint16_t*)ch)[kbl * 32 + r] << 16);
    const int8_t* cp = (const int8_t*)(ch + 512 + (r >> 4) * 4096 + kbl * 512 + (r & 15));
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = __fmul_rn((float)cp[i * 16], sc);
    float mn = v[0], mx = v[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) {
        mn = v[i] < mn ? v[i] : mn;
        mx = v[i] > mx ? v[i] : mx;
    }
    const uint32_t m_u = bf16_floor_bits(mn);
    const float m = bf16_hi_to_f32(m_u << 16);
    const uint32_t d_u = bf16_ceil_bits(__fdiv_rn(__fsub_rn(mx, m), 15.0f));
    const float d = bf16_hi_to_f32(d_u << 16);
    const float inv = d > 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint8_t code[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const float t = __fadd_rn(__fmul_rn(__fsub_rn(v[i], m), inv), 0.5f);
        const int q = (int)t;
        code[i] = (uint8_t)(q < 0 ? 0 : (q > 15 ? 15 : q));
    }
    mx_write_block(packed, KB, n, kb, code, (d_u << 16) | m_u);
}

// q8 weights as the exact sum of two q4_1 matrices (recipes/pack.py:94-117,
// split_q8_q4_1): with q = 16 (q >> 4) + (q & 15) for a signed byte q,
//   part 0 "hi": d = 16 s, m = -128 s, code (q >> 4) + 8  -> reads 16 s (q >> 4)
//   part 1 "lo": d = s,    m = 0,      code q & 15        -> reads s (q & 15)
// and hi + lo = s q exactly (16 s and -128 s only move a bf16 exponent). Sources:
// 8704 B q8 chunks (src_format 0, band order rs; s the chunk's bf16 scale), GGUF Q8_0
// blocks (src_format 1: fp16 d then 32 int8, 34 B per 32 K; s = RNE_bf16(d), the same
// narrowing the Q4_1 blocks get) or the GGUF-direct pool's 9216 B q8 chunks (src_format
// 2: f32 scales[256] @0, codes @1024; s = RNE_bf16(scale); gguf_pool.py:28-33).
// One q8 block (row n, 32-K block kb) of any of the three sources: its bf16 scale bits
// and its 32 signed codes.
__device__ __forceinline__ void q8_source_block(const uint8_t* __restrict__ src, int src_format, int rs, int64_t n,
                                                int64_t kb, int64_t KB, uint32_t& s16, int8_t (&q)[32]) {
    if (src_format != 1) {
        const bool f32s = src_format == 2;
        const uint8_t* ch = src + band_chunk(n, kb, rs, KB * 32) * (f32s ? 9216 : 8704);
        const int r = (int)(n & 31), kbl = (int)(kb & 7);
        s16 = f32s ? f32_to_bf16_rne(((const float*)ch)[kbl * 32 + r]) : ((const uint16_t*)ch)[kbl * 32 + r];
        const int8_t* cp = (const int8_t*)(ch + (f32s ? 1024 : 512) + (r >> 4) * 4096 + kbl * 512 + (r & 15));
#pragma unroll
        for (int i = 0; i < 32; ++i) q[i] = cp[i * 16];
    } else {
        const uint8_t* b = src + (n * KB + kb) * 34;
        s16 = f32_to_bf16_rne(f16_bits_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8)));
#pragma unroll
        for (int i = 0; i < 32; ++i) q[i] = (int8_t)b[2 + i];
    }
}

__global__ __launch_bounds__(256) void repack_q8_split_kernel(const uint8_t* __restrict__ src, int src_format,
                                                              int rs, int part, uint8_t* __restrict__ packed,
                                                              int64_t N, int64_t KB) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= N * KB) return;
    const int64_t tile = idx >> 6;
    const int64_t n = (tile / KB) * 64 + (idx & 63);
    const int64_t kb = tile % KB;
    uint32_t s16;
    int8_t q[32];
    q8_source_block(src, src_format, rs, n, kb, KB, s16, q);
    const float sv = bf16_hi_to_f32(s16 << 16);
    uint8_t code[32];
    uint32_t word;
    if (part == 0) {
#pragma unroll
        for (int i = 0; i < 32; ++i) code[i] = (uint8_t)((q[i] >> 4) + 8);
        word = (f32_to_bf16_rne(16.0f * sv) << 16) | f32_to_bf16_rne(-128.0f * sv);
    } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) code[i] = (uint8_t)(q[i] & 15);
        word = s16 << 16;
    }
    mx_write_block(packed, KB, n, kb, code, word);
}

// The same q8 sources -> the native q8 layout (q4mi_device.h), one thread per (row, 32-K
// block): codes as b = q + 128, bytes of each dword in the order (k0, k2, k1, k3), and
// the bf16 scale as the split planes take it.
__global__ __launch_bounds__(256) void repack_mx8_kernel(const uint8_t* __restrict__ src, int src_format, int rs,
                                                         uint8_t* __restrict__ packed, int64_t N, int64_t KB) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= N * KB) return;
    const int64_t tile = idx >> 6;
    const int64_t n = (tile / KB) * 64 + (idx & 63);
    const int64_t kb = tile % KB;
    uint32_t s16;
    int8_t q[32];
    q8_source_block(src, src_format, rs, n, kb, KB, s16, q);
    const int i = (int)(n & 63), r = i >> 4, i16 = i & 15;
    uint8_t* t = packed + ((n >> 6) * KB + kb) * kQ8TileBytes;
#pragma unroll
    for (int kg = 0; kg < 4; ++kg)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k0 = 8 * kg + 4 * h;
            const uint32_t b0 = (uint8_t)q[k0] ^ 0x80u, b1 = (uint8_t)q[k0 + 1] ^ 0x80u;
            const uint32_t b2 = (uint8_t)q[k0 + 2] ^ 0x80u, b3 = (uint8_t)q[k0 + 3] ^ 0x80u;
            *(uint32_t*)(t + (r >> 1) * 1024 + (kg * 16 + i16) * 16 + (r & 1) * 8 + h * 4) =
                b0 | (b2 << 8) | (b1 << 16) | (b3 << 24);
        }
    *(uint16_t*)(t + kQ8ScaleOff + i16 * 8 + r * 2) = (uint16_t)s16;
}

// mx8 -> f32, w = s * q (exact). One thread per 8 consecutive k of a row.
__global__ __launch_bounds__(256) void dequant_mx8_kernel(const uint8_t* __restrict__ packed, float* __restrict__ w,
                                                          int64_t N, int64_t K) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t K8 = K >> 3;
    if (idx >= N * K8) return;
    const int64_t n = idx / K8, k8 = idx % K8;
    const int64_t kb = k8 >> 2;
    const int kg = (int)(k8 & 3), i = (int)(n & 63), r = i >> 4, i16 = i & 15;
    const uint8_t* t = packed + ((n >> 6) * (K >> 5) + kb) * kQ8TileBytes;
    const u32x2 c = *(const u32x2*)(t + (r >> 1) * 1024 + (kg * 16 + i16) * 16 + (r & 1) * 8);
    const float s = bf16_hi_to_f32((uint32_t)*(const uint16_t*)(t + kQ8ScaleOff + i16 * 8 + r * 2) << 16);
    float o[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t d = c[h];
        const int kx[4] = {0, 2, 1, 3};           // byte j holds k = kx[j]
#pragma unroll
        for (int j = 0; j < 4; ++j) o[4 * h + kx[j]] = s * (float)((int)((d >> (8 * j)) & 0xFF) - 128);
    }
    f32x4* dst = (f32x4*)(w + n * K + k8 * 8);
    dst[0] = f32x4{o[0], o[1], o[2], o[3]};
    dst[1] = f32x4{o[4], o[5], o[6], o[7]};
}

// Q4_0 -> mx0 (no m plane). Thread per (row n, 32-K block kb). src_format 0: GGUF Q4_0
// blocks (18 B: fp16 d | 16 code bytes, row-major [N][K/32]), d narrowed to bf16 by RNE as
// q4_1_pack.py:129-130 narrows it; 1: the reference's 4608 B Q4_0-native chunks in pool
// order with row split rs (q4_1_pack.py:145-152: the 5120 B chunk's d plane at 0, its codes
// at 512), bytes carried over.
__global__ __launch_bounds__(256) void repack_q40_kernel(const uint8_t* __restrict__ src, int src_format, int rs,
                                                         uint8_t* __restrict__ packed, int64_t N, int64_t KB) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= N * KB) return;
    const int64_t tile = idx >> 6;
    const int64_t n = (tile / KB) * 64 + (idx & 63);
    const int64_t kb = tile % KB;
    uint8_t code[32];
    uint32_t d16;
    if (src_format == 0) {
        const uint8_t* b = src + (n * KB + kb) * 18;
        d16 = f32_to_bf16_rne(f16_bits_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8)));
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            code[j] = b[2 + j] & 0xF;
            code[j + 16] = b[2 + j] >> 4;
        }
    } else {
        const int64_t per_band = (int64_t)rs * KB / 8;
        const int64_t band = n / (32 * rs);
        const int64_t ci = (kb / 8) * rs + (n % (32 * rs)) / 32;
        const uint8_t* ch = src + (band * per_band + ci) * 4608;
        const int r = (int)(n & 31), kbl = (int)(kb & 7);
        d16 = ((const uint16_t*)ch)[kbl * 32 + r];
        const uint8_t* nib = ch + 512 + (r >> 4) * 2048 + (r & 15) / 2;
        const int sh = 4 * (r & 1);
#pragma unroll
        for (int v = 0; v < 32; ++v) code[v] = (nib[(32 * kbl + v) * 8] >> sh) & 0xF;
    }
    const int i = (int)(n & 63), r = i >> 4, i16 = i & 15;
    uint8_t* t = packed + ((n >> 6) * KB + kb) * kQ0TileBytes;
#pragma unroll
    for (int kg = 0; kg < 4; ++kg) {
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            w |= (uint32_t)code[8 * kg + e] << (16 * (e & 1) + 4 * (e >> 1));
        *(uint32_t*)(t + (kg * 16 + i16) * 16 + r * 4) = w;
    }
    *(uint16_t*)(t + kCodeBytes + i16 * 8 + r * 2) = (uint16_t)d16;
}

// mx0 -> f32 [N][K]: fl32(q d + m), m = -8 d. Thread per (row n, 8-wide k group).
__global__ __launch_bounds__(256) void dequant_mx0_kernel(const uint8_t* __restrict__ packed, float* __restrict__ w,
                                                          int64_t N, int64_t K) {
    const int64_t K8 = K >> 3;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= N * K8) return;
    const int64_t n = idx / K8, k8 = idx % K8;
    const int64_t KB = K >> 5;
    const int64_t g = n >> 6, kb = k8 >> 2;
    const int i = (int)(n & 63), r = i >> 4, i16 = i & 15, kg = (int)(k8 & 3);
    const uint8_t* tile = packed + (g * KB + kb) * kQ0TileBytes;
    const uint32_t c = *(const uint32_t*)(tile + (kg * 16 + i16) * 16 + r * 4);
    const float d = bf16_hi_to_f32((uint32_t)*(const uint16_t*)(tile + kCodeBytes + i16 * 8 + r * 2) << 16);
    const float m = -8.0f * d;
    f32x4 lo, hi;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        lo[e] = __builtin_fmaf((float)((c >> (16 * (e & 1) + 4 * (e >> 1))) & 0xF), d, m);
        hi[e] = __builtin_fmaf((float)((c >> (16 * ((e + 4) & 1) + 4 * ((e + 4) >> 1))) & 0xF), d, m);
    }
    f32x4* out = (f32x4*)(w + n * K + k8 * 8);
    out[0] = lo;
    out[1] = hi;
}

// Thread per (row n, 8-wide k group): one codes dword + one scale word -> 8 floats. F16S: the
// scale word holds fp16 d and m (scale_mode 1).
template <bool F16S>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ packed, float* __restrict__ w,
                                                      int64_t N, int64_t K) {
    const int64_t K8 = K >> 3;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= N * K8) return;
    const int64_t n = idx / K8, k8 = idx % K8;
    const int64_t KB = K >> 5;
    const int64_t g = n >> 6, kb = k8 >> 2;
    const int i = (int)(n & 63), r = i >> 4, i16 = i & 15, kg = (int)(k8 & 3);
    const uint8_t* tile = packed + (g * KB + kb) * kTileBytes;
    const uint32_t c = *(const uint32_t*)(tile + (kg * 16 + i16) * 16 + r * 4);
    const uint32_t s = *(const uint32_t*)(tile + kCodeBytes + i16 * 16 + r * 4);
    const float d = scale_d<F16S>(s), m = scale_m<F16S>(s);
    f32x4 lo, hi;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        lo[e] = __builtin_fmaf((float)((c >> (16 * (e & 1) + 4 * (e >> 1))) & 0xF), d, m);
        hi[e] = __builtin_fmaf((float)((c >> (16 * ((e + 4) & 1) + 4 * ((e + 4) >> 1))) & 0xF), d, m);
    }
    f32x4* out = (f32x4*)(w + n * K + k8 * 8);
    out[0] = lo;
    out[1] = hi;
}

}  // namespace

extern "C" int64_t q4_packed_bytes(int64_t N, int64_t K) {
    if (N == 0 && K > 0 && K % 32 == 0) return 0;
    if (N <= 0 || K <= 0 || N % 64 || K % 32) return Q4MI_E_SHAPE;
    return (N / 64) * (K / 32) * (int64_t)kTileBytes;
}

extern "C" int q4_repack(const uint8_t* gguf_blocks, int block_bytes, uint8_t* packed, int64_t N, int64_t K,
                         int scale_mode, void* stream) {
    if (block_bytes != 20 && block_bytes != 18) return Q4MI_E_ARG;
    if (scale_mode != 0 && scale_mode != 1) return Q4MI_E_ARG;
    if (scale_mode == 1 && block_bytes != 20) return Q4MI_E_ARG;   // Q4_0 has its exact mx0 layout
    if (N == 0 && K > 0 && K % 32 == 0) return Q4MI_OK;   // empty: nothing to touch
    if (!gguf_blocks || !packed) return Q4MI_E_ARG;
    if (misaligned16(packed)) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || N % 64 || K % 32) return Q4MI_E_SHAPE;
    const int64_t KB = K / 32, total = N * KB;
    const unsigned grid = (unsigned)((total + 255) / 256);
    hipLaunchKernelGGL(repack_gguf_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, gguf_blocks,
                       block_bytes, packed, N, KB, scale_mode);
    return launch_status();
}

extern "C" int q4_repack_pool(const uint8_t* pool, int rs, uint8_t* packed, int64_t N, int64_t K, void* stream) {
    if (rs <= 0) return Q4MI_E_ARG;
    if (N == 0 && K > 0 && K % 256 == 0) return Q4MI_OK;
    if (!pool || !packed) return Q4MI_E_ARG;
    if (misaligned16(packed)) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || K % 256 || N % 64 || N % (32 * rs)) return Q4MI_E_SHAPE;
    const int64_t KB = K / 32, total = N * KB;
    const unsigned grid = (unsigned)((total + 255) / 256);
    hipLaunchKernelGGL(repack_pool_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, pool, rs, 0, packed, N, KB);
    return launch_status();
}

extern "C" int q4_repack_pool_f32(const uint8_t* pool, int rs, uint8_t* packed, int64_t N, int64_t K, void* stream) {
    if (rs <= 0) return Q4MI_E_ARG;
    if (N == 0 && K > 0 && K % 256 == 0) return Q4MI_OK;
    if (!pool || !packed) return Q4MI_E_ARG;
    if (misaligned16(packed) || ((uintptr_t)pool & 3)) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || K % 256 || N % 64 || N % (32 * rs)) return Q4MI_E_SHAPE;
    const int64_t KB = K / 32, total = N * KB;
    hipLaunchKernelGGL(repack_pool_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       pool, rs, 1, packed, N, KB);
    return launch_status();
}

static int dequant_impl(const uint8_t* packed, float* w, int64_t N, int64_t K, void* stream, bool f16s) {
    if (N == 0 && K > 0 && K % 32 == 0) return Q4MI_OK;
    if (!packed || !w) return Q4MI_E_ARG;
    if (misaligned16(packed) || misaligned16(w)) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || N % 64 || K % 32) return Q4MI_E_SHAPE;
    const int64_t total = N * (K / 8);
    const unsigned grid = (unsigned)((total + 255) / 256);
    if (f16s)
        hipLaunchKernelGGL(dequant_kernel<true>, dim3(grid), dim3(256), 0, (hipStream_t)stream, packed, w, N, K);
    else
        hipLaunchKernelGGL(dequant_kernel<false>, dim3(grid), dim3(256), 0, (hipStream_t)stream, packed, w, N, K);
    return launch_status();
}

extern "C" int q4_dequant(const uint8_t* packed, float* w, int64_t N, int64_t K, void* stream) {
    return dequant_impl(packed, w, N, K, stream, false);
}

extern "C" int q4_dequant_fp16s(const uint8_t* packed, float* w, int64_t N, int64_t K, void* stream) {
    return dequant_impl(packed, w, N, K, stream, true);
}

extern "C" int q4_repack_q4k(const uint8_t* q4k_blocks, uint8_t* packed, int64_t N, int64_t K, void* stream) {
    if (N == 0 && K > 0 && K % 256 == 0) return Q4MI_OK;
    if (!q4k_blocks || !packed) return Q4MI_E_ARG;
    if (misaligned16(packed)) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || N % 64 || K % 256) return Q4MI_E_SHAPE;
    const int64_t KB = K / 32, total = N * KB;
    hipLaunchKernelGGL(repack_q4k_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       q4k_blocks, packed, N, KB);
    return launch_status();
}

extern "C" int q4_repack_q4k_chunks(const uint8_t* chunks, int rs, uint8_t* packed, int64_t N, int64_t K,
                                    void* stream) {
    if (rs <= 0) return Q4MI_E_ARG;
    if (N == 0 && K > 0 && K % 256 == 0) return Q4MI_OK;
    if (!chunks || !packed) return Q4MI_E_ARG;
    if (misaligned16(packed)) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || K % 256 || N % 64 || N % (32 * rs)) return Q4MI_E_SHAPE;
    const int64_t KB = K / 32, total = N * KB;
    hipLaunchKernelGGL(repack_q4k_chunk_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, chunks, rs, packed, N, KB);
    return launch_status();
}

extern "C" int q4_repack_pool_signed(const uint8_t* pool, int rs, uint8_t* packed, int64_t N, int64_t K,
                                     void* stream) {
    if (rs <= 0) return Q4MI_E_ARG;
    if (N == 0 && K > 0 && K % 256 == 0) return Q4MI_OK;
    if (!pool || !packed) return Q4MI_E_ARG;
    if (misaligned16(packed)) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || K % 256 || N % 64 || N % (32 * rs)) return Q4MI_E_SHAPE;
    const int64_t KB = K / 32, total = N * KB;
    hipLaunchKernelGGL(repack_pool_signed_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, pool, rs, packed, N, KB);
    return launch_status();
}

extern "C" int q4_repack_q8_chunks(const uint8_t* chunks, int rs, uint8_t* packed, int64_t N, int64_t K,
                                   void* stream) {
    if (rs <= 0) return Q4MI_E_ARG;
    if (N == 0 && K > 0 && K % 256 == 0) return Q4MI_OK;
    if (!chunks || !packed) return Q4MI_E_ARG;
    if (misaligned16(packed)) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || K % 256 || N % 64 || N % (32 * rs)) return Q4MI_E_SHAPE;
    const int64_t KB = K / 32, total = N * KB;
    hipLaunchKernelGGL(repack_q8_chunk_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, chunks, rs, packed, N, KB);
    return launch_status();
}

extern "C" int q4_repack_q8_split(const uint8_t* src, int src_format, int rs, int part, uint8_t* packed, int64_t N,
                                  int64_t K, void* stream) {
    if (src_format < 0 || src_format > 2 || (part != 0 && part != 1) || rs <= 0) return Q4MI_E_ARG;
    const int64_t kq = src_format == 1 ? 32 : 256;
    if (N == 0 && K > 0 && K % kq == 0) return Q4MI_OK;
    if (!src || !packed) return Q4MI_E_ARG;
    if (misaligned16(packed)) return Q4MI_E_ARG;
    if (src_format == 2 && ((uintptr_t)src & 3)) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || K % kq || N % 64 || (src_format != 1 && N % (32 * rs))) return Q4MI_E_SHAPE;
    const int64_t KB = K / 32, total = N * KB;
    hipLaunchKernelGGL(repack_q8_split_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, src, src_format, rs, part, packed, N, KB);
    return launch_status();
}

extern "C" int64_t q4_q4k_packed_bytes(int64_t N, int64_t K) {
    if (N < 0 || K <= 0 || N % 64 || K % 256) return -1;
    return (N / 64) * (K / 256) * (int64_t)kKTileBytes;
}

extern "C" int q4_repack_q4k_native(const uint8_t* q4k_blocks, uint8_t* packed, int64_t N, int64_t K, void* stream) {
    if (N == 0 && K > 0 && K % 256 == 0) return Q4MI_OK;
    if (!q4k_blocks || !packed) return Q4MI_E_ARG;
    if (misaligned16(packed)) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || N % 64 || K % 256) return Q4MI_E_SHAPE;
    const int64_t SB = K / 256, total = N * SB;
    hipLaunchKernelGGL(repack_mxk_gguf_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, q4k_blocks, packed, N, SB);
    return launch_status();
}

extern "C" int q4_repack_q4k_chunks_native(const uint8_t* chunks, int rs, uint8_t* packed, int64_t N, int64_t K,
                                           void* stream) {
    if (rs <= 0) return Q4MI_E_ARG;
    if (N == 0 && K > 0 && K % 256 == 0) return Q4MI_OK;
    if (!chunks || !packed) return Q4MI_E_ARG;
    if (misaligned16(packed)) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || K % 256 || N % 64 || N % (32 * rs)) return Q4MI_E_SHAPE;
    const int64_t SB = K / 256, total = N * SB;
    hipLaunchKernelGGL(repack_mxk_chunk_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, chunks, rs, packed, N, SB);
    return launch_status();
}

extern "C" int q4_dequant_q4k(const uint8_t* packed, float* w, int64_t N, int64_t K, void* stream) {
    if (N == 0 && K > 0 && K % 256 == 0) return Q4MI_OK;
    if (!packed || !w) return Q4MI_E_ARG;
    if (misaligned16(packed) || misaligned16(w)) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || N % 64 || K % 256) return Q4MI_E_SHAPE;
    const int64_t total = N * (K / 8);
    hipLaunchKernelGGL(dequant_mxk_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       packed, w, N, K);
    return launch_status();
}

extern "C" int64_t q4_q8_native_packed_bytes(int64_t N, int64_t K) {
    if (N < 0 || K <= 0 || N % 64 || K % 32) return -1;
    return (N / 64) * (K / 32) * (int64_t)kQ8TileBytes;
}

extern "C" int q4_repack_q8_native(const uint8_t* src, int src_format, int rs, uint8_t* packed, int64_t N, int64_t K,
                                   void* stream) {
    if (src_format < 0 || src_format > 2 || rs <= 0) return Q4MI_E_ARG;
    const int64_t kmod = src_format == 1 ? 32 : 256;
    if (N == 0 && K > 0 && K % kmod == 0) return Q4MI_OK;
    if (!src || !packed) return Q4MI_E_ARG;
    if (misaligned16(packed) || (src_format == 2 && ((uintptr_t)src & 3))) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || N % 64 || K % kmod || (src_format != 1 && N % (32 * rs))) return Q4MI_E_SHAPE;
    const int64_t KB = K / 32, total = N * KB;
    hipLaunchKernelGGL(repack_mx8_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       src, src_format, rs, packed, N, KB);
    return launch_status();
}

extern "C" int q4_dequant_q8_native(const uint8_t* packed, float* w, int64_t N, int64_t K, void* stream) {
    if (N == 0 && K > 0 && K % 32 == 0) return Q4MI_OK;
    if (!packed || !w) return Q4MI_E_ARG;
    if (misaligned16(packed) || misaligned16(w)) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || N % 64 || K % 32) return Q4MI_E_SHAPE;
    const int64_t total = N * (K / 8);
    hipLaunchKernelGGL(dequant_mx8_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       packed, w, N, K);
    return launch_status();
}

extern "C" int64_t q4_q40_packed_bytes(int64_t N, int64_t K) {
    if (N == 0 && K > 0 && K % 32 == 0) return 0;
    if (N <= 0 || K <= 0 || N % 64 || K % 32) return Q4MI_E_SHAPE;
    return (N / 64) * (K / 32) * (int64_t)kQ0TileBytes;
}

extern "C" int q4_repack_q40(const uint8_t* src, int src_format, int rs, uint8_t* packed, int64_t N, int64_t K,
                             void* stream) {
    if (src_format != 0 && src_format != 1) return Q4MI_E_ARG;
    if (src_format == 1 && rs <= 0) return Q4MI_E_ARG;
    const int64_t kmul = src_format == 1 ? 256 : 32;
    if (N == 0 && K > 0 && K % kmul == 0) return Q4MI_OK;
    if (!src || !packed) return Q4MI_E_ARG;
    if (misaligned16(packed)) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || N % 64 || K % kmul) return Q4MI_E_SHAPE;
    if (src_format == 1 && (N % (32 * rs) || ((uintptr_t)src & 1))) return N % (32 * rs) ? Q4MI_E_SHAPE : Q4MI_E_ARG;
    const int64_t KB = K / 32, total = N * KB;
    hipLaunchKernelGGL(repack_q40_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       src, src_format, rs, packed, N, KB);
    return launch_status();
}

extern "C" int q4_dequant_q40(const uint8_t* packed, float* w, int64_t N, int64_t K, void* stream) {
    if (N == 0 && K > 0 && K % 32 == 0) return Q4MI_OK;
    if (!packed || !w) return Q4MI_E_ARG;
    if (misaligned16(packed) || misaligned16(w)) return Q4MI_E_ARG;
    if (N < 0 || K <= 0 || N % 64 || K % 32) return Q4MI_E_SHAPE;
    const int64_t total = N * (K / 8);
    hipLaunchKernelGGL(dequant_mx0_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       packed, w, N, K);
    return launch_status();
}
