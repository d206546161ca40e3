// gemv_core.h -- the decode GEMV inner loop on the mx layout, shared by the
// dense GEMV (gemv.hip) and the routed-expert kernels (moe.hip).
//
// A 256-thread workgroup works on one 64-row group; its four waves take every
// fourth 32-K tile of a K range. Per tile (64 rows x 32 K, 1280 B) a wave
// issues two 128-bit loads per lane (codes, scales) and the activation
// fragment, then:
//   ns  = MFMA(X, -128)             -> -128 * sum_k x, per token (the C input)
//   P_r = MFMA(X, 128 + q_r, ns)    -> sum_k q x, rows 16r..16r+15
//   acc_r += d_r * P_r + m_r * sum_k x
// which is the Q4_1 factorisation the reference GEMV uses,
//   y[r] = sum_kb { d[kb][r] * sum_k q x + m[kb][r] * sum_k x }
// (open_kernels/designs/gemv_q4/gemv_q4.h:33-34), here with the exact 4-bit
// codes and bf16 activations on the bf16 MFMA and the scales applied in fp32.
// The MFMA's A operand is the activation (tokens as rows), so each lane's
// outputs are tokens of one weight row: one d and one m per lane per row
// tile. MFMA row r carries token slot (r % 4) * 4 + r / 4, so the lane of
// k-group kg holds tokens kg, kg + 4, kg + 8, kg + 12 in its outputs j = 0..3
// and M tokens need only NTL = ceil(M / 4) accumulators per row (M <= 4: one,
// as for a single token). f32 activations are split x = hi + lo (two bf16s,
// |residual| <= 2^-18 |x|) and both halves go through the MFMA.
//
// gemv_rows_multi streams several row groups per K position with compiler-tracked
// loads; gemv_rows_pipe is the same arithmetic as a rolling pipeline of inline-asm loads
// with explicit waits, so a wave always has UNR K positions in flight (the routed-expert
// kernels, whose workgroups stream short row-group spans and gain most from it).
#pragma once

#include <type_traits>

#include "norm_core.h"
#include "q4mi_device.h"

namespace q4mi {

constexpr int kWaves = 4;      // waves per workgroup
constexpr int kUnroll = 4;     // tiles in flight per wave


// MFMA row r (A operand row, output row) <-> token slot: rows 4 kg + j hold
// token j * 4 + kg, so a lane's j-th output is token token_of(kg, j).
__device__ __forceinline__ int token_of_row(int r) { return (r & 3) * 4 + (r >> 2); }
__device__ __forceinline__ int token_of(int kg, int j) { return j * 4 + kg; }

// Token slot -> activation row. Slots at or past M map to the last real
// token: MFMA rows (tokens) are independent and those rows of the result are
// never stored, so no lane needs a branch or a zero fill.
struct DenseRows {
    int M;
    __device__ __forceinline__ int64_t operator()(int tok) const { return tok < M ? tok : M - 1; }
};
struct GatherRows {            // rows listed in LDS (routed tokens of one expert)
    const int* rows;
    int M;
    __device__ __forceinline__ int64_t operator()(int tok) const { return rows[tok < M ? tok : M - 1]; }
};

// Activation fragment of one tile: the 8 x of activation row `row` at k0.
template <bool XF32>
__device__ __forceinline__ void load_xfrag(const void* __restrict__ x, int64_t K, int64_t row, int64_t k0,
                                           bf16x8& hi, bf16x8& lo) {
    if constexpr (XF32) {
        const float* p = (const float*)x + row * K + k0;
        const f32x4 a = load_global<f32x4>(p), b = load_global<f32x4>(p + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const __bf16 ha = (__bf16)a[e], hb = (__bf16)b[e];
            hi[e] = ha;
            hi[e + 4] = hb;
            lo[e] = (__bf16)(a[e] - (float)ha);
            lo[e + 4] = (__bf16)(b[e] - (float)hb);
        }
    } else {
        hi = load_global<bf16x8>((const __bf16*)x + row * K + k0);
    }
}

// Accumulate this wave's share of tiles [kb0, kb1) of row group g: with WAVES waves in
// the workgroup, wave w takes tiles kb0 + w, kb0 + w + WAVES, ...
// Loads are unconditional (a tile index past kb1 is clamped to kb1 - 1 and
// its data skipped) so the compiler can count them statically and wait for
// each tile's loads only, keeping kUnroll tiles in flight per wave.
// The activation row normalised in the GEMV (RMSNorm, norm_core.h): x is the f32 residual
// stream, w the norm weight (bf16 or f32), r the rows' 1/rms (LDS, per activation row).
struct NormIn {
    const void* w;
    int w_bf16;
    const float* r;
};

// Q40: the mx0 layout (1152 B tiles, bf16 d only; m = -8 d), else the mx layout.
// NORM: x is f32 and normalised on the fly (nrm), rounded to bf16 as q4_rmsnorm_add rounds it.
template <int NTL, bool XF32, class Rows, int WAVES = kWaves, bool Q40 = false, bool NORM = false>
__device__ __forceinline__ void gemv_rows(const uint8_t* __restrict__ packed, const void* __restrict__ x, Rows rows,
                                          int64_t K, int64_t g, int kb0, int kb1, float (&acc)[4][NTL],
                                          NormIn nrm = {}) {
    constexpr int TB = Q40 ? kQ0TileBytes : kTileBytes;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: scalar branches
    kb0 = __builtin_amdgcn_readfirstlane(kb0);
    kb1 = __builtin_amdgcn_readfirstlane(kb1);
    const int i16 = lane & 15, kg = lane >> 4;
    const int64_t KB = K >> 5;
    const uint8_t* gbase = packed + g * KB * TB;
    const int coff = lane * 16, soff = kCodeBytes + i16 * (Q40 ? 8 : 16);   // per-lane byte offsets in a tile
    const bf16x8 neg128 = __builtin_bit_cast(bf16x8, u32x4{0xC300C300u, 0xC300C300u, 0xC300C300u, 0xC300C300u});
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    const CodeConsts kc = code_consts();
    const int64_t xrow = rows(token_of_row(i16));
    // From NTL = 2 on (M > 4) only lanes whose activation row reaches a stored output load
    // it: MFMA row i16 (a token slot) past M feeds only its own, discarded output row, so
    // those lanes keep a zero fragment. Every lane loads the scales (a lane of k-group kg
    // holds tokens kg, kg + 4, ..., and kg <= 3 < M). Measured on 8 Llama-3-8B layers:
    // M = 8 236.4 -> 230.1 us, M = 16 288.8 -> 279.7 us, bit-identical; at M <= 4 it
    // gained nothing (M = 1 194.9 -> 196.2 us), so one-accumulator instances load in
    // every lane.
    constexpr bool kPred = NTL >= 2;
    const bool need_x = !kPred || token_of_row(i16) < rows.M;
    u32x4 s[kUnroll];
    bf16x8 xh[kUnroll], xl[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        s[u] = u32x4{0u, 0u, 0u, 0u};
        xh[u] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
        xl[u] = xh[u];
    }

    for (int kb = kb0 + wave; kb < kb1; kb += WAVES * kUnroll) {
        u32x4 c[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int t = min(kb + WAVES * u, kb1 - 1);
            const uint8_t* tp = gbase + (int64_t)t * TB;              // wave-uniform tile base
            c[u] = load_nt_u32x4(tp + coff);
            if constexpr (Q40) {
                const u32x2 d2 = load_nt_u32x2(tp + soff);
                s[u] = u32x4{d2[0], d2[1], 0u, 0u};
            } else {
                s[u] = load_nt_u32x4(tp + soff);
            }
            if (need_x) {
                if constexpr (NORM)
                    xh[u] = norm_bf16x8((const float*)x + xrow * K + (int64_t)t * 32 + kg * 8,
                                        (const uint8_t*)nrm.w + ((int64_t)t * 32 + kg * 8) * (nrm.w_bf16 ? 2 : 4),
                                        nrm.w_bf16, nrm.r[xrow]);
                else
                    load_xfrag<XF32>(x, K, xrow, (int64_t)t * 32 + kg * 8, xh[u], xl[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (kb + WAVES * u < kb1) {
                f32x4 ns = mfma_bf16(xh[u], neg128, zero4);
                if constexpr (XF32) ns = mfma_bf16(xl[u], neg128, ns);
                f32x4 p[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bf16x8 b = codes_to_bf16(c[u][r], kc);
                    p[r] = mfma_bf16(xh[u], b, ns);
                    if constexpr (XF32) p[r] = mfma_bf16(xl[u], b, p[r]);
                }
                float sx[NTL];
#pragma unroll
                for (int j = 0; j < NTL; ++j) sx[j] = ns[j] * (-1.0f / 128.0f);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float d, m;
                    if constexpr (Q40) {
                        d = bf16_hi_to_f32(r & 1 ? s[u][r >> 1] : s[u][r >> 1] << 16);
                        m = -8.0f * d;
                    } else {
                        d = bf16_hi_to_f32(s[u][r]);
                        m = bf16_lo_to_f32(s[u][r]);
                    }
#pragma unroll
                    for (int j = 0; j < NTL; ++j) {
                        acc[r][j] = __builtin_fmaf(d, p[r][j], acc[r][j]);
                        acc[r][j] = __builtin_fmaf(m, sx[j], acc[r][j]);
                    }
                }
            }
        }
    }
}

// gemv_rows over the native Q4_K layout (kKTileBytes tiles): wave w takes the whole
// super-blocks sb0 + w, sb0 + w + kWaves, ... of [sb0, sb1): its 8 code sub-tiles and
// activation fragments, its rows' 16 (sc, mn) bytes and its d and m, then per 32-K block
// the scale d * sc and offset m * mn (both exact in f32), applied as above.
template <int NTL, bool XF32, class Rows>
__device__ __forceinline__ void q4k_rows(const uint8_t* __restrict__ packed, const void* __restrict__ x, Rows rows,
                                         int64_t K, int64_t g, int sb0, int sb1, float (&acc)[4][NTL]) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    sb0 = __builtin_amdgcn_readfirstlane(sb0);
    sb1 = __builtin_amdgcn_readfirstlane(sb1);
    const int i16 = lane & 15, kg = lane >> 4;
    const int64_t SB = K >> 8;
    const uint8_t* gbase = packed + g * SB * kKTileBytes;
    const int coff = lane * 16, soff = kKScOff + i16 * 64, doff = kKDOff + i16 * 16, moff = kKMOff + i16 * 16;
    const bf16x8 neg128 = __builtin_bit_cast(bf16x8, u32x4{0xC300C300u, 0xC300C300u, 0xC300C300u, 0xC300C300u});
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    const CodeConsts kc = code_consts();
    const int64_t xrow = rows(token_of_row(i16));

    for (int sb = sb0 + wave; sb < sb1; sb += kWaves) {
        const uint8_t* tp = gbase + (int64_t)sb * kKTileBytes;                 // wave-uniform
        // the super-block's scales first: loads land in issue order, so block 0's
        // epilogue then waits for its own codes only, not for every block's
        u32x4 c[8], sm[4];
        bf16x8 xh[8], xl[8];
        const f32x4 dv = *(const f32x4*)(tp + doff), mv = *(const f32x4*)(tp + moff);
#pragma unroll
        for (int r = 0; r < 4; ++r) sm[r] = load_nt_u32x4(tp + soff + r * 16);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            c[j] = load_nt_u32x4(tp + j * 1024 + coff);
            load_xfrag<XF32>(x, K, xrow, (int64_t)sb * 256 + j * 32 + kg * 8, xh[j], xl[j]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            f32x4 ns = mfma_bf16(xh[j], neg128, zero4);
            if constexpr (XF32) ns = mfma_bf16(xl[j], neg128, ns);
            f32x4 p[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bf16x8 b = codes_to_bf16(c[j][r], kc);
                p[r] = mfma_bf16(xh[j], b, ns);
                if constexpr (XF32) p[r] = mfma_bf16(xl[j], b, p[r]);
            }
            float sx[NTL];
#pragma unroll
            for (int t = 0; t < NTL; ++t) sx[t] = ns[t] * (-1.0f / 128.0f);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float d = dv[r] * (float)((sm[r][j >> 2] >> (8 * (j & 3))) & 0xFF);
                const float m = mv[r] * (float)((sm[r][2 + (j >> 2)] >> (8 * (j & 3))) & 0xFF);
#pragma unroll
                for (int t = 0; t < NTL; ++t) {
                    acc[r][t] = __builtin_fmaf(d, p[r][t], acc[r][t]);
                    acc[r][t] = __builtin_fmaf(m, sx[t], acc[r][t]);
                }
            }
        }
    }
}

// gemv_rows over the native q8 layout (kQ8TileBytes tiles). Each code byte b = q + 128
// splits into nibbles, q = 16 hi + lo - 128; per row tile two MFMAs on the nibble planes
// (the bf16 128 + nibble trick, offset taken out by the -128 sum x C input) give
// P_hi = sum hi x and P_lo = sum lo x, and acc += s (16 P_hi + P_lo) - 128 s sum x.
template <int NTL, bool XF32, class Rows>
__device__ __forceinline__ void q8n_rows(const uint8_t* __restrict__ packed, const void* __restrict__ x, Rows rows,
                                         int64_t K, int64_t g, int kb0, int kb1, float (&acc)[4][NTL]) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    kb0 = __builtin_amdgcn_readfirstlane(kb0);
    kb1 = __builtin_amdgcn_readfirstlane(kb1);
    const int i16 = lane & 15, kg = lane >> 4;
    const int64_t KB = K >> 5;
    const uint8_t* gbase = packed + g * KB * kQ8TileBytes;
    const int coff = lane * 16, soff = kQ8ScaleOff + i16 * 8;
    const bf16x8 neg128 = __builtin_bit_cast(bf16x8, u32x4{0xC300C300u, 0xC300C300u, 0xC300C300u, 0xC300C300u});
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    const CodeConsts kc = code_consts();
    const int64_t xrow = rows(token_of_row(i16));

    for (int kb = kb0 + wave; kb < kb1; kb += kWaves * kUnroll) {
        u32x4 c[kUnroll][2];
        u32x2 sv[kUnroll];
        bf16x8 xh[kUnroll], xl[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int t = min(kb + kWaves * u, kb1 - 1);
            const uint8_t* tp = gbase + (int64_t)t * kQ8TileBytes;              // wave-uniform
            c[u][0] = load_nt_u32x4(tp + coff);
            c[u][1] = load_nt_u32x4(tp + coff + 1024);
            sv[u] = load_nt_u32x2(tp + soff);
            load_xfrag<XF32>(x, K, xrow, (int64_t)t * 32 + kg * 8, xh[u], xl[u]);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (kb + kWaves * u < kb1) {
                f32x4 ns = mfma_bf16(xh[u], neg128, zero4);
                if constexpr (XF32) ns = mfma_bf16(xl[u], neg128, ns);
                float sx[NTL];
#pragma unroll
                for (int j = 0; j < NTL; ++j) sx[j] = ns[j] * (-1.0f / 128.0f);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t w0 = c[u][r >> 1][2 * (r & 1)], w1 = c[u][r >> 1][2 * (r & 1) + 1];
                    const bf16x8 blo = __builtin_bit_cast(bf16x8, u32x4{(w0 & kc.nib2) | kc.magic,
                                                                        ((w0 >> 8) & kc.nib2) | kc.magic,
                                                                        (w1 & kc.nib2) | kc.magic,
                                                                        ((w1 >> 8) & kc.nib2) | kc.magic});
                    const bf16x8 bhi = __builtin_bit_cast(bf16x8, u32x4{((w0 >> 4) & kc.nib2) | kc.magic,
                                                                        ((w0 >> 12) & kc.nib2) | kc.magic,
                                                                        ((w1 >> 4) & kc.nib2) | kc.magic,
                                                                        ((w1 >> 12) & kc.nib2) | kc.magic});
                    f32x4 plo = mfma_bf16(xh[u], blo, ns), phi = mfma_bf16(xh[u], bhi, ns);
                    if constexpr (XF32) {
                        plo = mfma_bf16(xl[u], blo, plo);
                        phi = mfma_bf16(xl[u], bhi, phi);
                    }
                    const float s = __builtin_bit_cast(float, (sv[u][r >> 1] >> (16 * (r & 1))) << 16);
                    const float ms = -128.0f * s;
#pragma unroll
                    for (int j = 0; j < NTL; ++j) {
                        const float t16 = __builtin_fmaf(16.0f, phi[j], plo[j]);
                        acc[r][j] = __builtin_fmaf(s, t16, acc[r][j]);
                        acc[r][j] = __builtin_fmaf(ms, sx[j], acc[r][j]);
                    }
                }
            }
        }
    }
}

// gemv_rows for 17 to 32 tokens (M > 16): two 16-token blocks share each tile's code and
// scale loads. Block 0 holds tokens 0..15 (four accumulators per row, acc0), block 1 tokens
// 16..M-1 (NTL2 accumulators, acc1); each block is the 16-token case above with its own
// activation fragment, -128 sum and MFMAs. Lanes of block 1 whose token slot is past M keep
// a zero fragment (their MFMA rows feed only discarded outputs).
template <int NTL2, bool XF32, int WAVES = kWaves>
__device__ __forceinline__ void gemv_rows_tb2(const uint8_t* __restrict__ packed, const void* __restrict__ x, int M,
                                              int64_t K, int64_t g, int kb0, int kb1, float (&acc0)[4][4],
                                              float (&acc1)[4][NTL2]) {
    constexpr int UNR = 2;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    kb0 = __builtin_amdgcn_readfirstlane(kb0);
    kb1 = __builtin_amdgcn_readfirstlane(kb1);
    const int i16 = lane & 15, kg = lane >> 4;
    const int64_t KB = K >> 5;
    const uint8_t* gbase = packed + g * KB * kTileBytes;
    const int coff = lane * 16, soff = kCodeBytes + i16 * 16;
    const bf16x8 neg128 = __builtin_bit_cast(bf16x8, u32x4{0xC300C300u, 0xC300C300u, 0xC300C300u, 0xC300C300u});
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    const CodeConsts kc = code_consts();
    const int64_t row0 = token_of_row(i16), tok1 = 16 + token_of_row(i16);
    const bool need1 = tok1 < M;
    const bf16x8 zx = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
    bf16x8 xh1[UNR], xl1[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) xh1[u] = xl1[u] = zx;

    for (int kb = kb0 + wave; kb < kb1; kb += WAVES * UNR) {
        u32x4 c[UNR], s[UNR];
        bf16x8 xh0[UNR], xl0[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int t = min(kb + WAVES * u, kb1 - 1);
            const uint8_t* tp = gbase + (int64_t)t * kTileBytes;
            c[u] = load_nt_u32x4(tp + coff);
            s[u] = load_nt_u32x4(tp + soff);
            load_xfrag<XF32>(x, K, row0, (int64_t)t * 32 + kg * 8, xh0[u], xl0[u]);
            if (need1) load_xfrag<XF32>(x, K, tok1, (int64_t)t * 32 + kg * 8, xh1[u], xl1[u]);
        }
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            if (kb + WAVES * u < kb1) {
                f32x4 ns0 = mfma_bf16(xh0[u], neg128, zero4), ns1 = mfma_bf16(xh1[u], neg128, zero4);
                if constexpr (XF32) {
                    ns0 = mfma_bf16(xl0[u], neg128, ns0);
                    ns1 = mfma_bf16(xl1[u], neg128, ns1);
                }
                f32x4 p0[4], p1[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bf16x8 b = codes_to_bf16(c[u][r], kc);
                    p0[r] = mfma_bf16(xh0[u], b, ns0);
                    p1[r] = mfma_bf16(xh1[u], b, ns1);
                    if constexpr (XF32) {
                        p0[r] = mfma_bf16(xl0[u], b, p0[r]);
                        p1[r] = mfma_bf16(xl1[u], b, p1[r]);
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float d = bf16_hi_to_f32(s[u][r]), m = bf16_lo_to_f32(s[u][r]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        acc0[r][j] = __builtin_fmaf(d, p0[r][j], acc0[r][j]);
                        acc0[r][j] = __builtin_fmaf(m, ns0[j] * (-1.0f / 128.0f), acc0[r][j]);
                    }
#pragma unroll
                    for (int j = 0; j < NTL2; ++j) {
                        acc1[r][j] = __builtin_fmaf(d, p1[r][j], acc1[r][j]);
                        acc1[r][j] = __builtin_fmaf(m, ns1[j] * (-1.0f / 128.0f), acc1[r][j]);
                    }
                }
            }
        }
    }
}

// The MFMAs and scale FMAs of one K position (32 K) of NG row groups: c / s the tiles' code
// and scale words of this lane, xh / xl the activation fragment (xl only for f32 x).
template <int NTL, bool XF32, int NG>
__device__ __forceinline__ void multi_tile(const u32x4 (&c)[NG], const u32x4 (&s)[NG], bf16x8 xh, bf16x8 xl,
                                           CodeConsts kc, float (&acc)[NG][4][NTL]) {
    const bf16x8 neg128 = __builtin_bit_cast(bf16x8, u32x4{0xC300C300u, 0xC300C300u, 0xC300C300u, 0xC300C300u});
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    f32x4 ns = mfma_bf16(xh, neg128, zero4);
    if constexpr (XF32) ns = mfma_bf16(xl, neg128, ns);
    float sx[NTL];
#pragma unroll
    for (int j = 0; j < NTL; ++j) sx[j] = ns[j] * (-1.0f / 128.0f);
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        f32x4 p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bf16x8 b = codes_to_bf16(c[i][r], kc);
            p[r] = mfma_bf16(xh, b, ns);
            if constexpr (XF32) p[r] = mfma_bf16(xl, b, p[r]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float d = bf16_hi_to_f32(s[i][r]), m = bf16_lo_to_f32(s[i][r]);
#pragma unroll
            for (int j = 0; j < NTL; ++j) {
                acc[i][r][j] = __builtin_fmaf(d, p[r][j], acc[i][r][j]);
                acc[i][r][j] = __builtin_fmaf(m, sx[j], acc[i][r][j]);
            }
        }
    }
}

// gemv_rows over NG row groups at once (tile bases gbase[i], same K range and
// activations): per K position the activation fragment and the -128 sum x
// MFMA are shared by the NG groups, and NG x UNR tiles are in flight per wave.
template <int NTL, bool XF32, int NG, int UNR, int WAVES = kWaves, bool NORM = false, class Rows>
__device__ __forceinline__ void gemv_rows_multi(const uint8_t* const (&gbase)[NG], const void* __restrict__ x, Rows rows,
                                                int64_t K, int kb0, int kb1, float (&acc)[NG][4][NTL],
                                                NormIn nrm = {}) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    kb0 = __builtin_amdgcn_readfirstlane(kb0);
    kb1 = __builtin_amdgcn_readfirstlane(kb1);
    const int i16 = lane & 15, kg = lane >> 4;
    const int coff = lane * 16, soff = kCodeBytes + i16 * 16;
    const CodeConsts kc = code_consts();
    const int64_t xrow = rows(token_of_row(i16));

    for (int kb = kb0 + wave; kb < kb1; kb += WAVES * UNR) {
        u32x4 c[UNR][NG], s[UNR][NG];
        bf16x8 xh[UNR], xl[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int t = min(kb + WAVES * u, kb1 - 1);
#pragma unroll
            for (int i = 0; i < NG; ++i) {
                const uint8_t* tp = gbase[i] + (int64_t)t * kTileBytes;
                c[u][i] = load_nt_u32x4(tp + coff);
                s[u][i] = load_nt_u32x4(tp + soff);
            }
            if constexpr (NORM)
                xh[u] = norm_bf16x8((const float*)x + xrow * K + (int64_t)t * 32 + kg * 8,
                                    (const uint8_t*)nrm.w + ((int64_t)t * 32 + kg * 8) * (nrm.w_bf16 ? 2 : 4),
                                    nrm.w_bf16, nrm.r[xrow]);
            else
                load_xfrag<XF32>(x, K, xrow, (int64_t)t * 32 + kg * 8, xh[u], xl[u]);
        }
#pragma unroll
        for (int u = 0; u < UNR; ++u)
            if (kb + WAVES * u < kb1) multi_tile<NTL, XF32, NG>(c[u], s[u], xh[u], xl[u], kc, acc);
    }
}

// 16 bytes per lane into registers, streaming, that the compiler does not track: the caller
// waits for it (s_waitcnt vmcnt, in issue order) and passes the registers through
// pipe_landed before any use. Weights: wave-uniform base + 32-bit lane offset.
__device__ __forceinline__ void pipe_load_w(u32x4& dst, const void* gbase, uint32_t goff) {
    asm volatile("global_load_dwordx4 %0, %1, %2 nt" : "=v"(dst) : "v"(goff), "s"(gbase) : "memory");
}
// Activations: a per-lane 64-bit address (gathered rows), cached.
__device__ __forceinline__ void pipe_load_x(u32x4& dst, const void* p) {
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(dst) : "v"(p) : "memory");
}
__device__ __forceinline__ void pipe_landed(u32x4& v) { asm volatile("" : "+v"(v)); }

constexpr int pipe_wait_imm(int vm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (15 << 8); }

// f(std::integral_constant<int, I>{}) for I = B .. E - 1, so f can use I as a constant.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// gemv_rows_multi as a rolling pipeline with explicit waits: a wave keeps UNR K positions of
// loads (NG tiles' codes and scales plus the activation fragment each) in flight at all
// times. Its K positions are kb0 + wave + WAVES b, b = 0 .. cnt - 1; while b + UNR lies
// before the last chunk of UNR positions, position b + UNR is issued into the registers of
// position b as soon as b has been used, so the wait before each position is "all but the
// (UNR - 1) younger positions' loads"; the last chunk waits down to zero. Positions of the
// last chunk past cnt load the wave's last tile again (at most UNR - 1, cache hits) and
// are not accumulated.
template <int NTL, bool XF32, int NG, int UNR, int WAVES, class Rows>
__device__ __forceinline__ void gemv_rows_pipe(const uint8_t* const (&gbase)[NG], const void* __restrict__ x, Rows rows,
                                               int64_t K, int kb0, int kb1, float (&acc)[NG][4][NTL]) {
    constexpr int XL = XF32 ? 2 : 1;                // activation loads per K position
    constexpr int L = 2 * NG + XL;                  // loads per K position
    static_assert((UNR - 1) * L <= 63, "vmcnt holds 6 bits");
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    kb0 = __builtin_amdgcn_readfirstlane(kb0);
    kb1 = __builtin_amdgcn_readfirstlane(kb1);
    const int first = kb0 + wave;
    if (first >= kb1) return;
    const int cnt = (kb1 - first + WAVES - 1) / WAVES;
    const int i16 = lane & 15, kg = lane >> 4;
    const uint32_t coff = lane * 16, soff = kCodeBytes + i16 * 16;
    const CodeConsts kc = code_consts();
    const int64_t es = XF32 ? 4 : 2;
    const uint8_t* xp = (const uint8_t*)x + (rows(token_of_row(i16)) * K + kg * 8) * es;
    u32x4 c[UNR][NG], s[UNR][NG], xr[UNR][XL];
    auto issue = [&](int b, int slot) {
        const int t = first + WAVES * min(b, cnt - 1);
        const uint32_t toff = (uint32_t)t * kTileBytes;
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            pipe_load_w(c[slot][i], gbase[i], toff + coff);
            pipe_load_w(s[slot][i], gbase[i], toff + soff);
        }
        const uint8_t* xa = xp + (int64_t)t * 32 * es;
#pragma unroll
        for (int h = 0; h < XL; ++h) pipe_load_x(xr[slot][h], xa + 16 * h);
    };
    auto land = [&](int slot) {
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            pipe_landed(c[slot][i]);
            pipe_landed(s[slot][i]);
        }
#pragma unroll
        for (int h = 0; h < XL; ++h) pipe_landed(xr[slot][h]);
    };
    auto run = [&](int u) {
        bf16x8 xh, xl;
        if constexpr (XF32) {
            const f32x4 a = __builtin_bit_cast(f32x4, xr[u][0]), bb = __builtin_bit_cast(f32x4, xr[u][1]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const __bf16 ha = (__bf16)a[e], hb = (__bf16)bb[e];
                xh[e] = ha;
                xh[e + 4] = hb;
                xl[e] = (__bf16)(a[e] - (float)ha);
                xl[e + 4] = (__bf16)(bb[e] - (float)hb);
            }
        } else {
            xh = __builtin_bit_cast(bf16x8, xr[u][0]);
        }
        multi_tile<NTL, XF32, NG>(c[u], s[u], xh, xl, kc, acc);
    };
#pragma unroll
    for (int u = 0; u < UNR; ++u) issue(u, u);
    int b0 = 0;
    for (; b0 + UNR < cnt; b0 += UNR) {
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            __builtin_amdgcn_s_waitcnt(pipe_wait_imm((UNR - 1) * L));
            land(u);
            run(u);
            issue(b0 + u + UNR, u);
        }
    }
    static_for<0, UNR>([&](auto U) {      // the last chunk: nothing more to issue
        constexpr int u = decltype(U)::value;
        __builtin_amdgcn_s_waitcnt(pipe_wait_imm((UNR - 1 - u) * L));
        land(u);
        if (b0 + u < cnt) run(u);
    });
}

// One K position's arithmetic over NG row groups (gemv_rows' per-tile body; multi_tile's
// for NG > 1): codes c[i], scale words s[i] (mx: d<<16 | m per row sub-tile; mx0: four
// bf16 d in s[i][0..1]), activation fragment xh (+ xl for f32 x) shared by the groups.
// F16S: the scale words hold fp16 d and m (q4_repack scale_mode 1).
template <int NTL, bool XF32, bool Q40, int NG, bool F16S = false>
__device__ __forceinline__ void tile_math(const u32x4 (&c)[NG], const u32x4 (&s)[NG], bf16x8 xh, bf16x8 xl,
                                          CodeConsts kc, float (&acc)[NG][4][NTL]) {
    const bf16x8 neg128 = __builtin_bit_cast(bf16x8, u32x4{0xC300C300u, 0xC300C300u, 0xC300C300u, 0xC300C300u});
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    f32x4 ns = mfma_bf16(xh, neg128, zero4);
    if constexpr (XF32) ns = mfma_bf16(xl, neg128, ns);
    float sx[NTL];
#pragma unroll
    for (int j = 0; j < NTL; ++j) sx[j] = ns[j] * (-1.0f / 128.0f);
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        f32x4 p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bf16x8 b = codes_to_bf16(c[i][r], kc);
            p[r] = mfma_bf16(xh, b, ns);
            if constexpr (XF32) p[r] = mfma_bf16(xl, b, p[r]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float d, m;
            if constexpr (Q40) {
                d = bf16_hi_to_f32(r & 1 ? s[i][r >> 1] : s[i][r >> 1] << 16);
                m = -8.0f * d;
            } else {
                d = scale_d<F16S>(s[i][r]);
                m = scale_m<F16S>(s[i][r]);
            }
#pragma unroll
            for (int j = 0; j < NTL; ++j) {
                acc[i][r][j] = __builtin_fmaf(d, p[r][j], acc[i][r][j]);
                acc[i][r][j] = __builtin_fmaf(m, sx[j], acc[i][r][j]);
            }
        }
    }
}

// gemv_rows (NG = 1) and gemv_rows_multi (NG row groups with tile bases gbase[i], the same
// K range and activations) as a rolling pipeline with explicit waits: a wave issues its
// first UNR K positions (per group the codes and scales, and the activation fragment; NW:
// the f32 row and the norm weight, bf16 (NW 1) or f32 (NW 2)), then per position b waits
// for "all but the positions issued after b", runs the position and, while b + UNR lies
// before the last chunk of UNR positions, issues b + UNR into b's registers. Every issue is
// unconditional (an asm load issued under a branch merges with the slot's old value, and the
// register allocator may then copy the asm output before its wait): the last chunk's
// positions past the wave's count re-load its last tile (at most UNR - 1 of them, cache
// hits) and are not accumulated. Positions are visited in the same order as the batched
// loops, with the same arithmetic, so the sums are bit-identical to theirs for the same
// waves and K range.
//
// XS: the activations were staged in LDS as bf16 fragments (xs[m][kr] over the K range
// [kb0, kb1) of 32-wide positions, e.g. by stage_norm_acc_row), so a position is its weight
// loads only.
template <int NTL, bool XF32, int NG, int UNR, int WAVES, bool Q40, int NW, class Rows, bool XS = false,
          bool F16S = false>
__device__ __forceinline__ void gemv_rows_stream(const uint8_t* const (&gbase)[NG], const void* __restrict__ x,
                                                 Rows rows, int64_t K, int kb0, int kb1, float (&acc)[NG][4][NTL],
                                                 NormIn nrm = {}, const __bf16* xs = nullptr, int kr = 0) {
    static_assert(!XS || (!XF32 && NW == 0), "staged fragments are one bf16 plane");
    static_assert(!F16S || !Q40, "fp16 scale words are an mx-layout mode");
    constexpr int TB = Q40 ? kQ0TileBytes : kTileBytes;
    constexpr int XL = XS ? 0 : NW == 0 ? (XF32 ? 2 : 1) : (NW == 1 ? 3 : 4);   // activation-side loads
    constexpr int L = 2 * NG + XL;                                     // loads per K position
    static_assert((UNR - 1) * L <= 63, "vmcnt holds 6 bits");
    static_assert(NW == 0 || !XF32, "a normalised row feeds the MFMA as one bf16 fragment");
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    kb0 = __builtin_amdgcn_readfirstlane(kb0);
    kb1 = __builtin_amdgcn_readfirstlane(kb1);
    const int first = kb0 + wave;
    if (first >= kb1) return;
    const int cnt = (kb1 - first + WAVES - 1) / WAVES;
    const int i16 = lane & 15, kg = lane >> 4;
    // mx0: the 16 aligned bytes holding this lane's 8 scale bytes and its neighbour's (an asm
    // load into a register pair drew compiler copies ahead of its wait)
    const uint32_t coff = lane * 16, soff = kCodeBytes + (Q40 ? (i16 & ~1) * 8 : i16 * 16);
    const bool odd = Q40 && (i16 & 1);
    const CodeConsts kc = code_consts();
    const int64_t xrow = rows(token_of_row(i16));
    constexpr int64_t es = (XF32 || NW) ? 4 : 2;                       // activation element bytes
    const uint8_t* xp = (const uint8_t*)x + (xrow * K + kg * 8) * es;
    constexpr int64_t ws = NW == 1 ? 2 : 4;                            // norm weight element bytes
    const uint8_t* wp = NW ? (const uint8_t*)nrm.w + kg * 8 * ws : nullptr;
    const float rr = NW ? nrm.r[xrow] : 0.f;
    u32x4 c[UNR][NG], s[UNR][NG], xr[UNR][XL > 0 ? XL : 1];
    const __bf16* xsl = XS ? xs + xrow * kr + kg * 8 - (int64_t)kb0 * 32 : nullptr;   // this lane's fragments
    auto issue = [&](int b, int slot) {
        const int t = first + WAVES * min(b, cnt - 1);
        const uint32_t toff = (uint32_t)t * TB;
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            pipe_load_w(c[slot][i], gbase[i], toff + coff);
            pipe_load_w(s[slot][i], gbase[i], toff + soff);
        }
        if constexpr (XS) return;
        const uint8_t* xa = xp + (int64_t)t * 32 * es;
        pipe_load_x(xr[slot][0], xa);
        if constexpr (XF32 || NW) pipe_load_x(xr[slot][1], xa + 16);
        if constexpr (NW) {
            const uint8_t* wa = wp + (int64_t)t * 32 * ws;
            pipe_load_x(xr[slot][2], wa);
            if constexpr (NW == 2) pipe_load_x(xr[slot][3], wa + 16);
        }
    };
    auto land = [&](int slot) {
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            pipe_landed(c[slot][i]);
            pipe_landed(s[slot][i]);
        }
#pragma unroll
        for (int h = 0; h < XL; ++h) pipe_landed(xr[slot][h]);
    };
    auto run = [&](int u, int b) {
        bf16x8 xh, xl;
        if constexpr (XS) {
            xh = *(const bf16x8*)(xsl + (int64_t)(first + WAVES * b) * 32);
        } else if constexpr (NW) {
            float wv[8];
            if constexpr (NW == 1) {
                norm_w_of_bf16(xr[u][2], wv);
            } else {
                const f32x4 w0 = __builtin_bit_cast(f32x4, xr[u][2]), w1 = __builtin_bit_cast(f32x4, xr[u][3]);
#pragma unroll
                for (int e = 0; e < 4; ++e) wv[e] = w0[e], wv[e + 4] = w1[e];
            }
            xh = norm_bf16x8_of(__builtin_bit_cast(f32x4, xr[u][0]), __builtin_bit_cast(f32x4, xr[u][1]), wv, rr);
        } else if constexpr (XF32) {
            const f32x4 a = __builtin_bit_cast(f32x4, xr[u][0]), bb = __builtin_bit_cast(f32x4, xr[u][1]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const __bf16 ha = (__bf16)a[e], hb = (__bf16)bb[e];
                xh[e] = ha;
                xh[e + 4] = hb;
                xl[e] = (__bf16)(a[e] - (float)ha);
                xl[e + 4] = (__bf16)(bb[e] - (float)hb);
            }
        } else {
            xh = __builtin_bit_cast(bf16x8, xr[u][0]);
        }
        u32x4 sw[NG];
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            sw[i] = s[u][i];
            if constexpr (Q40) sw[i] = odd ? u32x4{sw[i][2], sw[i][3], 0u, 0u} : u32x4{sw[i][0], sw[i][1], 0u, 0u};
        }
        tile_math<NTL, XF32, Q40, NG, F16S>(c[u], sw, xh, xl, kc, acc);
    };
#pragma unroll
    for (int u = 0; u < UNR; ++u) issue(u, u);
    int b0 = 0;
    for (; b0 + UNR < cnt; b0 += UNR) {
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            __builtin_amdgcn_s_waitcnt(pipe_wait_imm((UNR - 1) * L));
            land(u);
            run(u, b0 + u);
            issue(b0 + u + UNR, u);
        }
    }
    static_for<0, UNR>([&](auto U) {      // the last chunk: nothing more to issue
        constexpr int u = decltype(U)::value;
        __builtin_amdgcn_s_waitcnt(pipe_wait_imm((UNR - 1 - u) * L));
        land(u);
        if (b0 + u < cnt) run(u, b0 + u);
    });
}

// One activation row of K <= 256 kAccRowJ values that a split GEMV left as partial sums:
//   x = res + (((0 + part[0]) + part[1]) + ...)     (S > 1: split_reduce's order)
//   x = res + part[0]                               (S = 1: the unsplit store's)
//   x = res                                         (S = 0)
// with part planes plane_stride floats apart. From one read of res and the planes: x into
// x_out (when given: one workgroup writes it), the row's 1/rms with rms_inv_rows'
// arithmetic and order, and ((x * r) * w) rounded to bf16 over columns [k0, k0 + kr) into
// xs. All NT threads of the workgroup share the loads (element i = tid + NT e), the
// planes in batches whose loads are all issued before the first add (the planes were just
// written by another kernel: each batch pays one trip to memory); x passes through LDS
// (xf) to the 256 threads that form the sum of squares in rms_inv_rows' order. Every
// thread calls it; barriers inside.
constexpr int kAccRowJ = 16;
template <int NW, int NT>
__device__ __forceinline__ void stage_norm_acc_row(const float* __restrict__ res, const float* __restrict__ part,
                                                   int S, int64_t plane_stride, int64_t K, float eps,
                                                   const void* __restrict__ w, int64_t k0, int kr, __bf16* xs,
                                                   float* __restrict__ x_out, float* xf) {
    constexpr int E = 256 * kAccRowJ / NT;            // elements per thread in the sum
    // planes per batch: 64 values in flight, 32 in a 1024-thread workgroup (128 VGPRs a lane)
    constexpr int kFly = NT >= 1024 ? 32 : 64, PB = E >= kFly ? 1 : kFly / E;
    __shared__ double partd[4];
    const int tid = threadIdx.x;
    // every load below is unconditional, at an index clamped into the row (a load under a
    // lane condition is compiled as a branch with a wait for it inside): values past K or
    // outside this workgroup's columns are loaded and not used
    auto ix = [&](int64_t i) { return i < K ? i : K - 1; };
    // this workgroup's columns of the norm weight, as raw words converted where used (a
    // bf16 weight: the word holding element i, i's half picked by i's parity; 16-bit loads
    // drew waits for packing ahead of the plane loads)
    uint32_t wl[kAccRowJ];
    if (tid < 256) {
#pragma unroll
        for (int j = 0; j < kAccRowJ; ++j) {
            const int64_t i = ix(tid + 256 * j);
            wl[j] = ((const uint32_t*)w)[NW == 1 ? i >> 1 : i];
        }
    }
    float r0[E], v[E];
#pragma unroll
    for (int e = 0; e < E; ++e) r0[e] = res[ix(tid + NT * e)];
    if (S == 1) {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = part[ix(tid + NT * e)];
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = r0[e] + v[e];
    } else {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = 0.f;
        for (int q = 0; q < S; q += PB) {
            float t[PB][E];
#pragma unroll
            for (int u = 0; u < PB; ++u)
#pragma unroll
                for (int e = 0; e < E; ++e) t[u][e] = part[min(q + u, S - 1) * plane_stride + ix(tid + NT * e)];
#pragma unroll
            for (int u = 0; u < PB; ++u)
                if (q + u < S) {
#pragma unroll
                    for (int e = 0; e < E; ++e) v[e] += t[u][e];
                }
        }
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = S == 0 ? r0[e] : r0[e] + v[e];
    }
#pragma unroll
    for (int e = 0; e < E; ++e)
        if (tid + NT * e < K) {
            xf[tid + NT * e] = v[e];
            if (x_out) x_out[tid + NT * e] = v[e];
        }
    __syncthreads();
    float x[kAccRowJ];
    if (tid < 256) {
#pragma unroll
        for (int j = 0; j < kAccRowJ; ++j) x[j] = tid + 256 * j < K ? xf[tid + 256 * j] : 0.f;
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < kAccRowJ; ++j)
            if (tid + 256 * j < K) ss += (double)x[j] * (double)x[j];
        const double wsum = wave_sum_ss(ss);
        if ((tid & 63) == 0) partd[tid >> 6] = wsum;
    }
    __syncthreads();
    if (tid < 256) {
        const float r = inv_rms(partd, K, eps);
#pragma unroll
        for (int j = 0; j < kAccRowJ; ++j) {
            const int64_t i = tid + 256 * j;
            const float wi = NW == 1 ? bf16_hi_to_f32(i & 1 ? wl[j] & 0xffff0000u : wl[j] << 16)
                                     : __uint_as_float(wl[j]);
            if (i >= k0 && i < k0 + kr) ((uint16_t*)xs)[i - k0] = (uint16_t)f32_to_bf16_rne(x[j] * r * wi);
        }
    }
    __syncthreads();
}

// Sum the WAVES waves' accumulators through LDS. Afterwards thread t < 256 owns
// row 16 r + lane % 16 of the row group (r = t >> 6, lane = t & 63) for the
// tokens token_of(lane / 16, j), j < NTL: v[j] (the waves' sums pairwise, in a
// fixed order). Threads from 256 on own nothing.
template <int NTL, int WAVES = kWaves>
__device__ __forceinline__ void wave_sum(float (&acc)[4][NTL], float (*red)[4][NTL][64], float (&v)[NTL]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < NTL; ++j) red[wave][r][j][lane] = acc[r][j];
    __syncthreads();
    if (wave >= 4) return;
    const int r = wave;
#pragma unroll
    for (int j = 0; j < NTL; ++j) {
        float t[WAVES];
#pragma unroll
        for (int w = 0; w < WAVES; ++w) t[w] = red[w][r][j][lane];
#pragma unroll
        for (int h = WAVES / 2; h >= 1; h /= 2)
#pragma unroll
            for (int w = 0; w < h; ++w) t[w] = t[2 * w] + t[2 * w + 1];
        v[j] = t[0];
    }
}

// Store the row group's result (S == 1, plus the residual when one is given) or this
// split's partial sums (res null).
template <int NTL, int WAVES = kWaves>
__device__ __forceinline__ void gemv_finish(float (&acc)[4][NTL], float (*red)[4][NTL][64], int M,
                                            float* y, int64_t N, int64_t g, const float* res = nullptr) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int r = tid >> 6, i16 = lane & 15, kg = lane >> 4;
    const int64_t n = g * 64 + r * 16 + i16;
    float v[NTL];
    wave_sum<NTL, WAVES>(acc, red, v);
    if (r >= 4) return;
#pragma unroll
    for (int j = 0; j < NTL; ++j) {
        const int tok = token_of(kg, j);
        if (tok < M) y[(int64_t)tok * N + n] = res ? res[(int64_t)tok * N + n] + v[j] : v[j];
    }
}

}  // namespace q4mi
