// prefill.hip -- prefill GEMM: Y[T][N] = X[T][K] . W[N][K]^T, W in the mx layout,
// dequantized into LDS tiles that feed the 16x16x32 MFMA, fp32 accumulate.
//
// The reference prefill dequantizes one 64x64 tile of a band into a bf16 A
// operand in core memory, then runs mlir-aie's bf16 matmul on it
// (open_kernels/designs/gemm_q4_prefill/gemm_q4_dequant.h:315-376,
// gemm_q4_prefill.py:198-203). Rounding each weight once to bf16 costs a
// maxrel of ~1.8e-3 against the fp64 reference (gemm_q4_dequant.h:283-286),
// over the 1e-3 bar. Two precisions are built from one kernel:
//   PREC 0 (default): fp16 MFMA (CDNA4's dense fp16 and bf16 MFMA peaks are
//     equal) on power-of-two-scaled operands, so fp16's narrow exponent range
//     costs nothing: token row t is scaled by 2^-s_t so its max |x| lands in
//     [2^14, 2^15) (bf16 -> fp16 is then exact: 8 significant bits, no
//     overflow, no subnormal short of 2^-10 of the row max), and weight row n
//     by 2^-e_n so its bound max_kb (15 |d| + |m|) >= max |w| lands there too:
//     w16 = RNE_f16(q (d 2^-e) + m 2^-e) (one v_pk_fma_f16 per pair, 11-bit
//     significand; d 2^-e and m 2^-e are exact in fp16 for every block within
//     2^-24 of the row's bound). The output is ldexp(acc, s_t + e_n), exact.
//     The token exponents come from the activation pre-pass. The weight rows'
//     exponents and their scale words, scaled and in fp16, form the "prefill
//     scales" of a matrix (q4_prefill_scales): a side plane laid out as the mx
//     tiles' scale blocks (256 B per tile) from which the GEMM reads its scale
//     words. Weights are static, so a caller computes them once per matrix
//     (q4_gemm_prefill_scaled); q4_gemm_prefill computes them per call.
//   PREC 1: the reference tile RNE_bf16(fl32(q*d + m)) with bf16 X, bf16 MFMA.
// The exact-code alternative (4-bit codes on the MFMA, d and m applied per
// 32-K block in fp32, as the decode kernel does) needs two VALU FMAs per
// output per block, i.e. twice the MFMA time of the same block at
// 512 MAC/clk vs 16 FMA/clk per SIMD, so it cannot reach the MFMA roofline.
//
// Tiling: a workgroup computes BN weight rows x BT tokens with WGN x WGT
// waves. Per LDS stage (KS blocks of 32 K) the waves turn the stage's mx
// tiles (one 64-row group x 32 K each) into 16-bit weights in LDS and copy
// the activations to LDS; stages are double buffered so the global loads and
// the dequant of stage s+1 overlap the MFMAs of stage s, with one barrier per
// stage. The default variant runs 8 waves (two per SIMD, 128x64 wave tiles),
// so one wave's dequant and LDS traffic hide behind the other's MFMAs. LDS
// rows are padded by 8 halves so a 16-lane ds_read_b128 phase hits distinct
// banks.
#include <stdlib.h>

#include "norm_core.h"
#include "q4mi_device.h"
#include "q4mi_internal.h"

using namespace q4mi;

namespace {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
constexpr uint32_t kMagic1024 = 0x64006400u;   // fp16 1024.0 in both halves


__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// One codes dword + its row's scale word -> eight 16-bit weights (as u32x4),
// element e = k offset e of the dword's k-group. The scale word is (d << 16 | m):
// PREC 0 reads it from the fp16 side plane (d and m already scaled by the row's
// 2^-e), PREC 1 from the mx tile (bf16).
template <int PREC>
__device__ __forceinline__ u32x4 dequant8(uint32_t w, uint32_t s, uint32_t nib2, uint32_t magic) {
    u32x4 out;
    if constexpr (PREC == 0) {
        const f16x2 sv = __builtin_bit_cast(f16x2, s);                  // [0] m, [1] d
        const f16x2 d2 = __builtin_shufflevector(sv, sv, 1, 1), m2 = __builtin_shufflevector(sv, sv, 0, 0);
        const f16x2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t v = ((w >> (4 * p)) & nib2) | magic;           // 1024 + q, exact
            const f16x2 q = __builtin_bit_cast(f16x2, v) - k1024;         // q, exact
            out[p] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, d2, m2));
        }
    } else {
        const float d = bf16_hi_to_f32(s), m = bf16_lo_to_f32(s);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const float lo = __builtin_fmaf((float)((w >> (4 * p)) & 0xF), d, m);
            const float hi = __builtin_fmaf((float)((w >> (16 + 4 * p)) & 0xF), d, m);
            const bf16x2 b = {(__bf16)lo, (__bf16)hi};
            out[p] = __builtin_bit_cast(uint32_t, b);
        }
    }
    return out;
}

// Store a wave's FN x FT fragments of 16 x 16 (rows from wn0, tokens from wt0): the lane
// holds D[n = 4 kg + r][t = i16] of each, 4 consecutive rows of one token, scaled back by
// 2^(s_t + e_n) when the operands were scaled (texp / wexp not null), exactly; accum adds
// the result to what y holds (the second pass of f32 activations). tmap: token t's exponent
// is texp[tmap[t]] (activations gathered from another row order), else texp[t].
template <int FN, int FT, bool SCALED>
__device__ __forceinline__ void store_tile(const f32x4 (&acc)[FN][FT], float* __restrict__ y,
                                           const int* __restrict__ texp, const int* __restrict__ wexp, int T, int N,
                                           int wt0, int wn0, int accum, const int* __restrict__ tmap = nullptr) {
    const int lane = threadIdx.x & 63, i16 = lane & 15, kg = lane >> 4;
#pragma unroll
    for (int j = 0; j < FT; ++j) {
        const int t = wt0 + j * 16 + i16;
        if (t >= T) continue;
        const int st = SCALED ? texp[tmap ? max(tmap[t], 0) : t] : 0;
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            const int n = wn0 + i * 16 + kg * 4;
            if (n < N) {
                f32x4 v = acc[i][j];
                if constexpr (SCALED) {
                    const int4 e = *(const int4*)(wexp + n);
                    v[0] = ldexpf(v[0], st + e.x);
                    v[1] = ldexpf(v[1], st + e.y);
                    v[2] = ldexpf(v[2], st + e.z);
                    v[3] = ldexpf(v[3], st + e.w);
                }
                if (SCALED && accum) v += *(const f32x4*)(y + (int64_t)t * N + n);   // PREC 0 only
                *(f32x4*)(y + (int64_t)t * N + n) = v;
            }
        }
    }
}

// The SwiGLU epilogue of the gate/up GEMM over an interleaved matrix (per 128-row pair p,
// 64 gate rows of F, then the same 64 rows of up: N = 2F). A 256-row tile's wave holds one
// pair, fragments 0..3 gate and 4..7 up at the same lane positions, so
// h = bf16(silu(g) * u) (q4_swiglu_prepare's arithmetic) is formed from the accumulators and
// only h [T][F] bf16 is stored: the f32 gate/up output never reaches memory.
template <int FT, bool SCALED>
__device__ __forceinline__ void store_swiglu(const f32x4 (&acc)[8][FT], uint16_t* __restrict__ h,
                                             const int* __restrict__ texp, const int* __restrict__ wexp, int T, int N,
                                             int wt0, int wn0, const int* __restrict__ tmap = nullptr) {
    const int lane = threadIdx.x & 63, i16 = lane & 15, kg = lane >> 4;
    const int F = N >> 1, f0 = wn0 >> 1;          // wn0 = 128 p: gate rows from 64 p
#pragma unroll
    for (int j = 0; j < FT; ++j) {
        const int t = wt0 + j * 16 + i16;
        if (t >= T) continue;
        const int st = SCALED ? texp[tmap ? max(tmap[t], 0) : t] : 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ng = wn0 + i * 16 + kg * 4;
            f32x4 g = acc[i][j], u = acc[i + 4][j];
            if constexpr (SCALED) {
                const int4 eg = *(const int4*)(wexp + ng), eu = *(const int4*)(wexp + ng + 64);
                g[0] = ldexpf(g[0], st + eg.x), g[1] = ldexpf(g[1], st + eg.y);
                g[2] = ldexpf(g[2], st + eg.z), g[3] = ldexpf(g[3], st + eg.w);
                u[0] = ldexpf(u[0], st + eu.x), u[1] = ldexpf(u[1], st + eu.y);
                u[2] = ldexpf(u[2], st + eu.z), u[3] = ldexpf(u[3], st + eu.w);
            }
            uint32_t o[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const float a = g[2 * e] / (1.0f + expf(-g[2 * e])) * u[2 * e];
                const float b = g[2 * e + 1] / (1.0f + expf(-g[2 * e + 1])) * u[2 * e + 1];
                o[e] = f32_to_bf16_rne(a) | (f32_to_bf16_rne(b) << 16);
            }
            *(uint2*)(h + (int64_t)t * F + f0 + i * 16 + kg * 4) = make_uint2(o[0], o[1]);
        }
    }
}

// BN x BT workgroup tile, WGN x WGT waves (wave tile BN/WGN x BT/WGT), KS
// 32-K blocks per LDS stage.
template <int BN, int BT, int WGN, int WGT, int KS, int PREC>
__global__ __launch_bounds__(64 * WGN * WGT) void prefill_kernel(const uint8_t* __restrict__ packed,
                                                                 const uint16_t* __restrict__ x16,
                                                                 const int* __restrict__ texp,
                                                                 const int* __restrict__ wexp,
                                                                 const uint32_t* __restrict__ s16,
                                                                 float* __restrict__ y, int T, int N, int K,
                                                                 int tiles_t, int accum) {
    constexpr int NT = 64 * WGN * WGT, NW = WGN * WGT;
    constexpr int WN = BN / WGN, WT = BT / WGT;      // wave tile
    constexpr int FN = WN / 16, FT = WT / 16;        // 16-wide fragments per wave
    constexpr int RG = BN / 64;                      // mx row groups per workgroup tile
    constexpr int WTILES = RG * KS;                  // mx tiles per stage
    constexpr int WPW = (WTILES + NW - 1) / NW;      // mx tiles per wave per stage
    constexpr int BK = 32 * KS;
    constexpr int STR = BK + 8;                      // halves per LDS row (pad: conflict-free b128 reads)
    constexpr int XCH = BT * KS * 4 / NT;            // 16-byte activation chunks per thread per stage
    static_assert(XCH * NT == BT * KS * 4, "activation chunks must divide evenly");
    typedef typename std::conditional<PREC == 0, f16x8, bf16x8>::type frag_t;

    __shared__ __attribute__((aligned(16))) uint16_t wl[2][BN * STR];
    __shared__ __attribute__((aligned(16))) uint16_t xl[2][BT * STR];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave % WGN, wt = wave / WGN;
    const int bt = blockIdx.x % tiles_t, bn = blockIdx.x / tiles_t;
    const int n0 = bn * BN, t0 = bt * BT;
    const int KB = K >> 5, NSTAGE = KB / KS;
    const int G = N >> 6;
    const int i16 = lane & 15, kg = lane >> 4;

    // This wave's mx tiles: tile u = wave + NW*i -> (row group u % RG, block u / RG of the
    // stage). Tile bases are wave-uniform and advance by a uniform stride per stage, and
    // the per-lane offsets are fixed 32-bit values, so no address register is rewritten
    // inside the K loop (rewriting one that a pending load targets forces a vmcnt wait).
    const uint8_t* wbase[WPW];
    const uint8_t* sbase[WPW];
    int wrow[WPW], wcol[WPW];
    bool wown[WPW];
#pragma unroll
    for (int i = 0; i < WPW; ++i) {
        const int u = wave + NW * i;
        wown[i] = u < WTILES;
        const int rgl = u % RG, kbl = u / RG;
        const int rg = min(n0 / 64 + rgl, G - 1);                       // clamp ragged N
        wbase[i] = packed + ((int64_t)rg * KB + kbl) * kTileBytes;
        sbase[i] = PREC == 0 ? (const uint8_t*)s16 + ((int64_t)rg * KB + kbl) * 256 : wbase[i] + kCodeBytes;
        wrow[i] = rgl * 64 + i16;
        wcol[i] = kbl * 32 + kg * 8;
    }
    const uint32_t coff = lane * 16, soff = i16 * 16;
    constexpr int SSTR = PREC == 0 ? 256 : kTileBytes;               // scale block stride per 32-K block
    const uint16_t* xbase = x16 + (int64_t)t0 * K;                    // workgroup-uniform
    int xoff[XCH], xdst[XCH];
#pragma unroll
    for (int c = 0; c < XCH; ++c) {
        const int ch = tid + NT * c, tok = ch / (KS * 4), part = ch % (KS * 4);
        xoff[c] = (min(t0 + tok, T - 1) - t0) * K + part * 8;            // halves, fits 32 bits
        xdst[c] = tok * STR + part * 8;
    }
    const uint32_t nib2 = vgpr_const(kNib2);
    const uint32_t magic = vgpr_const(PREC == 0 ? kMagic1024 : kMagic128);

    f32x4 acc[FN][FT];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 wc[WPW], wsc[WPW];
    u32x4 xr[XCH];
    auto gload = [&](int st) {
        const uint16_t* xs = xbase + st * BK;                            // uniform
#pragma unroll
        for (int c = 0; c < XCH; ++c) xr[c] = *(const u32x4*)(xs + xoff[c]);
#pragma unroll
        for (int i = 0; i < WPW; ++i) {
            if (wown[i]) {
                const uint8_t* tp = wbase[i] + st * (KS * kTileBytes);  // uniform
                wc[i] = load_nt_u32x4(tp + coff);
                wsc[i] = load_nt_u32x4(sbase[i] + st * (KS * SSTR) + soff);
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < WPW; ++i) {
            if (wown[i]) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const u32x4 v = dequant8<PREC>(wc[i][r], wsc[i][r], nib2, magic);
                    *(u32x4*)&wl[buf][(wrow[i] + r * 16) * STR + wcol[i]] = v;
                }
            }
        }
#pragma unroll
        for (int c = 0; c < XCH; ++c) *(u32x4*)&xl[buf][xdst[c]] = xr[c];
    };

    gload(0);
    lstore(0);
    __syncthreads();
    for (int st = 0; st < NSTAGE; ++st) {
        const int buf = st & 1;
        const bool more = st + 1 < NSTAGE;
        if (more) gload(st + 1);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            frag_t a[FN], b[FT];
#pragma unroll
            for (int i = 0; i < FN; ++i)
                a[i] = *(const frag_t*)&wl[buf][(wn * WN + i * 16 + i16) * STR + kk * 32 + kg * 8];
#pragma unroll
            for (int j = 0; j < FT; ++j)
                b[j] = *(const frag_t*)&xl[buf][(wt * WT + j * 16 + i16) * STR + kk * 32 + kg * 8];
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FT; ++j) acc[i][j] = mfma16(a[i], b[j], acc[i][j]);
        }
        if (more) lstore(buf ^ 1);
        __syncthreads();
    }

    store_tile<FN, FT, PREC == 0>(acc, y, texp, wexp, T, N, t0 + wt * WT, n0 + wn * WN, accum);
}

// ---------------------------------------------------------------------------
// The pipelined variant (default for K % 64 == 0): 256 x 256 workgroup tile,
// 8 waves (2 along N x 4 along T, 128 x 64 wave tiles), 64-K stages.
//   * weights: each wave loads one mx tile (64 rows x 32 K) per stage into
//     registers three stages ahead (three register sets) and dequantizes
//     stage s+1 into the other 16-bit weight buffer during stage s,
//     interleaved with the MFMAs of the stage's second half;
//   * activations: LDS-DMA (global_load_lds_dwordx4) into a 3-deep ring, two
//     stages ahead;
//   * one barrier per stage; every wait names the youngest loads it may
//     leave in flight (vector memory loads retire in issue order).
// The DMA is issued from inline asm: the compiler's wait insertion would
// otherwise assume the DMA may write the fragments read next and wait for it
// right away.
// LDS tiles are planar: [32-K plane][row][32 halves] (64 B rows, 16 KB per
// plane of 256 rows). The 16-byte chunk c of row r sits at chunk slot
// c ^ ((r >> 1) & 3). A fragment access is 16 consecutive rows x one chunk
// per 16 lanes; with this swizzle ds_read_b128 runs conflict-free on gfx950
// (measured 543 B/ns per CU, against 284 with slot c ^ ((r >> 2) & 3), which
// also spreads each 16-lane group over all 64 banks but conflicts between
// the groups the hardware serves together), and every fragment, store and
// DMA address is one base register plus an immediate.
// LDS map: weight buffers at 0 and 32 KB, activation ring at 64, 96, 128 KB.
constexpr int kPlaneB = 256 * 64;                // one 32-K plane of a 256-row tile: 16 KB
constexpr int kTileB = 2 * kPlaneB;              // one 64-K stage of a 256-row tile: 32 KB
constexpr int kXRing = 2 * kTileB;               // LDS offset of the activation ring

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] + vmcnt_hi[15:14], expcnt[6:4], lgkmcnt[11:8]).
constexpr int wait_imm(int vm, int lgkm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (lgkm << 8); }
constexpr int kWaitVm0 = wait_imm(0, 15);
constexpr int kWaitVm6 = wait_imm(6, 15);
constexpr int kWaitVm10 = wait_imm(10, 15);
constexpr int kWaitVm0Lgkm0 = wait_imm(0, 0);
constexpr int kWaitVm4Lgkm0 = wait_imm(4, 0);
constexpr int kWaitVm6Lgkm0 = wait_imm(6, 0);
constexpr int kWaitLgkm0 = wait_imm(63, 0);

// 16 bytes per lane from global memory (uniform base + 32-bit lane offset) into LDS at
// m0 + 16 * lane.
__device__ __forceinline__ void lds_dma16(const void* gbase, uint32_t goff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(goff), "s"(gbase), "s"(lds_base)
                 : "memory", "m0");
}

// The same through a buffer resource: 16 bytes per lane from rsrc's base + soff + voff into
// LDS at m0 + 16 * lane. A lane whose voff is past the resource's num_records reads zeros
// (the buffer range check), with no memory access.
__device__ __forceinline__ void lds_dma16_buf(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff,
                                              uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff),
                 "s"(lds_base)
                 : "memory", "m0");
}
constexpr uint32_t kPadOffset = 0x80000000u;   // past the gather resource's range: a zero row
constexpr int kBufferWord3 = 0x00020000;       // raw buffer resource, 32-bit data format

// 16 bytes per lane into registers (uniform base + 32-bit lane offset). The compiler does not
// track this load: the caller waits for it (s_waitcnt vmcnt) and then passes the registers
// through vgpr_landed before any other use. No non-temporal hint: every weight tile is read
// by each token tile's workgroup, and kept in the caches it costs less (measured at T = 2048,
// gate/up 224 -> 216 us per call; the chip is at its power limit here, so bytes fetched from
// HBM rather than the MALL show up as time).
__device__ __forceinline__ void load16_async(u32x4& dst, const void* gbase, uint32_t goff) {
    asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(dst) : "v"(goff), "s"(gbase) : "memory");
}

// Workgroup b of a launch runs on XCD b % 8. xcd_group maps the b-th of `count` workgroups
// to the tile index that gives each XCD a contiguous run of tiles (count % 8 == 0; else the
// identity): with the token tile fastest in tile order, an XCD's CUs then work on a few row
// tiles across all token tiles, so a weight tile is fetched once per XCD and shared in its
// L2, instead of once per token tile across all XCDs (T = 2048 gate/up: 216 -> 209 us).
__device__ __forceinline__ int xcd_group(int b, int count) {
    return count % 8 ? b : (b % 8) * (count / 8) + b / 8;
}
__device__ __forceinline__ void vgpr_landed(u32x4& v) { asm volatile("" : "+v"(v)); }

// One output tile of the pipelined kernel: 32 * FN weight rows from n0 x 256 tokens from
// 256 * bt, K split `split` of `splits` (split s covers stages [st0, st0 + NST) of K / 64 and
// writes its partial sums to y + s * T * N; the host sums the splits in order).
// FN = 8: 256 rows, 128x64 wave tiles. FN = 6: 192 rows, 96x64 wave tiles, with the 256-row
// tile's loads, DMA and dequant unchanged: the waves of row group 3 load row group 2's mx
// tile again and store it to LDS rows 192..255, which no fragment reads, so every wave
// issues the same loads and the wait counts below hold for both.
// Invariant: every wave issues the same loads, DMA, dequant, waits and barriers in every
// stage. Wave w's loads and dequant fill row group w & 3, K block w >> 2 of the shared weight
// buffer for all waves; its DMA copies token rows [32 w, 32 w + 32) of the stage; its wait
// counts cover only its own loads. Only a wave's fragment reads and MFMAs are private (its
// accumulators reach memory only for its tokens [64 (w >> 1), +64) below T).
// GATHER: x16 is a row-major 16-bit matrix of K columns instead of the pre-tiled image, and
// tile row s (token slot 256 bt + s) is DMA'd from its row gmap[256 bt + s] (gmap null: row
// 256 bt + s itself) through a buffer resource over x16. A padding slot (a negative entry, or
// a slot at or past T, the tile's valid end) gets a lane offset past the resource's range, so
// its LDS row is zeros and no memory is read: its products feed only that slot's
// accumulators, which are never stored, and zero operands spare the MFMAs' power. Each lane
// fetches the 16-byte chunk that its LDS slot holds under the swizzle, so the LDS image is
// the pre-tiled one's. The token exponents (PREC 0) are then indexed by source row too:
// texp[gmap[s]].
template <int PREC, int FN, bool SWI = false, bool GATHER = false>
__device__ __forceinline__ void dma_tile(uint8_t* lds, const uint8_t* __restrict__ packed,
                                         const uint16_t* __restrict__ x16, const int* __restrict__ texp,
                                         const int* __restrict__ wexp, const uint32_t* __restrict__ s16,
                                         float* __restrict__ y, int T, int N, int K, int n0, int bt, int split,
                                         int splits, int accum, const int* __restrict__ gmap = nullptr) {
    static_assert(FN == 8 || FN == 6, "256- or 192-row tiles");
    static_assert(!SWI || FN == 8, "the SwiGLU epilogue pairs a 256-row tile's gate and up halves");
    constexpr int WN = 16 * FN, WT = 64, FT = WT / 16, RG = FN / 2;
    typedef typename std::conditional<PREC == 0, f16x8, bf16x8>::type frag_t;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 1, wt = wave >> 1;
    const int t0 = bt * 256;
    const int KB = K >> 5, NSTK = KB >> 1;
    const int st0 = (int)((int64_t)split * NSTK / splits), NST = (int)((int64_t)(split + 1) * NSTK / splits) - st0;
    y += (int64_t)split * T * N;
    const int G = N >> 6;
    const int i16 = lane & 15, kg = lane >> 4;
    const uint32_t lane_row = i16 * 64 + ((kg ^ ((i16 >> 1) & 3)) << 4);   // row i16, chunk kg, swizzled

    // weights: this wave's mx tile of each stage (row group wave & 3, 32-K block wave >> 2)
    const int rgl = wave & 3, kbl = wave >> 2;
    const int rg = min(n0 / 64 + min(rgl, RG - 1), G - 1);              // clamp ragged N
    const uint8_t* const wsrc = packed + ((int64_t)rg * KB + kbl + 2 * st0) * kTileBytes;
    // scale words: PREC 0 from the fp16 side plane (256 B per tile), PREC 1 from the tile
    constexpr int SSTR = PREC == 0 ? 256 : kTileBytes;
    const uint8_t* const ssrc = PREC == 0 ? (const uint8_t*)s16 + ((int64_t)rg * KB + kbl + 2 * st0) * 256
                                          : wsrc + kCodeBytes;
    const uint32_t coff = lane * 16, soff = i16 * 16;
    const uint32_t wst = kbl * kPlaneB + rgl * 64 * 64 + lane_row;     // + buffer + r * 1 KB

    // activations: pre-tiled as the LDS image of each stage (32 KB contiguous per token tile
    // and stage, zero-padded to whole tiles); this wave copies its 32 rows as 4 DMAs of 1 KB.
    const uint8_t* const xsrc = (const uint8_t*)x16 + (((int64_t)bt * NSTK + st0) * kTileB + wave * 32 * 64);
    const uint32_t xoff = lane * 16;
    const uint32_t xdst = (uint32_t)(uintptr_t)lds + kXRing + wave * 32 * 64;   // LDS byte address
    // GATHER: the byte offset of this lane's chunk in its two token rows (rows 32 w + 16 h +
    // lane / 4 of the tile; LDS slot lane & 3 holds chunk (lane & 3) ^ ((lane >> 3) & 3))
    uint32_t goff[2] = {0u, 0u};
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void*)x16, 0, (int)(kPadOffset - 1),
                                                                         kBufferWord3);   // GATHER only
    if constexpr (GATHER) {
        const uint32_t chunk = (uint32_t)((lane & 3) ^ ((lane >> 3) & 3)) * 16;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int slot = t0 + wave * 32 + h * 16 + (lane >> 2);
            const int r = slot >= T ? -1 : gmap ? gmap[slot] : slot;
            goff[h] = r < 0 ? kPadOffset : (uint32_t)r * (uint32_t)(2 * K) + chunk;
        }
    }

    // fragment bases: A = weight rows wn*128 + 16i + i16, B = token rows wt*64 + 16j + i16
    const uint32_t abase = (wn * WN) * 64 + lane_row;
    const uint32_t bbase = kXRing + (wt * WT) * 64 + lane_row;
    const uint32_t bbase2 = bbase + 2 * kTileB;                         // ring slot 2 (offset > 64 KB)
    const uint32_t nib2 = vgpr_const(kNib2);
    const uint32_t magic = vgpr_const(PREC == 0 ? kMagic1024 : kMagic128);

    f32x4 acc[FN][FT];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 wc[3], ws[3];                          // three register sets of weight codes + scales
    auto issue_x = [&](int st, int slot) {
        const uint32_t dst = xdst + slot * kTileB;
        if constexpr (GATHER) {
            const uint32_t col = (uint32_t)(st0 + st) * 128;   // uniform: columns 64 (st0 + st)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk)
                    lds_dma16_buf(xrs, goff[h], col + kk * 64, dst + kk * kPlaneB + h * 1024);
        } else {
            const uint8_t* src = xsrc + (int64_t)st * kTileB;           // uniform
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk)
                    lds_dma16(src + kk * kPlaneB + h * 1024, xoff, dst + kk * kPlaneB + h * 1024);
        }
    };
    auto issue_w = [&](int st, u32x4& c, u32x4& sc) {
        load16_async(c, wsrc + st * (2 * kTileBytes), coff);           // uniform bases
        load16_async(sc, ssrc + st * (2 * SSTR), soff);
    };
    auto store_w = [&](int buf, const u32x4& c, const u32x4& sc, int r0, int r1) {
#pragma unroll
        for (int r = r0; r < r1; ++r)
            *(u32x4*)(lds + wst + buf * kTileB + r * 1024) = dequant8<PREC>(c[r], sc[r], nib2, magic);
    };
    auto read_frags = [&](int buf, int slot, int kk, frag_t (&a)[FN], frag_t (&b)[FT]) {
        const uint8_t* xp = lds + (slot == 2 ? bbase2 : bbase + slot * kTileB) + kk * kPlaneB;
        const uint8_t* wp = lds + abase + buf * kTileB + kk * kPlaneB;
#pragma unroll
        for (int j = 0; j < FT; ++j) b[j] = *(const frag_t*)(xp + j * 1024);
#pragma unroll
        for (int i = 0; i < FN; ++i) a[i] = *(const frag_t*)(wp + i * 1024);
    };
    auto mfmas = [&](const frag_t (&a)[FN], const frag_t (&b)[FT]) {
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FT; ++j) acc[i][j] = mfma16(a[i], b[j], acc[i][j]);
    };

    // Issue order: stage s's weights two stages before its activations (W(s+3) and X(s+2) at
    // the start of stage s), so the in-order vmcnt lets each wait name the youngest loads it
    // may leave in flight. Prologue: W(0), W(1), X(0), W(2), X(1).
    issue_w(0, wc[0], ws[0]);
    if (NST > 1) issue_w(1, wc[1], ws[1]);
    issue_x(0, 0);
    if (NST > 2) issue_w(2, wc[2], ws[2]);
    if (NST > 1) issue_x(1, 1);
    if (NST > 2) __builtin_amdgcn_s_waitcnt(kWaitVm6);        // W(0), W(1), X(0) landed
    else __builtin_amdgcn_s_waitcnt(kWaitVm0);
    vgpr_landed(wc[0]);
    vgpr_landed(ws[0]);
    store_w(0, wc[0], ws[0], 0, 4);
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    asm volatile("s_barrier" ::: "memory");

    // Stage st, phase P = st % 6: weights in buffer P & 1, activations in ring slot P % 3.
    // Start: wait for W(st+1) (issued at the start of stage st-2); W(st+3) -> register set
    // P % 3 (W(st)'s, dequantized in stage st-1); X(st+2) -> slot (P+2) % 3 (X(st-1)'s,
    // released by the barrier that ended stage st-1). The dequantization of W(st+1) into the
    // other weight buffer is spread over both halves of the MFMAs: an MFMA hides about two
    // independent VALU instructions, not more. End: wait for X(st+1) and the LDS stores,
    // barrier.
    auto stage = [&](auto phase, int st) {
        constexpr int P = decltype(phase)::value;
        constexpr int cur = P & 1, slot = P % 3, nslot = (P + 2) % 3, wset = P % 3, nset = (P + 1) % 3;
        const bool w3 = st + 3 < NST, x2 = st + 2 < NST;
        if (x2) __builtin_amdgcn_s_waitcnt(kWaitVm10);        // W(st+1) landed
        else __builtin_amdgcn_s_waitcnt(kWaitVm0);
        vgpr_landed(wc[nset]);
        vgpr_landed(ws[nset]);
        if (w3) issue_w(st + 3, wc[wset], ws[wset]);
        if (x2) issue_x(st + 2, nslot);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            frag_t a[FN], b[FT];
            read_frags(cur, slot, kk, a, b);
            store_w(cur ^ 1, wc[nset], ws[nset], 2 * kk, 2 * kk + 2);   // rows 16r.., r in [2kk, 2kk+2)
            mfmas(a, b);
            __builtin_amdgcn_sched_group_barrier(0x100, FN + FT, 0);
#pragma unroll
            for (int g = 0; g < 20; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
            }
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, FN * FT - 22, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (w3) __builtin_amdgcn_s_waitcnt(kWaitVm6Lgkm0);    // X(st+1) landed, LDS stores done
        else if (x2) __builtin_amdgcn_s_waitcnt(kWaitVm4Lgkm0);
        else __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);
        asm volatile("s_barrier" ::: "memory");
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    using I4 = std::integral_constant<int, 4>;
    using I5 = std::integral_constant<int, 5>;
    int st = 0;
    for (; st + 6 <= NST; st += 6) {
        stage(I0{}, st);
        stage(I1{}, st + 1);
        stage(I2{}, st + 2);
        stage(I3{}, st + 3);
        stage(I4{}, st + 4);
        stage(I5{}, st + 5);
    }
    if (st < NST) stage(I0{}, st);
    if (st + 1 < NST) stage(I1{}, st + 1);
    if (st + 2 < NST) stage(I2{}, st + 2);
    if (st + 3 < NST) stage(I3{}, st + 3);
    if (st + 4 < NST) stage(I4{}, st + 4);

    // gathered activations carry their exponents by source row
    const int* tmap = GATHER ? gmap : nullptr;
    if constexpr (SWI)
        store_swiglu<FT, PREC == 0>(acc, (uint16_t*)y, texp, wexp, T, N, t0 + wt * WT, n0 + wn * WN, tmap);
    else
        store_tile<FN, FT, PREC == 0>(acc, y, texp, wexp, T, N, t0 + wt * WT, n0 + wn * WN, accum, tmap);
}

// Workgroups [0, wide_wgs) take the 256-row tiles of rows [0, narrow_row0), the rest the
// 192-row tiles from narrow_row0 on (token tile fastest, then K split innermost). The longer
// tiles come first in dispatch order, so the shorter ones fill the CUs the last round of
// long tiles leaves idle. MIXED = false: 256-row tiles only (wide_wgs = the grid), an
// instance without the 192-row body.
template <int PREC, bool MIXED>
__global__ __launch_bounds__(512) void prefill_dma_kernel(const uint8_t* __restrict__ packed,
                                                          const uint16_t* __restrict__ x16,
                                                          const int* __restrict__ texp, const int* __restrict__ wexp,
                                                          const uint32_t* __restrict__ s16, float* __restrict__ y,
                                                          int T, int N, int K, int tiles_t, int splits, int wide_wgs,
                                                          int narrow_row0, int accum) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[5 * kTileB];
    const int G = (int)gridDim.x, wide = MIXED ? wide_wgs : G;
    const int b = (int)blockIdx.x < wide ? xcd_group((int)blockIdx.x, wide)
                                         : wide + xcd_group((int)blockIdx.x - wide, G - wide);
    if (!MIXED || b < wide_wgs) {
        const int tile = b / splits;
        dma_tile<PREC, 8>(lds, packed, x16, texp, wexp, s16, y, T, N, K, (tile / tiles_t) * 256, tile % tiles_t,
                          b % splits, splits, accum);
    } else {
        const int i = b - wide_wgs, tile = i / splits;
        dma_tile<PREC, 6>(lds, packed, x16, texp, wexp, s16, y, T, N, K, narrow_row0 + (tile / tiles_t) * 192,
                          tile % tiles_t, i % splits, splits, accum);
    }
}

// The gate/up GEMM with the SwiGLU epilogue: workgroup b takes the 256-row tile of pair rows
// (b / tiles_t) * 256 and token tile b % tiles_t over all of K (no split), writing h.
template <int PREC>
__global__ __launch_bounds__(512) void prefill_swiglu_kernel(const uint8_t* __restrict__ packed,
                                                             const uint16_t* __restrict__ x16,
                                                             const int* __restrict__ texp,
                                                             const int* __restrict__ wexp,
                                                             const uint32_t* __restrict__ s16,
                                                             uint16_t* __restrict__ h, int T, int N, int K,
                                                             int tiles_t) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[5 * kTileB];
    const int b = xcd_group((int)blockIdx.x, (int)gridDim.x);
    dma_tile<PREC, 8, true>(lds, packed, x16, texp, wexp, s16, (float*)h, T, N, K, (b / tiles_t) * 256, b % tiles_t,
                            0, 1, 0);
}

// The exponent that puts a positive finite magnitude v in [2^14, 2^15) after scaling by
// 2^-e: v in [2^(x-1), 2^x) -> e = x - 15. 0 for zero, inf and NaN (those are passed
// through unscaled).
__device__ __forceinline__ int fp16_fit_exponent(float v) {
    if (!(v > 0.0f) || v > 3.0e38f) return 0;
    int x;
    frexpf(v, &x);
    return x - 15;
}

// Activations -> the MFMA's 16-bit type, one workgroup per token row (padded to whole
// token tiles). PREC 0: fp16, token row t scaled by 2^-s_t with s_t = fp16_fit_exponent(max
// |x_t|), and texp[t] = s_t. PREC 1: bf16 (RNE from f32), no exponents.
// TILED: the 16-byte chunk i (k = 8i..8i+7) of token t goes to its place in the LDS image
// of the pipelined kernel's activation tiles: [token tile][64-K stage][32-K plane][256 rows]
// [4 chunks], chunk c of row r at slot c ^ ((r >> 1) & 3). Each stage of a token tile is then
// one contiguous 32 KB block, copied to LDS verbatim. Otherwise rows stay [T][K].
__device__ __forceinline__ int64_t xchunk_dst(int t, int i, int K) {
    const int r = t & 255, st = i >> 3, kk = (i >> 2) & 1, c = i & 3;
    return ((((int64_t)(t >> 8) * (K >> 6) + st) * 2 + kk) * 256 + r) * 4 + (c ^ ((r >> 1) & 3));
}

// Block-wide max of a non-negative value over 256 threads (result in every thread).
__device__ __forceinline__ float block_max256(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// The prefill scales of an [N, K] mx matrix, in two launches over (row group g, chunk c of
// kScaleChunk 32-K blocks) workgroups, each of 64 rows x 4 parts (thread (part, row) takes
// blocks part, part + 4, ... of the chunk):
//   max pass:   cmax[n][c] = max over the chunk's blocks of 15 |d| + |m| for row n;
//   write pass: wexp[n] = fp16_fit_exponent(max over c of cmax[n][c]) (chunk 0 stores it),
//               s16 word (g KB + kb) * 64 + (n % 16) * 4 + (n % 64) / 16 = fp16(d 2^-e) << 16 |
//               fp16(m 2^-e), the mx scale block's word order.
constexpr int kScaleChunk = 32;

__device__ __forceinline__ const uint8_t* scale_word_base(const uint8_t* packed, int64_t g, int KB, int row) {
    return packed + g * KB * kTileBytes + kCodeBytes + ((row & 15) * 4 + (row >> 4)) * 4;
}

__global__ __launch_bounds__(256) void prefill_scale_max_kernel(const uint8_t* __restrict__ packed, int K, int nchunk,
                                                                float* __restrict__ cmax) {
    __shared__ float red[4][64];
    const int64_t g = blockIdx.x / nchunk;
    const int c = blockIdx.x % nchunk, row = threadIdx.x & 63, part = threadIdx.x >> 6;
    const int KB = K >> 5, kb0 = c * kScaleChunk, kb1 = min(kb0 + kScaleChunk, KB);
    const uint8_t* base = scale_word_base(packed, g, KB, row);
    float b = 0.f;
#pragma unroll 8
    for (int kb = kb0 + part; kb < kb1; kb += 4) {
        const uint32_t sw = load_global<uint32_t>(base + (int64_t)kb * kTileBytes);
        b = fmaxf(b, __builtin_fmaf(15.0f, fabsf(bf16_hi_to_f32(sw)), fabsf(bf16_lo_to_f32(sw))));
    }
    red[part][row] = b;
    __syncthreads();
    if (part == 0)
        cmax[(g * 64 + row) * nchunk + c] = fmaxf(fmaxf(red[0][row], red[1][row]), fmaxf(red[2][row], red[3][row]));
}

__global__ __launch_bounds__(256) void prefill_scale_write_kernel(const uint8_t* __restrict__ packed, int K,
                                                                  int nchunk, const float* __restrict__ cmax,
                                                                  int* __restrict__ wexp, uint32_t* __restrict__ s16) {
    const int64_t g = blockIdx.x / nchunk;
    const int c = blockIdx.x % nchunk, row = threadIdx.x & 63, part = threadIdx.x >> 6;
    const int KB = K >> 5, kb0 = c * kScaleChunk, kb1 = min(kb0 + kScaleChunk, KB);
    const float* cm = cmax + (g * 64 + row) * nchunk;
    float m = 0.f;
    for (int i = 0; i < nchunk; ++i) m = fmaxf(m, cm[i]);
    const int e = fp16_fit_exponent(m);
    if (c == 0 && part == 0) wexp[g * 64 + row] = e;
    const uint8_t* base = scale_word_base(packed, g, KB, row);
    uint32_t* out = s16 + g * KB * 64 + ((row & 15) * 4 + (row >> 4));
#pragma unroll 8
    for (int kb = kb0 + part; kb < kb1; kb += 4) {
        const uint32_t sw = load_global<uint32_t>(base + (int64_t)kb * kTileBytes);
        const uint32_t dh = __builtin_bit_cast(uint16_t, (_Float16)ldexpf(bf16_hi_to_f32(sw), -e));
        const uint32_t mh = __builtin_bit_cast(uint16_t, (_Float16)ldexpf(bf16_lo_to_f32(sw), -e));
        out[(int64_t)kb * 64] = (dh << 16) | mh;
    }
}

// lo_pass (f32 activations, PREC 0): the fp16 remainder x 2^-s - fp16(x 2^-s) instead of the
// rounded value; the two passes' products add up to the f32 activations' to ~2^-22.
// One token row of prefill_xprep (all 256 threads): ld8(i, v) loads the row's 8-element
// group i as f32 (zero: a padding row, written as zeros). F32SRC: the source is f32, so the
// lo pass of PREC 0 writes the fp16 remainder. HELD: 8-element groups per thread kept in
// registers between the max and the conversion (0: ld8 is called twice, for a row in LDS).
template <bool F32SRC, int PREC, bool TILED, int HELD = 8, class Load>
__device__ __forceinline__ void xprep_row(Load ld8, bool zero, uint16_t* __restrict__ x16, int* __restrict__ texp,
                                          int t, int K, int lo_pass) {
    const int n8 = K >> 3;                       // 8-element groups of the row (K % 32 == 0)
    const int64_t row = (int64_t)t * K;
    u32x4* const out = (u32x4*)x16;
    auto dst = [&](int i) -> int64_t { return TILED ? xchunk_dst(t, i, K) : row / 8 + i; };
    if (zero) {
        for (int i = threadIdx.x; i < n8; i += 256) out[dst(i)] = u32x4{0u, 0u, 0u, 0u};
        return;
    }
    // Rows of up to 256 HELD chunks (K <= 16384 for the default) are read once and held in
    // registers for both the max and the conversion; longer rows are read twice.
    constexpr int kHeld = HELD > 0 ? HELD : 1;
    const bool held = HELD > 0 && n8 <= 256 * HELD;
    float hv[kHeld][8];
    if (held) {
#pragma unroll
        for (int c = 0; c < kHeld; ++c) {
            const int i = threadIdx.x + 256 * c;
            if (i < n8) ld8(i, hv[c]);
        }
    }
    int s = 0;
    if constexpr (PREC == 0) {
        __shared__ float red[4];
        float mx = 0.f;
        if (held) {
#pragma unroll
            for (int c = 0; c < kHeld; ++c)
                if (threadIdx.x + 256 * c < n8) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(hv[c][e]));
                }
        } else {
            for (int i = threadIdx.x; i < n8; i += 256) {
                float v[8];
                ld8(i, v);
#pragma unroll
                for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[e]));
            }
        }
        s = fp16_fit_exponent(block_max256(mx, red));
        if (threadIdx.x == 0) texp[t] = s;
    }
    auto cvt8 = [&](const float (&v)[8]) -> u32x4 {
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint32_t lo, hi;
            if constexpr (PREC == 0) {
                const float a = ldexpf(v[2 * e], -s), b = ldexpf(v[2 * e + 1], -s);
                _Float16 ha = (_Float16)a, hb = (_Float16)b;
                if (F32SRC && lo_pass) {
                    ha = (_Float16)(a - (float)ha);
                    hb = (_Float16)(b - (float)hb);
                }
                lo = __builtin_bit_cast(uint16_t, ha);
                hi = __builtin_bit_cast(uint16_t, hb);
            } else {
                lo = f32_to_bf16_rne(v[2 * e]);
                hi = f32_to_bf16_rne(v[2 * e + 1]);
            }
            o[e] = lo | (hi << 16);
        }
        return o;
    };
    if (held) {
#pragma unroll
        for (int c = 0; c < kHeld; ++c) {
            const int i = threadIdx.x + 256 * c;
            if (i < n8) out[dst(i)] = cvt8(hv[c]);
        }
    } else {
        for (int i = threadIdx.x; i < n8; i += 256) {
            float v[8];
            ld8(i, v);
            out[dst(i)] = cvt8(v);
        }
    }
}

// The 8 activations of group i of a row, as f32.
template <bool XF32>
__device__ __forceinline__ void load_x8(const void* __restrict__ xrow, int i, float (&v)[8]) {
    if constexpr (XF32) {
        const f32x4* p = (const f32x4*)xrow + 2 * i;
        const f32x4 a = p[0], b = p[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = a[e], v[e + 4] = b[e];
    } else {
        const u32x4 w = ((const u32x4*)xrow)[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[2 * e] = bf16_lo_to_f32(w[e]), v[2 * e + 1] = bf16_hi_to_f32(w[e]);
    }
}

template <bool XF32, int PREC, bool TILED>
__global__ __launch_bounds__(256) void prefill_xprep(const void* __restrict__ x, uint16_t* __restrict__ x16,
                                                     int* __restrict__ texp, int T, int K, int lo_pass) {
    const int t = blockIdx.x;
    const void* xrow = (const uint8_t*)x + (int64_t)t * K * (XF32 ? 4 : 2);
    xprep_row<XF32, PREC, TILED>([&](int i, float (&v)[8]) { load_x8<XF32>(xrow, i, v); }, t >= T, x16, texp, t,
                                 K, lo_pass);
}

// The RMSNorm producer writing the prefill's prepared activations directly: per token row t
// (one workgroup; rows past T are the tile padding, written as zeros)
//   y  = x + add (f32, stored when y is given; y may be x: the row is read before y is written),
//   xn = bf16((y * r) * w) with r as q4_rmsnorm_add forms it (norm_core.h),
// then xn goes through prefill_xprep's conversion (bf16 source) from an LDS copy of the row.
// The same bits as q4_rmsnorm_add (bf16 xn) followed by q4_prefill_prepare(xn, bf16), with
// one launch and no bf16 row in memory. PER values per thread (K <= 256 PER); extra j terms
// are zeros, which leave the fp64 sum of squares unchanged.
template <int PER, int PREC, bool TILED>
__global__ __launch_bounds__(256) void rmsnorm_prepare_kernel(const float* x, const float* __restrict__ add,
                                                              int add_planes, const void* __restrict__ w, int w_bf16,
                                                              float* y, uint16_t* __restrict__ x16,
                                                              int* __restrict__ texp, int T, int K, float eps) {
    __shared__ double part[4];
    __shared__ __attribute__((aligned(16))) uint16_t xs[256 * PER];
    const int t = blockIdx.x, tid = threadIdx.x;
    if (t < T) {
        const float* xr = x + (int64_t)t * K;
        const float* ar = add ? add + (int64_t)t * K : nullptr;
        const int64_t pstride = (int64_t)T * K;      // plane q of add at add + q T K
        float v[PER], wv[PER];
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int i = tid + 256 * j;
            float a = 0.0f;
            if (ar && i < K) {          // the planes in prefill_reduce_kernel's order
                a = ar[i];
                for (int q = 1; q < add_planes; ++q) a += ar[q * pstride + i];
            }
            v[j] = i < K ? (ar ? xr[i] + a : xr[i]) : 0.0f;
            wv[j] = i >= K ? 0.0f
                           : (w_bf16 ? bf16_hi_to_f32((uint32_t)((const uint16_t*)w)[i] << 16) : ((const float*)w)[i]);
        }
#pragma unroll
        for (int j = 0; j < PER; ++j) ss += (double)v[j] * (double)v[j];
        const double ws = wave_sum_ss(ss);
        if ((tid & 63) == 0) part[tid >> 6] = ws;
        __syncthreads();
        if (y) {
            float* yr = y + (int64_t)t * K;
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const int i = tid + 256 * j;
                if (i < K) yr[i] = v[j];
            }
        }
        const float r = inv_rms(part, K, eps);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int i = tid + 256 * j;
            if (i < K) xs[i] = (uint16_t)f32_to_bf16_rne(v[j] * r * wv[j]);
        }
        __syncthreads();
    }
    xprep_row<false, PREC, TILED, 0>(            // the row sits in LDS: read it there twice
        [&](int i, float (&o)[8]) {
            const u32x4 wd = *(const u32x4*)(xs + 8 * i);
#pragma unroll
            for (int e = 0; e < 4; ++e) o[2 * e] = bf16_lo_to_f32(wd[e]), o[2 * e + 1] = bf16_hi_to_f32(wd[e]);
        },
        t >= T, x16, texp, t, K, 0);
}

// The SwiGLU producer writing the down projection's prepared activations: per token row t
//   h[f] = bf16(silu(g[t][f]) * u[t][f]), silu(g) = g / (1 + exp(-g))
// (the reference's h, moe_batch.h:181-202 mb_silu_tile; the decode kernels' silu), staged
// in LDS and converted as prefill_xprep converts a bf16 row; h is also stored [T][F] when
// h_out is given. g and u are f32 rows with strides ldg / ldu (one fused gate/up output:
// u = g + F, both strides 2F). Rows past T are the tile padding (zeros).
template <int PREC, bool TILED>
__global__ __launch_bounds__(256) void swiglu_prepare_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                             int64_t ldg, int64_t ldu, uint16_t* __restrict__ h_out,
                                                             uint16_t* __restrict__ x16, int* __restrict__ texp,
                                                             int T, int F) {
    __shared__ __attribute__((aligned(16))) uint16_t hs[256 * 64];
    const int t = blockIdx.x, tid = threadIdx.x;
    if (t < T) {
        const float* gr = g + (int64_t)t * ldg;
        const float* ur = u + (int64_t)t * ldu;
        for (int i = 4 * tid; i < F; i += 4 * 256) {
            const f32x4 gv = *(const f32x4*)(gr + i), uv = *(const f32x4*)(ur + i);
            uint32_t o[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const float a = gv[2 * e] / (1.0f + expf(-gv[2 * e])) * uv[2 * e];
                const float b = gv[2 * e + 1] / (1.0f + expf(-gv[2 * e + 1])) * uv[2 * e + 1];
                o[e] = f32_to_bf16_rne(a) | (f32_to_bf16_rne(b) << 16);
            }
            *(uint2*)(hs + i) = make_uint2(o[0], o[1]);
            if (h_out) *(uint2*)(h_out + (int64_t)t * F + i) = make_uint2(o[0], o[1]);
        }
        __syncthreads();
    }
    xprep_row<false, PREC, TILED, 0>(
        [&](int i, float (&o)[8]) {
            const u32x4 wd = *(const u32x4*)(hs + 8 * i);
#pragma unroll
            for (int e = 0; e < 4; ++e) o[2 * e] = bf16_lo_to_f32(wd[e]), o[2 * e + 1] = bf16_hi_to_f32(wd[e]);
        },
        t >= T, x16, texp, t, F, 0);
}

// Kernel variants: (BN, BT, waves along N, waves along T, 32-K blocks per stage).
struct TileCfg {
    int bn, bt, wgn, wgt, ks;
};
constexpr TileCfg kCfgs[] = {
    {256, 256, 2, 4, 2},     // 8 waves, 128x64 wave tiles, 64-K stages
    {256, 128, 2, 4, 2},     // 8 waves, 128x32
    {128, 256, 2, 4, 2},     // 8 waves, 64x64
    {128, 128, 2, 4, 2},     // 8 waves, 64x32
    {256, 256, 2, 2, 1},     // 4 waves, 128x128 wave tiles, 32-K stages
    {256, 256, 2, 4, 2},     // the LDS-DMA pipelined kernel (prefill_dma_kernel)
};
constexpr int kDmaCfg = 5;
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

// Kernel variant: the pipelined kernel whenever K % 64 == 0 (K splits keep small grids
// busy); otherwise the generic variant with the fewest rounds of 256 workgroups
// (Q4MI_PREFILL_CFG overrides).
int choose_cfg(int T, int N, int K) {
    static int forced = [] {
        const char* e = getenv("Q4MI_PREFILL_CFG");
        return e ? atoi(e) : -1;
    }();
    if (forced >= 0 && forced < kNumCfgs && K % (32 * kCfgs[forced].ks) == 0) return forced;
    if (K % 64 == 0) return kDmaCfg;
    const double eff[] = {1.0, 0.9, 0.9, 0.75, 0.8};   // relative per-workgroup efficiency
    double best = 1e300;
    int pick = 4;
    for (int i = 0; i < kDmaCfg; ++i) {
        if (K % (32 * kCfgs[i].ks)) continue;
        const int64_t wgs = ceil_div(N, kCfgs[i].bn) * ceil_div(T, kCfgs[i].bt);
        const int64_t rounds = ceil_div(wgs, 256);
        const double cost = (double)rounds * kCfgs[i].bn * kCfgs[i].bt / eff[i];
        if (cost < best) {
            best = cost;
            pick = i;
        }
    }
    return pick;
}

template <int C, int PREC>
void launch_cfg(int64_t grid, hipStream_t st, const uint8_t* w, const uint16_t* x16, const int* te, const int* we,
                const uint32_t* s16, float* y, int T, int N, int K, int tiles_t, int accum) {
    constexpr TileCfg c = kCfgs[C];
    hipLaunchKernelGGL((prefill_kernel<c.bn, c.bt, c.wgn, c.wgt, c.ks, PREC>), dim3((unsigned)grid),
                       dim3(64 * c.wgn * c.wgt), 0, st, w, x16, te, we, s16, y, T, N, K, tiles_t, accum);
}

template <int PREC>
void launch_prefill(int cfg, int64_t grid, hipStream_t st, const uint8_t* w, const uint16_t* x16, const int* te,
                    const int* we, const uint32_t* s16, float* y, int T, int N, int K, int tiles_t, int splits,
                    int wide_wgs, int narrow_row0, int accum) {
    switch (cfg) {
        case 0: launch_cfg<0, PREC>(grid, st, w, x16, te, we, s16, y, T, N, K, tiles_t, accum); break;
        case 1: launch_cfg<1, PREC>(grid, st, w, x16, te, we, s16, y, T, N, K, tiles_t, accum); break;
        case 2: launch_cfg<2, PREC>(grid, st, w, x16, te, we, s16, y, T, N, K, tiles_t, accum); break;
        case 3: launch_cfg<3, PREC>(grid, st, w, x16, te, we, s16, y, T, N, K, tiles_t, accum); break;
        case 4: launch_cfg<4, PREC>(grid, st, w, x16, te, we, s16, y, T, N, K, tiles_t, accum); break;
        default:
            if (wide_wgs < grid)
                hipLaunchKernelGGL((prefill_dma_kernel<PREC, true>), dim3((unsigned)grid), dim3(512), 0, st, w, x16, te,
                                   we, s16, y, T, N, K, tiles_t, splits, wide_wgs, narrow_row0, accum);
            else
                hipLaunchKernelGGL((prefill_dma_kernel<PREC, false>), dim3((unsigned)grid), dim3(512), 0, st, w, x16, te,
                                   we, s16, y, T, N, K, tiles_t, splits, wide_wgs, narrow_row0, accum);
            break;
    }
}

// y = sum of the S partials in split order (deterministic), 4 floats per thread; accum adds
// it to what y holds.
__global__ __launch_bounds__(256) void prefill_reduce_kernel(const f32x4* __restrict__ part, f32x4* __restrict__ y,
                                                             int64_t MN4, int S, int accum) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= MN4) return;
    f32x4 s = part[i];
    for (int q = 1; q < S; ++q) s += part[(int64_t)q * MN4 + i];
    y[i] = accum ? y[i] + s : s;
}

// CUs of the current device (the MI355X's 256 when no device is visible, e.g. for a
// workspace query on a host without a GPU).
int device_cus() {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
            (void)hipGetLastError();
            return 256;
        }
        return n;
    }();
    return cus;
}

// Launch plan of one prefill GEMM: the kernel variant, its token tiles and K splits, and for
// the pipelined kernel the rows covered by 256-row tiles ([0, narrow_row0), wide_wgs
// workgroups) and by 192-row tiles (the rest). That kernel holds one workgroup per CU (160 KB
// of LDS). Two levers fit its work to the CUs: a K split (partial sums reduced in order
// afterwards) and 192-row tiles, which fill the CUs the last round of 256-row tiles leaves
// idle without any partial traffic (Llama-3-8B gate_up at T = 2048: 448 tiles of 256 rows
// run in 2 rounds of 256 CUs; 256 of 256 rows + 256 of 192 rows in 1 + 3/4). 192-row
// strips also cover N % 256 != 0 without repeating rows.
// Q4MI_PREFILL_SPLITS and Q4MI_PREFILL_NARROW (the count of 192-row strips) override.
struct PrefillPlan {
    int cfg, tiles_t, splits, wide_wgs, narrow_row0;
    int64_t grid;
};

// Finish time of A units of cost cw followed by B units of cost cn when each starts on the
// earliest free of C CUs (workgroups dispatch in index order, one per CU).
double makespan(int64_t A, int64_t B, int64_t C, double cw, double cn) {
    const int64_t q = A / C, r = A % C;
    const double wide_end = (double)(q + (r ? 1 : 0)) * cw;
    if (B == 0) return wide_end;
    double t[2] = {(double)q * cw, (double)(q + 1) * cw};   // C - r CUs free at t[0], r at t[1]
    const int64_t cnt[2] = {C - r, r};
    double last = 0;
    for (int64_t left = B; left > 0;) {
        const int g = (cnt[1] > 0 && t[1] < t[0]) ? 1 : 0;
        last = t[g];
        left -= cnt[g];
        t[g] += cn;
    }
    return last + cn > wide_end ? last + cn : wide_end;
}

PrefillPlan make_plan_uncached(int T, int64_t N, int64_t K) {
    PrefillPlan p;
    p.cfg = choose_cfg(T, (int)N, (int)K);
    p.tiles_t = (int)ceil_div(T, kCfgs[p.cfg].bt);
    int64_t tiles = ceil_div(N, kCfgs[p.cfg].bn) * p.tiles_t;
    p.splits = 1;
    p.wide_wgs = (int)tiles;
    p.narrow_row0 = (int)N;
    if (p.cfg == kDmaCfg) {
        static const int forced = [] {
            const char* e = getenv("Q4MI_PREFILL_SPLITS");
            return e ? atoi(e) : 0;
        }();
        static const int forced_narrow = [] {
            const char* e = getenv("Q4MI_PREFILL_NARROW");
            return e ? atoi(e) : -1;
        }();
        // kNarrowRel: a 192-row tile's time relative to a 256-row tile's over the same stages,
        // measured: gate_up at T = 2048 took 236.6 us as 2 rounds of 256-row tiles and 224.9 us
        // as 1 round of each, so the 192-row round ran at ~0.9 of a 256-row one.
        constexpr double kStageSec = 1.0e-6, kReduceBytesPerSec = 4.0e12, kNarrowRel = 0.9;
        const int nst = (int)(K / 64), cap = nst < 16 ? nst : 16;
        const int64_t G = N / 64, tt = p.tiles_t;
        const int cus = device_cus();
        // a forced strip count is used only where it fits: 3b <= G and 4 | G - 3b
        const int64_t fb = forced_narrow > 0 && 3 * (int64_t)forced_narrow <= G &&
                                   (G - 3 * (int64_t)forced_narrow) % 4 == 0
                               ? forced_narrow
                               : forced_narrow == 0 ? 0 : -1;
        double best = 1e300;
        // b 192-row strips and a 256-row strips with 4a + 3b = G (b = 0: 256-row strips only,
        // the last one clamped when G % 4 != 0). 192-row tiles only fill the last round of
        // 256-row ones, so at most two rounds of them are considered.
        for (int64_t b = 0; 3 * b <= G && (b * tt <= 2 * cus || b == fb); ++b) {
            if (b > 0 && (G - 3 * b) % 4) continue;
            if (fb >= 0 && b != fb) continue;
            const int64_t a = b > 0 ? (G - 3 * b) / 4 : ceil_div(G, 4);
            for (int S = 1; S <= cap; ++S) {
                if (forced > 0 && S != (forced < cap ? forced : cap)) continue;
                if (b > 0 && b != fb && b * tt * S > 2 * cus) break;
                const double cw = (double)ceil_div(nst, S) * kStageSec;
                double cost = makespan(a * tt * S, b * tt * S, cus, cw, cw * kNarrowRel);
                if (S > 1) cost += (double)(S + 1) * T * N * 4 / kReduceBytesPerSec;
                // ties: fewer rows computed (a clamped last 256-row strip repeats rows)
                cost += 1e-12 * (double)(256 * a + 192 * b);
                if (cost < best) {
                    best = cost;
                    p.splits = S;
                    p.wide_wgs = (int)(a * tt * S);
                    p.narrow_row0 = b > 0 ? (int)(256 * a) : (int)N;
                    tiles = (a + b) * tt;
                }
            }
        }
    }
    p.grid = tiles * p.splits;
    return p;
}

// The plans of the last few shapes per host thread (the workspace query and the call that
// follows it plan the same shape).
PrefillPlan make_plan(int T, int64_t N, int64_t K) {
    struct Entry {
        int T;
        int64_t N, K;
        PrefillPlan p;
    };
    thread_local Entry cache[4] = {};
    thread_local int next = 0;
    for (const Entry& e : cache)
        if (e.T == T && e.N == N && e.K == K && T > 0) return e.p;
    const PrefillPlan p = make_plan_uncached(T, N, K);
    cache[next] = Entry{T, N, K, p};
    next = (next + 1) & 3;
    return p;
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

template <bool XF, int PR, bool TL>
void launch_xprep_t(dim3 g, hipStream_t st, const void* x, uint16_t* x16, int* te, int T, int K, int lo_pass) {
    hipLaunchKernelGGL((prefill_xprep<XF, PR, TL>), g, dim3(256), 0, st, x, x16, te, T, K, lo_pass);
}

void launch_xprep(bool xf32, int prec, bool tiled, dim3 g, hipStream_t st, const void* x, uint16_t* x16, int* te,
                  int T, int K, int lo_pass) {
    typedef void (*fn_t)(dim3, hipStream_t, const void*, uint16_t*, int*, int, int, int);
    static const fn_t table[8] = {launch_xprep_t<false, 0, false>, launch_xprep_t<false, 0, true>,
                                  launch_xprep_t<false, 1, false>, launch_xprep_t<false, 1, true>,
                                  launch_xprep_t<true, 0, false>,  launch_xprep_t<true, 0, true>,
                                  launch_xprep_t<true, 1, false>,  launch_xprep_t<true, 1, true>};
    table[(xf32 ? 4 : 0) + (prec ? 2 : 0) + (tiled ? 1 : 0)](g, st, x, x16, te, T, K, lo_pass);
}

}  // namespace

// Activation rows are padded with zeros to a multiple of 256 tokens (the widest token tile).
static size_t padded_tokens(int T) { return ((size_t)T + 255) / 256 * 256; }

// The prefill scales of an [N, K] matrix: wexp int32[N], then the fp16 scale plane (4 bytes
// per row and 32-K block), then the max pass's per-chunk maxima (f32 [N][chunks]).
static int64_t scale_chunks(int64_t K) { return ceil_div(K / 32, kScaleChunk); }
static size_t scales_wexp_bytes(int64_t N) { return align256((size_t)N * 4); }
static size_t scales_plane_bytes(int64_t N, int64_t K) { return align256((size_t)N * (K / 32) * 4); }
static size_t scales_bytes(int64_t N, int64_t K) {
    return scales_wexp_bytes(N) + scales_plane_bytes(N, K) + align256((size_t)N * scale_chunks(K) * 4);
}

extern "C" size_t q4_prefill_scales_bytes(int64_t N, int64_t K) {
    if (N <= 0 || K <= 0 || N % 64 || K % 32) return 0;
    return scales_bytes(N, K);
}

extern "C" int q4_prefill_scales(const uint8_t* packed, int64_t N, int64_t K, void* scales, size_t scales_bytes_,
                                 void* stream) {
    if (N < 0 || K <= 0 || N % 64 || K % 32) return Q4MI_E_SHAPE;
    if (N > 0x7FFFFFFF || K > 0x7FFFFFFF) return Q4MI_E_RANGE;
    if (N == 0) return Q4MI_OK;
    if (!packed || !scales || misaligned16(packed) || misaligned16(scales)) return Q4MI_E_ARG;
    if (scales_bytes_ < scales_bytes(N, K)) return Q4MI_E_WORKSPACE;
    int* wexp = (int*)scales;
    uint32_t* s16 = (uint32_t*)((char*)scales + scales_wexp_bytes(N));
    float* cmax = (float*)((char*)s16 + scales_plane_bytes(N, K));
    const int nchunk = (int)scale_chunks(K);
    const dim3 grid((unsigned)((N / 64) * nchunk));
    const hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(prefill_scale_max_kernel, grid, dim3(256), 0, st, packed, (int)K, nchunk, cmax);
    if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
    hipLaunchKernelGGL(prefill_scale_write_kernel, grid, dim3(256), 0, st, packed, (int)K, nchunk,
                       (const float*)cmax, wexp, s16);
    return launch_status();
}

// Workspace of the GEMM proper: activations in the kernel's 16-bit layout, the token
// exponents, and the K-split partial sums when the plan splits K.
static size_t x16_bytes(int T, int64_t K) { return align256(padded_tokens(T) * K * 2); }
static size_t xprep_bytes(int T, int64_t K) { return x16_bytes(T, K) + align256((size_t)T * 4); }
static size_t gemm_ws_bytes(int T, int64_t N, int64_t K) {
    const PrefillPlan p = make_plan(T, N, K);
    return xprep_bytes(T, K) + (p.splits > 1 ? align256((size_t)p.splits * T * N * 4) : 0);
}

extern "C" size_t q4_gemm_prefill_scaled_workspace_bytes(int T, int64_t N, int64_t K) {
    if (T <= 0 || K <= 0 || N < 0 || N % 64 || K % 32) return 0;
    return gemm_ws_bytes(T, N, K);
}

// q4_gemm_prefill's workspace also holds the matrix's prefill scales (precision 0).
extern "C" size_t q4_gemm_prefill_workspace_bytes(int T, int64_t N, int64_t K) {
    if (T <= 0 || K <= 0 || N < 0 || N % 64 || K % 32) return 0;
    return gemm_ws_bytes(T, N, K) + scales_bytes(N, K);
}

namespace {

// The GEMM with the matrix's prefill scales (precision 0) given; workspace of gemm_ws_bytes.
// One GEMM pass over activation plane x16 (exponents te): pass 0 writes y, later passes add
// their products to it (f32 activations' remainder). part: the split partials, when the plan
// splits K; the in-order reduce then writes (or adds to) y.
int gemm_pass(const uint8_t* packed, const void* scales, const uint16_t* x16, const int* te, float* y, int T,
              int64_t N, int64_t K, int precision, float* part, int pass, hipStream_t st) {
    const int* we = precision == 0 ? (const int*)scales : nullptr;
    const uint32_t* s16 = precision == 0 ? (const uint32_t*)((const char*)scales + scales_wexp_bytes(N)) : nullptr;
    const PrefillPlan plan = make_plan(T, N, K);
    float* out = plan.splits > 1 ? part : y;
    const int accum = plan.splits > 1 ? 0 : pass;
    if (precision == 0)
        launch_prefill<0>(plan.cfg, plan.grid, st, packed, x16, te, we, s16, out, T, (int)N, (int)K, plan.tiles_t,
                          plan.splits, plan.wide_wgs, plan.narrow_row0, accum);
    else
        launch_prefill<1>(plan.cfg, plan.grid, st, packed, x16, nullptr, nullptr, nullptr, out, T, (int)N, (int)K,
                          plan.tiles_t, plan.splits, plan.wide_wgs, plan.narrow_row0, accum);
    if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
    if (plan.splits > 1) {
        const int64_t MN4 = (int64_t)T * N / 4;
        hipLaunchKernelGGL(prefill_reduce_kernel, dim3((unsigned)ceil_div(MN4, 256)), dim3(256), 0, st,
                           (const f32x4*)out, (f32x4*)y, MN4, plan.splits, pass);
        if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
    }
    return Q4MI_OK;
}

// f32 activations in precision 0 take two passes: their fp16 rounding, then the fp16
// remainder, whose product the second pass adds to y.
int activation_passes(int x_dtype, int precision) { return x_dtype == Q4MI_F32 && precision == 0 ? 2 : 1; }

// The GEMM with the matrix's prefill scales (precision 0) given; workspace of gemm_ws_bytes:
// one activation plane, prepared and consumed pass by pass.
int prefill_impl(const uint8_t* packed, const void* scales, const void* x, int x_dtype, float* y, int T, int64_t N,
                 int64_t K, int precision, void* workspace, hipStream_t st) {
    uint16_t* x16 = (uint16_t*)workspace;
    int* te = (int*)((char*)workspace + x16_bytes(T, K));
    float* part = (float*)((char*)workspace + xprep_bytes(T, K));
    const bool tiled = make_plan(T, N, K).cfg == kDmaCfg;
    for (int pass = 0; pass < activation_passes(x_dtype, precision); ++pass) {
        launch_xprep(x_dtype == Q4MI_F32, precision, tiled, dim3((unsigned)padded_tokens(T)), st, x, x16, te, T,
                     (int)K, pass);
        if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
        const int rc = gemm_pass(packed, scales, x16, te, y, T, N, K, precision, part, pass, st);
        if (rc != Q4MI_OK) return rc;
    }
    return launch_status();
}

int prefill_args(const uint8_t* packed, const void* x, int x_dtype, float* y, int T, int64_t N, int64_t K,
                 void* workspace) {
    if (x_dtype != Q4MI_F32 && x_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (T < 0 || N < 0 || K <= 0 || N % 64 || K % 32) return Q4MI_E_SHAPE;
    if (N > 0x7FFFFFFF || K > 0x7FFFFFFF) return Q4MI_E_RANGE;
    if (T == 0 || N == 0) return 1;                              // nothing to compute
    if (!packed || !x || !y) return Q4MI_E_ARG;
    if (misaligned16(packed) || misaligned16(x) || misaligned16(y) || misaligned16(workspace)) return Q4MI_E_ARG;
    return Q4MI_OK;
}

}  // namespace

extern "C" int q4_gemm_prefill(const uint8_t* packed, const void* x, int x_dtype, float* y, int T, int64_t N,
                               int64_t K, int precision, void* workspace, size_t workspace_bytes, void* stream) {
    if (precision != 0 && precision != 1) return Q4MI_E_ARG;
    const int a = prefill_args(packed, x, x_dtype, y, T, N, K, workspace);
    if (a != Q4MI_OK) return a > 0 ? Q4MI_OK : a;
    if (!workspace || workspace_bytes < q4_gemm_prefill_workspace_bytes(T, N, K)) return Q4MI_E_WORKSPACE;
    const hipStream_t st = (hipStream_t)stream;
    void* scales = (char*)workspace + gemm_ws_bytes(T, N, K);
    if (precision == 0) {
        const int rc = q4_prefill_scales(packed, N, K, scales, scales_bytes(N, K), stream);
        if (rc != Q4MI_OK) return rc;
    }
    return prefill_impl(packed, scales, x, x_dtype, y, T, N, K, precision, workspace, st);
}

extern "C" int q4_gemm_prefill_scaled(const uint8_t* packed, const void* scales, const void* x, int x_dtype, float* y,
                                      int T, int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
                                      void* stream) {
    const int a = prefill_args(packed, x, x_dtype, y, T, N, K, workspace);
    if (a != Q4MI_OK) return a > 0 ? Q4MI_OK : a;
    if (!scales || misaligned16(scales)) return Q4MI_E_ARG;
    if (!workspace || workspace_bytes < gemm_ws_bytes(T, N, K)) return Q4MI_E_WORKSPACE;
    return prefill_impl(packed, scales, x, x_dtype, y, T, N, K, 0, workspace, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// Prepared activations: the pre-pass on its own, so a producer's output is converted once
// and read by several projections (gate and up of an FFN, Q, K and V), or written in this
// layout by the producer itself. Layout: the activation planes of the GEMM's passes (two for
// f32 x in precision 0: value and remainder), each x16_bytes(T, K), then the token exponents.
// The pipelined kernel's tiled image when K % 64 == 0, else rows [T][K].
// ---------------------------------------------------------------------------
namespace {
size_t prepared_bytes(int T, int64_t K, int x_dtype, int precision) {
    return (size_t)activation_passes(x_dtype, precision) * x16_bytes(T, K) + align256((size_t)T * 4);
}
}  // namespace

extern "C" size_t q4_prefill_prepared_bytes(int T, int64_t K, int x_dtype, int precision) {
    if (T <= 0 || K <= 0 || K % 32 || (x_dtype != Q4MI_F32 && x_dtype != Q4MI_BF16) || (precision != 0 && precision != 1))
        return 0;
    return prepared_bytes(T, K, x_dtype, precision);
}

extern "C" int q4_prefill_prepare(const void* x, int x_dtype, int T, int64_t K, int precision, void* prepared,
                                  size_t prepared_bytes_, void* stream) {
    if (precision != 0 && precision != 1) return Q4MI_E_ARG;
    if (x_dtype != Q4MI_F32 && x_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (T < 0 || K <= 0 || K % 32) return Q4MI_E_SHAPE;
    if (K > 0x7FFFFFFF) return Q4MI_E_RANGE;
    if (T == 0) return Q4MI_OK;
    if (!x || !prepared || misaligned16(x) || misaligned16(prepared)) return Q4MI_E_ARG;
    if (prepared_bytes_ < prepared_bytes(T, K, x_dtype, precision)) return Q4MI_E_WORKSPACE;
    const int passes = activation_passes(x_dtype, precision);
    int* te = (int*)((char*)prepared + passes * x16_bytes(T, K));
    for (int pass = 0; pass < passes; ++pass) {
        launch_xprep(x_dtype == Q4MI_F32, precision, K % 64 == 0, dim3((unsigned)padded_tokens(T)),
                     (hipStream_t)stream, x, (uint16_t*)((char*)prepared + pass * x16_bytes(T, K)), te, T, (int)K,
                     pass);
        if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
    }
    return Q4MI_OK;
}

extern "C" int q4_rmsnorm_prepare(const float* x, const float* add, int add_planes, const void* w, int w_dtype,
                                  float* y, int T, int64_t K, float eps, int precision, void* prepared,
                                  size_t prepared_bytes_, void* stream) {
    if (precision != 0 && precision != 1) return Q4MI_E_ARG;
    if (add_planes < 0 || add_planes > 64 || (add_planes > 0) != (add != nullptr)) return Q4MI_E_ARG;
    if (w_dtype != Q4MI_F32 && w_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (T < 0 || K <= 0 || K % 32) return Q4MI_E_SHAPE;
    if (K > 256 * 64) return Q4MI_E_RANGE;
    if (!(eps >= 0.0f)) return Q4MI_E_ARG;
    if (T == 0) return Q4MI_OK;
    if (!x || !w || !prepared || misaligned16(prepared)) return Q4MI_E_ARG;
    const size_t need = prepared_bytes(T, K, Q4MI_BF16, precision);
    if (prepared_bytes_ < need) return Q4MI_E_WORKSPACE;
    // y may be x itself, but no output may overlap another argument otherwise
    auto overlaps = [](const void* a, size_t na, const void* b, size_t nb) {
        const char *ca = (const char*)a, *cb = (const char*)b;
        return a && b && ca < cb + nb && cb < ca + na;
    };
    const size_t row_bytes = (size_t)T * K * 4, add_bytes = row_bytes * (size_t)add_planes;
    if (overlaps(prepared, need, x, row_bytes) || overlaps(prepared, need, add, add_bytes) ||
        overlaps(prepared, need, y, row_bytes) ||
        overlaps(prepared, need, w, (size_t)K * (w_dtype == Q4MI_BF16 ? 2 : 4)) ||
        (y != x && overlaps(y, row_bytes, x, row_bytes)) || overlaps(y, row_bytes, add, add_bytes))
        return Q4MI_E_ARG;
    uint16_t* x16 = (uint16_t*)prepared;
    int* te = (int*)((char*)prepared + x16_bytes(T, K));
    const dim3 grid((unsigned)padded_tokens(T)), block(256);
    const hipStream_t st = (hipStream_t)stream;
    const int wb = w_dtype == Q4MI_BF16;
    const bool tiled = K % 64 == 0, small = K <= 256 * 16;
#define Q4MI_RP(PER, PR, TL)                                                                                   \
    hipLaunchKernelGGL((rmsnorm_prepare_kernel<PER, PR, TL>), grid, block, 0, st, x, add, add_planes, w, wb, y, x16, \
                       te, T, (int)K, eps)
    if (precision == 0) {
        if (small) { if (tiled) Q4MI_RP(16, 0, true); else Q4MI_RP(16, 0, false); }
        else { if (tiled) Q4MI_RP(64, 0, true); else Q4MI_RP(64, 0, false); }
    } else {
        if (small) { if (tiled) Q4MI_RP(16, 1, true); else Q4MI_RP(16, 1, false); }
        else { if (tiled) Q4MI_RP(64, 1, true); else Q4MI_RP(64, 1, false); }
    }
#undef Q4MI_RP
    return launch_status();
}

extern "C" int q4_swiglu_prepare(const float* g, const float* u, int64_t ldg, int64_t ldu, int T, int64_t F,
                                 int precision, void* h, void* prepared, size_t prepared_bytes_, void* stream) {
    if (precision != 0 && precision != 1) return Q4MI_E_ARG;
    if (T < 0 || F <= 0 || F % 32 || ldg < F || ldu < F || ldg % 4 || ldu % 4) return Q4MI_E_SHAPE;
    if (F > 256 * 64) return Q4MI_E_RANGE;
    if (T == 0) return Q4MI_OK;
    if (!g || !u || !prepared || misaligned16(g) || misaligned16(u) || misaligned16(prepared) || misaligned16(h))
        return Q4MI_E_ARG;
    const size_t need = prepared_bytes(T, F, Q4MI_BF16, precision);
    if (prepared_bytes_ < need) return Q4MI_E_WORKSPACE;
    auto overlaps = [](const void* a, size_t na, const void* b, size_t nb) {
        const char *ca = (const char*)a, *cb = (const char*)b;
        return a && b && ca < cb + nb && cb < ca + na;
    };
    const size_t gb = ((size_t)(T - 1) * ldg + F) * 4, ub = ((size_t)(T - 1) * ldu + F) * 4, hb = (size_t)T * F * 2;
    if (overlaps(prepared, need, g, gb) || overlaps(prepared, need, u, ub) || overlaps(h, hb, g, gb) ||
        overlaps(h, hb, u, ub) || overlaps(h, hb, prepared, need))
        return Q4MI_E_ARG;
    uint16_t* x16 = (uint16_t*)prepared;
    int* te = (int*)((char*)prepared + x16_bytes(T, F));
    const dim3 grid((unsigned)padded_tokens(T)), block(256);
    const hipStream_t st = (hipStream_t)stream;
    const bool tiled = F % 64 == 0;
#define Q4MI_SP(PR, TL)                                                                                          \
    hipLaunchKernelGGL((swiglu_prepare_kernel<PR, TL>), grid, block, 0, st, g, u, ldg, ldu, (uint16_t*)h, x16, te, \
                       T, (int)F)
    if (precision == 0) { if (tiled) Q4MI_SP(0, true); else Q4MI_SP(0, false); }
    else { if (tiled) Q4MI_SP(1, true); else Q4MI_SP(1, false); }
#undef Q4MI_SP
    return launch_status();
}

extern "C" int q4_gemm_prefill_swiglu(const uint8_t* gate_up, const void* scales, const void* prepared, int x_dtype,
                                      void* h, int T, int64_t F, int64_t K, int precision, void* stream) {
    if (precision != 0 && precision != 1) return Q4MI_E_ARG;
    if (x_dtype != Q4MI_F32 && x_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (activation_passes(x_dtype, precision) != 1) return Q4MI_E_ARG;   // f32 x in precision 0: two passes
    if (T < 0 || F <= 0 || K <= 0 || F % 128 || K % 64) return Q4MI_E_SHAPE;
    if (2 * F > 0x7FFFFFFF || K > 0x7FFFFFFF) return Q4MI_E_RANGE;
    if (T == 0) return Q4MI_OK;
    if (!gate_up || !prepared || !h || misaligned16(gate_up) || misaligned16(prepared) || misaligned16(h))
        return Q4MI_E_ARG;
    if (precision == 0 && (!scales || misaligned16(scales))) return Q4MI_E_ARG;
    const int64_t N = 2 * F;
    const int* we = precision == 0 ? (const int*)scales : nullptr;
    const uint32_t* s16 = precision == 0 ? (const uint32_t*)((const char*)scales + scales_wexp_bytes(N)) : nullptr;
    const int* te = (const int*)((const char*)prepared + x16_bytes(T, K));
    const int tiles_t = (int)ceil_div(T, 256);
    const dim3 grid((unsigned)((N / 256) * tiles_t)), block(512);
    const hipStream_t st = (hipStream_t)stream;
    if (precision == 0)
        hipLaunchKernelGGL(prefill_swiglu_kernel<0>, grid, block, 0, st, gate_up, (const uint16_t*)prepared, te, we,
                           s16, (uint16_t*)h, T, (int)N, (int)K, tiles_t);
    else
        hipLaunchKernelGGL(prefill_swiglu_kernel<1>, grid, block, 0, st, gate_up, (const uint16_t*)prepared, nullptr,
                           nullptr, nullptr, (uint16_t*)h, T, (int)N, (int)K, tiles_t);
    return launch_status();
}

extern "C" size_t q4_gemm_prefill_prepared_workspace_bytes(int T, int64_t N, int64_t K) {
    if (T <= 0 || K <= 0 || N < 0 || N % 64 || K % 32) return 0;
    const PrefillPlan p = make_plan(T, N, K);
    return p.splits > 1 ? align256((size_t)p.splits * T * N * 4) : 0;
}

extern "C" int q4_gemm_prefill_prepared(const uint8_t* packed, const void* scales, const void* prepared, int x_dtype,
                                        float* y, int T, int64_t N, int64_t K, int precision, void* workspace,
                                        size_t workspace_bytes, void* stream) {
    if (precision != 0 && precision != 1) return Q4MI_E_ARG;
    const int a = prefill_args(packed, prepared, x_dtype, y, T, N, K, workspace);
    if (a != Q4MI_OK) return a > 0 ? Q4MI_OK : a;
    if (precision == 0 && (!scales || misaligned16(scales))) return Q4MI_E_ARG;
    const PrefillPlan plan = make_plan(T, N, K);
    if ((plan.cfg == kDmaCfg) != (K % 64 == 0)) return Q4MI_E_ARG;   // a forced generic variant reads rows
    if (plan.splits > 1 && (!workspace || workspace_bytes < q4_gemm_prefill_prepared_workspace_bytes(T, N, K)))
        return Q4MI_E_WORKSPACE;
    const int passes = activation_passes(x_dtype, precision);
    const int* te = (const int*)((const char*)prepared + passes * x16_bytes(T, K));
    for (int pass = 0; pass < passes; ++pass) {
        const uint16_t* x16 = (const uint16_t*)((const char*)prepared + pass * x16_bytes(T, K));
        const int rc = gemm_pass(packed, scales, x16, te, y, T, N, K, precision, (float*)workspace, pass,
                                 (hipStream_t)stream);
        if (rc != Q4MI_OK) return rc;
    }
    return Q4MI_OK;
}

extern "C" int q4_prefill_split_count(int T, int64_t N, int64_t K) {
    if (T <= 0 || N <= 0 || K <= 0 || N % 64 || K % 32) return 0;
    return make_plan(T, N, K).splits;
}

extern "C" int q4_gemm_prefill_prepared_partials(const uint8_t* packed, const void* scales, const void* prepared,
                                                 int x_dtype, float* part, size_t part_bytes, int T, int64_t N,
                                                 int64_t K, int precision, void* stream) {
    if (precision != 0 && precision != 1) return Q4MI_E_ARG;
    if (activation_passes(x_dtype, precision) != 1) return Q4MI_E_ARG;   // f32 x in precision 0: two passes
    const int a = prefill_args(packed, prepared, x_dtype, part, T, N, K, nullptr);
    if (a != Q4MI_OK) return a > 0 ? Q4MI_OK : a;
    if (precision == 0 && (!scales || misaligned16(scales))) return Q4MI_E_ARG;
    const PrefillPlan plan = make_plan(T, N, K);
    if ((plan.cfg == kDmaCfg) != (K % 64 == 0)) return Q4MI_E_ARG;
    // the planes this call writes follow this process's plan, not a count queried elsewhere
    if (part_bytes < (size_t)plan.splits * T * N * sizeof(float)) return Q4MI_E_WORKSPACE;
    const int* te = (const int*)((const char*)prepared + x16_bytes(T, K));
    const int* we = precision == 0 ? (const int*)scales : nullptr;
    const uint32_t* s16 = precision == 0 ? (const uint32_t*)((const char*)scales + scales_wexp_bytes(N)) : nullptr;
    const hipStream_t st = (hipStream_t)stream;
    // plane s of the K split at part + s T N (one plane, the whole product, when unsplit)
    if (precision == 0)
        launch_prefill<0>(plan.cfg, plan.grid, st, packed, (const uint16_t*)prepared, te, we, s16, part, T, (int)N,
                          (int)K, plan.tiles_t, plan.splits, plan.wide_wgs, plan.narrow_row0, 0);
    else
        launch_prefill<1>(plan.cfg, plan.grid, st, packed, (const uint16_t*)prepared, nullptr, nullptr, nullptr, part, T,
                          (int)N, (int)K, plan.tiles_t, plan.splits, plan.wide_wgs, plan.narrow_row0, 0);
    return launch_status();
}

// ---------------------------------------------------------------------------
// Routed MoE at prefill scale: out[t] = sum_j w[t][j] down_e(silu(gate_e x_t) (up_e x_t)).
//
// The reference batches an expert's tokens into slots and runs them through its expert
// GEMM dispatch by dispatch (moe_batch.h:98-172, a host loop over dispatches in
// Core::moe_block, core.cpp:5163-5178). Here the batching is on the device and the expert
// GEMMs are the pipelined prefill tiles (dma_tile) over all experts in one launch each:
//   1. route (one workgroup): tokens per expert from an LDS histogram of ids; expert e's
//      slots are [off_e, off_e + n_e), padded to whole 256-token tiles, experts in
//      ascending order; per tile its expert and the end of that expert's slots.
//   2. slots (a workgroup per expert): the pairs routed to e, in pair order, get the slots
//      off_e, off_e + 1, ...; slot -> token row (pads -1) and pair -> slot.
//   3. the token rows gathered into the slots in the GEMM's tiled 16-bit layout (pads 0);
//   4. gate/up: workgroup (tile, 256-row tile) runs dma_tile on expert e's [2F, H] matrix
//      into G[slot][2F] (f32);
//   5. h = silu(g) u from G (gate and up row groups alternate), into the 16-bit layout;
//   6. down: as 4 on the [H, F] matrices into Y[slot][H];
//   7. combine: out[t] = sum_j w[t][j] Y[slot(t, j)] in slot order j.
// Precision 0 (fp16 tiles with power-of-two scaling, the matrices' prefill scales given)
// takes f32 activations and h in two passes (fp16 value + remainder), as q4_gemm_prefill
// does; precision 1 (the reference's bf16 tile, RNE(q d + m)) rounds x and h to bf16, as
// the reference's moe_batch rounds h (moe_batch.h:181-202). A token row's result does not
// depend on its slot (MFMA rows are independent), and the combine sums in slot order, so
// results are deterministic.
// ---------------------------------------------------------------------------
namespace {

constexpr int kMoePfMaxExperts = 8192;
constexpr int64_t kMoePfMaxPairs = (int64_t)1 << 22;

__global__ __launch_bounds__(1024) void moe_route_kernel(const int32_t* __restrict__ ids, int P, int E,
                                                         int* __restrict__ cnt, int* __restrict__ off,
                                                         int* __restrict__ tile_e, int* __restrict__ tile_end,
                                                         int* __restrict__ meta) {
    __shared__ int hist[kMoePfMaxExperts];
    __shared__ int wsum[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int e = tid; e < E; e += 1024) hist[e] = 0;
    __syncthreads();
    constexpr int kR = 8;                           // ids per thread in flight together
    for (int p0 = 0; p0 < P; p0 += 1024 * kR) {
        int ev[kR];
#pragma unroll
        for (int j = 0; j < kR; ++j) {
            const int p = p0 + tid + 1024 * j;
            ev[j] = p < P ? ids[p] : -1;
        }
#pragma unroll
        for (int j = 0; j < kR; ++j)
            if (ev[j] >= 0 && ev[j] < E) atomicAdd(&hist[ev[j]], 1);
    }
    __syncthreads();
    const int per = (E + 1023) / 1024;               // experts per thread, consecutive
    int tiles = 0;
    for (int j = 0; j < per; ++j) {
        const int e = tid * per + j;
        if (e < E) tiles += (hist[e] + 255) >> 8;
    }
    int incl = tiles;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o);
        if (lane >= o) incl += v;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int tp = incl - tiles;
    for (int w = 0; w < wave; ++w) tp += wsum[w];
    for (int j = 0; j < per; ++j) {
        const int e = tid * per + j;
        if (e >= E) break;
        const int n = hist[e], nt = (n + 255) >> 8;
        cnt[e] = n;
        off[e] = tp * 256;
        for (int i = 0; i < nt; ++i) {
            tile_e[tp + i] = e;
            tile_end[tp + i] = tp * 256 + n;
        }
        tp += nt;
    }
    if (tid == 1023) meta[0] = tp;
}

// A workgroup barrier for LDS only: this wave's LDS operations are complete, its global
// stores may still be in flight (__syncthreads would also wait for those).
__device__ __forceinline__ void lds_sync() {
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    asm volatile("s_barrier" ::: "memory");
}

// Expert e's pairs, in pair order, take slots off[e], off[e] + 1, ...: slot_of_pair and the
// slot -> token row map (padding slots -1). A batch is 4096 pairs: thread t holds the 16
// consecutive ids [16 t, 16 t + 16) in registers (four 16-byte loads, issued together), so
// a block-wide prefix sum of the per-thread counts orders the matches; only the waves' sums
// go through LDS, and the slot stores are never waited for inside the loop.
__global__ __launch_bounds__(256) void moe_slots_kernel(const int32_t* __restrict__ ids, int P, int topk,
                                                        const int* __restrict__ cnt, const int* __restrict__ off,
                                                        int* __restrict__ slot_of_pair, int* __restrict__ rowmap) {
    constexpr int kPer = 16, kBatch = 256 * kPer;
    __shared__ int wsum[2][4];
    const int e = blockIdx.x, n = cnt[e];
    if (n == 0) return;
    const int o = off[e];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool vec = ((uintptr_t)ids & 15) == 0;    // 16-byte loads of ids
    int base = 0;                                   // slots given out before this batch
    for (int b0 = 0, par = 0; b0 < P && base < n; b0 += kBatch, par ^= 1) {
        const int i0 = b0 + tid * kPer;
        int iv[kPer];
        if (vec && i0 + kPer <= P) {
#pragma unroll
            for (int q = 0; q < kPer / 4; ++q) {
                const int4 v = *(const int4*)(ids + i0 + 4 * q);
                iv[4 * q] = v.x, iv[4 * q + 1] = v.y, iv[4 * q + 2] = v.z, iv[4 * q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < kPer; ++j) iv[j] = i0 + j < P ? ids[i0 + j] : -1;
        }
        int c = 0;
#pragma unroll
        for (int j = 0; j < kPer; ++j) c += iv[j] == e;
        int incl = c;
#pragma unroll
        for (int sft = 1; sft < 64; sft <<= 1) {
            const int v = __shfl_up(incl, sft);
            if (lane >= sft) incl += v;
        }
        if (lane == 63) wsum[par][wave] = incl;     // two sets: no barrier needed before reuse
        lds_sync();
        int r = base + incl - c;
        for (int w = 0; w < wave; ++w) r += wsum[par][w];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            if (iv[j] == e) {
                const int p = i0 + j;
                slot_of_pair[p] = o + r;
                rowmap[o + r] = p / topk;
                ++r;
            }
        }
        base += wsum[par][0] + wsum[par][1] + wsum[par][2] + wsum[par][3];
    }
    const int pad = ((n + 255) >> 8) << 8;
    for (int i = n + tid; i < pad; i += 256) rowmap[o + i] = -1;
}

// One slot row per wave (4 per workgroup) of the MoE activation preps: xprep_row's
// conversion with the row max reduced within the wave. ld8(i, v) loads 8-element group i
// of the row as f32; zero writes a padding row. Rows of up to 512 groups (K <= 4096) are
// held in registers, longer ones read twice.
template <bool F32SRC, int PREC, class Load>
__device__ __forceinline__ void xprep_row_wave(Load ld8, bool zero, uint16_t* __restrict__ x16,
                                               int* __restrict__ texp, int t, int K, int lo_pass) {
    const int n8 = K >> 3, lane = threadIdx.x & 63;
    u32x4* const out = (u32x4*)x16;
    if (zero) {
        for (int i = lane; i < n8; i += 64) out[xchunk_dst(t, i, K)] = u32x4{0u, 0u, 0u, 0u};
        return;
    }
    constexpr int kHeld = 8;
    const bool held = n8 <= 64 * kHeld;
    float hv[kHeld][8];
    if (held) {
#pragma unroll
        for (int c = 0; c < kHeld; ++c) {
            const int i = lane + 64 * c;
            if (i < n8) ld8(i, hv[c]);
        }
    }
    int s = 0;
    if constexpr (PREC == 0) {
        float mx = 0.f;
        if (held) {
#pragma unroll
            for (int c = 0; c < kHeld; ++c)
                if (lane + 64 * c < n8) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(hv[c][e]));
                }
        } else {
            for (int i = lane; i < n8; i += 64) {
                float v[8];
                ld8(i, v);
#pragma unroll
                for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[e]));
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        s = fp16_fit_exponent(mx);
        if (lane == 0) texp[t] = s;
    }
    auto cvt8 = [&](const float (&v)[8]) -> u32x4 {
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint32_t lo, hi;
            if constexpr (PREC == 0) {
                const float a = ldexpf(v[2 * e], -s), b = ldexpf(v[2 * e + 1], -s);
                _Float16 ha = (_Float16)a, hb = (_Float16)b;
                if (F32SRC && lo_pass) {
                    ha = (_Float16)(a - (float)ha);
                    hb = (_Float16)(b - (float)hb);
                }
                lo = __builtin_bit_cast(uint16_t, ha);
                hi = __builtin_bit_cast(uint16_t, hb);
            } else {
                lo = f32_to_bf16_rne(v[2 * e]);
                hi = f32_to_bf16_rne(v[2 * e + 1]);
            }
            o[e] = lo | (hi << 16);
        }
        return o;
    };
    if (held) {
#pragma unroll
        for (int c = 0; c < kHeld; ++c) {
            const int i = lane + 64 * c;
            if (i < n8) out[xchunk_dst(t, i, K)] = cvt8(hv[c]);
        }
    } else {
        for (int i = lane; i < n8; i += 64) {
            float v[8];
            ld8(i, v);
            out[xchunk_dst(t, i, K)] = cvt8(v);
        }
    }
}

template <bool XF32, int PREC>
__global__ __launch_bounds__(256) void moe_xprep_kernel(const void* __restrict__ x, const int* __restrict__ rowmap,
                                                        const int* __restrict__ meta, uint16_t* __restrict__ x16,
                                                        int* __restrict__ texp, int K, int lo_pass) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= meta[0] * 256) return;
    const int row = rowmap[t];
    const void* xrow = (const uint8_t*)x + (int64_t)(row < 0 ? 0 : row) * K * (XF32 ? 4 : 2);
    xprep_row_wave<XF32, PREC>([&](int i, float (&v)[8]) { load_x8<XF32>(xrow, i, v); }, row < 0, x16, texp, t, K,
                               lo_pass);
}

// h[f] = silu(g[f]) u[f] of slot t from G[t][2F], where the 64 gate rows of row group j are
// columns 128 j .. 128 j + 63 and its up rows the next 64. HB16 (PREC 0): h rounded to bf16
// first (the reference's h, moe_batch.h:181-202), so the fp16 tile takes it in one pass.
template <int PREC, bool HB16 = false>
__global__ __launch_bounds__(256) void moe_hprep_kernel(const float* __restrict__ G, const int* __restrict__ rowmap,
                                                        const int* __restrict__ meta, uint16_t* __restrict__ x16,
                                                        int* __restrict__ texp, int F, int lo_pass) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= meta[0] * 256) return;
    const float* g = G + (int64_t)t * 2 * F;
    auto ld8 = [&](int i, float (&v)[8]) {
        const int f = 8 * i, c = (f >> 6) * 128 + (f & 63);
        const f32x4 g0 = *(const f32x4*)(g + c), g1 = *(const f32x4*)(g + c + 4);
        const f32x4 u0 = *(const f32x4*)(g + c + 64), u1 = *(const f32x4*)(g + c + 68);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = g0[e] / (1.0f + expf(-g0[e])) * u0[e];
            v[e + 4] = g1[e] / (1.0f + expf(-g1[e])) * u1[e];
        }
        if constexpr (HB16) {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = bf16_hi_to_f32(f32_to_bf16_rne(v[e]) << 16);
        }
    };
    xprep_row_wave<!HB16, PREC>(ld8, rowmap[t] < 0, x16, texp, t, F, lo_pass);
}

// Slot t's bf16 h row (from the gate/up GEMM's SwiGLU epilogue, h[S][F]) into down's 16-bit
// layout; pad slots (rowmap < 0) as zeros.
template <int PREC>
__global__ __launch_bounds__(256) void moe_h16prep_kernel(const uint16_t* __restrict__ h,
                                                          const int* __restrict__ rowmap, const int* __restrict__ meta,
                                                          uint16_t* __restrict__ x16, int* __restrict__ texp, int F) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= meta[0] * 256) return;
    const uint16_t* hrow = h + (int64_t)t * F;
    xprep_row_wave<false, PREC>([&](int i, float (&v)[8]) { load_x8<false>(hrow, i, v); }, rowmap[t] < 0, x16, texp,
                                t, F, 0);
}

// Workgroup (token tile tt, 256-row tile rt) of a grouped expert GEMM: dma_tile on tile tt's
// expert's matrix (N rows, ebytes each expert), slots [256 tt, tile_end) valid. GATHER: x16
// is row-major ([rows][K]), slot s's row gmap[s] (gmap null: row s).
template <int PREC, bool SWI = false, bool GATHER = false>
__global__ __launch_bounds__(512) void moe_dma_kernel(const uint8_t* __restrict__ packed, int64_t ebytes,
                                                      const uint16_t* __restrict__ x16,
                                                      const int* __restrict__ texp, const int* __restrict__ wexp,
                                                      const uint32_t* __restrict__ s16, int64_t s16_words,
                                                      float* __restrict__ y, const int* __restrict__ tile_e,
                                                      const int* __restrict__ tile_end, const int* __restrict__ meta,
                                                      int N, int K, int tiles_n, int accum,
                                                      const int* __restrict__ gmap = nullptr) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[5 * kTileB];
    const int b = blockIdx.x, tt = b / tiles_n, rt = b % tiles_n;
    if (tt >= meta[0]) return;
    const int e = tile_e[tt];
    dma_tile<PREC, 8, SWI, GATHER>(lds, packed + e * ebytes, x16, texp, PREC == 0 ? wexp + (int64_t)e * N : nullptr,
                                   PREC == 0 ? s16 + e * s16_words : nullptr, y, tile_end[tt], N, K, rt * 256, tt, 0,
                                   1, accum, gmap);
}

// out[t][n..n+3] = sum_j w[t][j] Y[slot(t, j)][n..n+3], slot order j.
__global__ __launch_bounds__(256) void moe_prefill_combine_kernel(const float* __restrict__ Y,
                                                                  const int* __restrict__ slot_of_pair,
                                                                  const int32_t* __restrict__ ids,
                                                                  const float* __restrict__ w, int topk, int E,
                                                                  int H, float* __restrict__ out) {
    const int64_t t = blockIdx.y, n = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (n >= H) return;
    // the token's ids, weights and slots first, then all its Y loads, then the sum in slot
    // order j (topk <= 16): no load waits on the previous slot's
    constexpr int kMaxK = 16;
    int slot[kMaxK];
    float wv[kMaxK];
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
        const int64_t p = t * topk + j;
        const int e = j < topk ? ids[p] : -1;
        const bool ok = e >= 0 && e < E;
        slot[j] = ok ? slot_of_pair[p] : -1;
        wv[j] = ok ? w[p] : 0.f;
    }
    f32x4 v[kMaxK];
#pragma unroll
    for (int j = 0; j < kMaxK; ++j)
        if (slot[j] >= 0) v[j] = *(const f32x4*)(Y + (int64_t)slot[j] * H + n);
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < kMaxK; ++j)
        if (slot[j] >= 0) {
#pragma unroll
            for (int c = 0; c < 4; ++c) s[c] += wv[j] * v[j][c];
        }
    *(f32x4*)(out + t * H + n) = s;
}

struct MoePfWs {
    size_t cnt, off, meta, tile_e, tile_end, sop, rowmap, texp, x16, gy, total;
    int64_t tiles_max;
};

// Workspace layout for T tokens x topk over E experts (slots: every tile an expert could use).
MoePfWs moe_pf_ws(int T, int E, int topk, int64_t H, int64_t F) {
    MoePfWs w{};
    const int64_t P = (int64_t)T * topk;
    w.tiles_max = ceil_div(P, 256) + (E < P ? E : P);
    const size_t S = (size_t)w.tiles_max * 256;
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o += align256(bytes);
        return at;
    };
    w.cnt = take((size_t)E * 4);
    w.off = take((size_t)E * 4);
    w.meta = take(16);
    w.tile_e = take((size_t)w.tiles_max * 4);
    w.tile_end = take((size_t)w.tiles_max * 4);
    w.sop = take((size_t)P * 4);
    w.rowmap = take(S * 4);
    w.texp = take(S * 4);
    const size_t x16a = S * H * 2, x16b = 2 * S * F * 2;
    w.x16 = take(x16a > x16b ? x16a : x16b);       // x, then h (value and remainder planes)
    w.gy = take(S * (2 * F > H ? 2 * F : H) * 4);  // G, then Y
    w.total = o;
    return w;
}

}  // namespace

extern "C" size_t q4_moe_prefill_workspace_bytes(int T, int E, int topk, int H, int F) {
    if (T <= 0 || E <= 0 || topk <= 0 || H <= 0 || F <= 0) return 0;
    return moe_pf_ws(T, E, topk, H, F).total;
}

extern "C" int q4_moe_prefill(const uint8_t* gate_up, const uint8_t* down, const void* gate_up_scales,
                              const void* down_scales, const void* x, int x_dtype, const int32_t* topk_ids,
                              const float* topk_w, float* out, int T, int E, int topk, int64_t H, int64_t F,
                              int precision, void* workspace, size_t workspace_bytes, void* stream) {
    if (precision < 0 || precision > 2) return Q4MI_E_ARG;
    // precision 2: the fp16 tile of precision 0 with h rounded to bf16 (one down pass)
    const bool hb16 = precision != 0;
    precision = precision == 2 ? 0 : precision;
    if (x_dtype != Q4MI_F32 && x_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (H <= 0 || F <= 0 || H % 256 || F % 128) return Q4MI_E_SHAPE;
    if (H > (1 << 20) || F > (1 << 20)) return Q4MI_E_RANGE;
    if (T < 0 || E <= 0 || E > kMoePfMaxExperts || topk <= 0 || topk > 16 || (int64_t)T * topk > kMoePfMaxPairs)
        return Q4MI_E_RANGE;
    if (T == 0) return Q4MI_OK;
    if (!gate_up || !down || !x || !topk_ids || !topk_w || !out) return Q4MI_E_ARG;
    if (misaligned16(gate_up) || misaligned16(down) || misaligned16(x) || misaligned16(out) || misaligned16(workspace))
        return Q4MI_E_ARG;
    if (precision == 0 && (!gate_up_scales || !down_scales || misaligned16(gate_up_scales) ||
                           misaligned16(down_scales)))
        return Q4MI_E_ARG;
    const MoePfWs w = moe_pf_ws(T, E, topk, H, F);
    if (!workspace || workspace_bytes < w.total) return Q4MI_E_WORKSPACE;
    char* ws = (char*)workspace;
    int* cnt = (int*)(ws + w.cnt);
    int* off = (int*)(ws + w.off);
    int* meta = (int*)(ws + w.meta);
    int* tile_e = (int*)(ws + w.tile_e);
    int* tile_end = (int*)(ws + w.tile_end);
    int* sop = (int*)(ws + w.sop);
    int* rowmap = (int*)(ws + w.rowmap);
    int* texp = (int*)(ws + w.texp);
    uint16_t* x16 = (uint16_t*)(ws + w.x16);
    float* gy = (float*)(ws + w.gy);
    const int P = T * topk;
    const hipStream_t st = (hipStream_t)stream;
    const unsigned S = (unsigned)(w.tiles_max * 256), SP = S / 4;
    const bool xf32 = x_dtype == Q4MI_F32;

    hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(1024), 0, st, topk_ids, P, E, cnt, off, tile_e, tile_end, meta);
    if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
    hipLaunchKernelGGL(moe_slots_kernel, dim3((unsigned)E), dim3(256), 0, st, topk_ids, P, topk, cnt, off, sop, rowmap);
    if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;

    // the prefill scales: wexp int32[N], then the fp16 plane, per stacked matrix
    auto plane = [](const void* sc, int64_t N) {
        return (const uint32_t*)((const char*)sc + align256((size_t)N * 4));
    };
    const int64_t N1 = 2 * F, N2 = H;
    const int64_t eb1 = (N1 / 64) * (H / 32) * kTileBytes, eb2 = (N2 / 64) * (F / 32) * kTileBytes;
    const int64_t sw1 = (N1 / 64) * (H / 32) * 64, sw2 = (N2 / 64) * (F / 32) * 64;
    const int* we1 = precision == 0 ? (const int*)gate_up_scales : nullptr;
    const int* we2 = precision == 0 ? (const int*)down_scales : nullptr;
    const uint32_t* s1 = precision == 0 ? plane(gate_up_scales, (int64_t)E * N1) : nullptr;
    const uint32_t* s2 = precision == 0 ? plane(down_scales, (int64_t)E * N2) : nullptr;
    const unsigned g1 = (unsigned)(w.tiles_max * (N1 / 256)), g2 = (unsigned)(w.tiles_max * (N2 / 256));

    // precision 1 on bf16 x: the expert GEMMs DMA their token rows straight from x (gate/up,
    // slot s <- token rowmap[s]) and from h (down, slot s <- h row s): no per-slot activation
    // images. h [S][F] bf16 from the gate/up epilogue goes to the x16 region, Y to gy. The DMA
    // offsets are 32-bit.
    const bool gather = precision == 1 && !xf32 && (uint64_t)T * H * 2 <= 0xffffffffull &&
                        (uint64_t)S * F * 2 <= 0xffffffffull;
    if (gather) {
        hipLaunchKernelGGL((moe_dma_kernel<1, true, true>), dim3(g1), dim3(512), 0, st, gate_up, eb1,
                           (const uint16_t*)x, texp, we1, s1, sw1, (float*)x16, tile_e, tile_end, meta, (int)N1,
                           (int)H, (int)(N1 / 256), 0, (const int*)rowmap);
        if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
        hipLaunchKernelGGL((moe_dma_kernel<1, false, true>), dim3(g2), dim3(512), 0, st, down, eb2, x16, texp, we2, s2,
                           sw2, gy, tile_e, tile_end, meta, (int)N2, (int)F, (int)(N2 / 256), 0, (const int*)nullptr);
        if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
        hipLaunchKernelGGL(moe_prefill_combine_kernel, dim3((unsigned)ceil_div(H / 4, 256), (unsigned)T), dim3(256), 0,
                           st, gy, sop, topk_ids, topk_w, topk, E, (int)H, out);
        return launch_status();
    }

    // gate/up: G = X . [gate; up]^T per expert. Precision 0: the token rows go through the
    // pre-pass once per token ([T][H] fp16 and the token exponents, in the x16 and texp
    // regions) and the GEMM gathers them per slot; the h preps overwrite both afterwards.
    const int xpasses = precision == 0 && xf32 ? 2 : 1;
    const bool swi = hb16 && xpasses == 1;
    const bool gx = precision == 0 && (uint64_t)T * H * 2 <= 0xffffffffull;
    for (int pass = 0; pass < xpasses; ++pass) {
        if (gx) {
            launch_xprep(xf32, 0, false, dim3((unsigned)T), st, x, x16, texp, T, (int)H, pass);
        } else if (xf32) {
            if (precision == 0)
                hipLaunchKernelGGL((moe_xprep_kernel<true, 0>), dim3(SP), dim3(256), 0, st, x, rowmap, meta, x16, texp,
                                   (int)H, pass);
            else
                hipLaunchKernelGGL((moe_xprep_kernel<true, 1>), dim3(SP), dim3(256), 0, st, x, rowmap, meta, x16, texp,
                                   (int)H, pass);
        } else {
            if (precision == 0)
                hipLaunchKernelGGL((moe_xprep_kernel<false, 0>), dim3(SP), dim3(256), 0, st, x, rowmap, meta, x16,
                                   texp, (int)H, pass);
            else
                hipLaunchKernelGGL((moe_xprep_kernel<false, 1>), dim3(SP), dim3(256), 0, st, x, rowmap, meta, x16,
                                   texp, (int)H, pass);
        }
        if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
        // bf16 h from one activation pass: SwiGLU in the gate/up epilogue, h [S][F] bf16 in
        // the G/Y buffer (G itself is never written)
        if (swi && gx)
            hipLaunchKernelGGL((moe_dma_kernel<0, true, true>), dim3(g1), dim3(512), 0, st, gate_up, eb1, x16, texp,
                               we1, s1, sw1, gy, tile_e, tile_end, meta, (int)N1, (int)H, (int)(N1 / 256), 0,
                               (const int*)rowmap);
        else if (swi && precision == 0)
            hipLaunchKernelGGL((moe_dma_kernel<0, true>), dim3(g1), dim3(512), 0, st, gate_up, eb1, x16, texp, we1, s1,
                               sw1, gy, tile_e, tile_end, meta, (int)N1, (int)H, (int)(N1 / 256), 0);
        else if (swi)
            hipLaunchKernelGGL((moe_dma_kernel<1, true>), dim3(g1), dim3(512), 0, st, gate_up, eb1, x16, texp, we1, s1,
                               sw1, gy, tile_e, tile_end, meta, (int)N1, (int)H, (int)(N1 / 256), 0);
        else if (gx)
            hipLaunchKernelGGL((moe_dma_kernel<0, false, true>), dim3(g1), dim3(512), 0, st, gate_up, eb1, x16, texp,
                               we1, s1, sw1, gy, tile_e, tile_end, meta, (int)N1, (int)H, (int)(N1 / 256), pass,
                               (const int*)rowmap);
        else if (precision == 0)
            hipLaunchKernelGGL((moe_dma_kernel<0>), dim3(g1), dim3(512), 0, st, gate_up, eb1, x16, texp, we1, s1, sw1,
                               gy, tile_e, tile_end, meta, (int)N1, (int)H, (int)(N1 / 256), pass);
        else
            hipLaunchKernelGGL((moe_dma_kernel<1>), dim3(g1), dim3(512), 0, st, gate_up, eb1, x16, texp, we1, s1, sw1,
                               gy, tile_e, tile_end, meta, (int)N1, (int)H, (int)(N1 / 256), 0);
        if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
    }
    // h = silu(g) u into the 16-bit layout (precision 0: value and remainder planes, both
    // made before the down GEMM overwrites G with Y)
    const int hpasses = precision == 0 && !hb16 ? 2 : 1;
    uint16_t* h16[2] = {x16, x16 + (size_t)S * F};
    for (int pass = 0; pass < hpasses; ++pass) {
        if (swi && precision == 0)
            hipLaunchKernelGGL((moe_h16prep_kernel<0>), dim3(SP), dim3(256), 0, st, (const uint16_t*)gy, rowmap, meta,
                               h16[0], texp, (int)F);
        else if (swi)
            hipLaunchKernelGGL((moe_h16prep_kernel<1>), dim3(SP), dim3(256), 0, st, (const uint16_t*)gy, rowmap, meta,
                               h16[0], texp, (int)F);
        else if (precision == 0 && hb16)
            hipLaunchKernelGGL((moe_hprep_kernel<0, true>), dim3(SP), dim3(256), 0, st, gy, rowmap, meta, h16[pass],
                               texp, (int)F, 0);
        else if (precision == 0)
            hipLaunchKernelGGL((moe_hprep_kernel<0>), dim3(SP), dim3(256), 0, st, gy, rowmap, meta, h16[pass], texp,
                               (int)F, pass);
        else
            hipLaunchKernelGGL((moe_hprep_kernel<1>), dim3(SP), dim3(256), 0, st, gy, rowmap, meta, h16[pass], texp,
                               (int)F, pass);
        if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
    }
    for (int pass = 0; pass < hpasses; ++pass) {
        if (precision == 0)
            hipLaunchKernelGGL((moe_dma_kernel<0>), dim3(g2), dim3(512), 0, st, down, eb2, h16[pass], texp, we2, s2,
                               sw2, gy, tile_e, tile_end, meta, (int)N2, (int)F, (int)(N2 / 256), pass);
        else
            hipLaunchKernelGGL((moe_dma_kernel<1>), dim3(g2), dim3(512), 0, st, down, eb2, h16[pass], texp, we2, s2,
                               sw2, gy, tile_e, tile_end, meta, (int)N2, (int)F, (int)(N2 / 256), 0);
        if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
    }
    hipLaunchKernelGGL(moe_prefill_combine_kernel, dim3((unsigned)ceil_div(H / 4, 256), (unsigned)T), dim3(256), 0, st,
                       gy, sop, topk_ids, topk_w, topk, E, (int)H, out);
    return launch_status();
}
