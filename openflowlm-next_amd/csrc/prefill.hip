// prefill.hip -- prefill GEMM: Y[T][N] = X[T][K] . W[N][K]^T, W in the mx layout,
// dequantized into LDS tiles that feed the 16x16x32 MFMA, fp32 accumulate.
//
// The reference prefill dequantizes one 64x64 tile of a band into a bf16 A
// operand in core memory, then runs mlir-aie's bf16 matmul on it
// (open_kernels/designs/gemm_q4_prefill/gemm_q4_dequant.h:315-376,
// gemm_q4_prefill.py:198-203). Rounding each weight once to bf16 costs a
// maxrel of ~1.8e-3 against the fp64 reference (gemm_q4_dequant.h:283-286),
// over the 1e-3 bar. Two precisions are built from one kernel:
//   PREC 0 (default): w16 = RNE_f16(q*d + m) (one v_pk_fma_f16 per pair, 11-bit
//     significand), X -> fp16 (exact for bf16 inputs inside fp16's range; each
//     token row is pre-scaled by a power of two when max|x| >= 2^15 and the
//     output scaled back, both exact), fp16 MFMA. CDNA4's dense fp16 and bf16
//     MFMA peaks are equal.
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
// element e = k offset e of the dword's k-group.
template <int PREC>
__device__ __forceinline__ u32x4 dequant8(uint32_t w, uint32_t s, uint32_t nib2, uint32_t magic) {
    u32x4 out;
    if constexpr (PREC == 0) {
        const _Float16 dh = (_Float16)bf16_hi_to_f32(s), mh = (_Float16)bf16_lo_to_f32(s);
        const f16x2 d2 = {dh, dh}, m2 = {mh, mh};
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

// BN x BT workgroup tile, WGN x WGT waves (wave tile BN/WGN x BT/WGT), KS
// 32-K blocks per LDS stage.
template <int BN, int BT, int WGN, int WGT, int KS, int PREC>
__global__ __launch_bounds__(64 * WGN * WGT) void prefill_kernel(const uint8_t* __restrict__ packed,
                                                                 const uint16_t* __restrict__ x16,
                                                                 const float* __restrict__ tscale,
                                                                 float* __restrict__ y, int T, int N, int K,
                                                                 int tiles_t) {
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

    // this wave's mx tiles: tile u = wave + NW*i -> (row group u % RG, block u / RG of the stage)
    const uint8_t* wbase[WPW];
    int wrow[WPW], wcol[WPW];
    bool wown[WPW];
#pragma unroll
    for (int i = 0; i < WPW; ++i) {
        const int u = wave + NW * i;
        wown[i] = u < WTILES;
        const int rgl = u % RG, kbl = u / RG;
        const int rg = min(n0 / 64 + rgl, G - 1);                       // clamp ragged N
        wbase[i] = packed + ((int64_t)rg * KB + kbl) * kTileBytes;
        wrow[i] = rgl * 64 + i16;
        wcol[i] = kbl * 32 + kg * 8;
    }
    const int coff = lane * 16, soff = kCodeBytes + i16 * 16;
    const uint16_t* xsrc[XCH];
    int xdst[XCH];
#pragma unroll
    for (int c = 0; c < XCH; ++c) {
        const int ch = tid + NT * c, tok = ch / (KS * 4), part = ch % (KS * 4);
        xsrc[c] = x16 + (int64_t)min(t0 + tok, T - 1) * K + part * 8;
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
#pragma unroll
        for (int i = 0; i < WPW; ++i) {
            if (wown[i]) {
                const uint8_t* tp = wbase[i] + (int64_t)st * KS * kTileBytes;
                wc[i] = load_nt_u32x4(tp + coff);
                wsc[i] = load_nt_u32x4(tp + soff);
            }
        }
#pragma unroll
        for (int c = 0; c < XCH; ++c) xr[c] = *(const u32x4*)(xsrc[c] + st * BK);
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

    // lane holds D[n = 4*kg + r][t = i16] of each 16x16 fragment: 4 consecutive n of one token
#pragma unroll
    for (int j = 0; j < FT; ++j) {
        const int t = t0 + wt * WT + j * 16 + i16;
        if (t >= T) continue;
        const float sc = tscale ? tscale[t] : 1.0f;
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            const int n = n0 + wn * WN + i * 16 + kg * 4;
            if (n < N) {
                f32x4 v = acc[i][j];
                v = v * sc;
                *(f32x4*)(y + (int64_t)t * N + n) = v;
            }
        }
    }
}

// Activations -> the MFMA's 16-bit type, one workgroup per token row.
// PREC 0: fp16, with the row scaled by 2^-s (s >= 0 the least that keeps
// max|x| 2^-s < 2^15) and tscale[t] = 2^s; PREC 1: bf16 (RNE from f32).
template <bool XF32, int PREC>
__global__ __launch_bounds__(256) void prefill_xprep(const void* __restrict__ x, uint16_t* __restrict__ x16,
                                                     float* __restrict__ tscale, int K) {
    const int t = blockIdx.x;
    const int64_t row = (int64_t)t * K;
    auto ld = [&](int k) -> float {
        if constexpr (XF32) return ((const float*)x)[row + k];
        else return __builtin_bit_cast(float, (uint32_t)((const uint16_t*)x)[row + k] << 16);
    };
    float scale = 1.0f;
    if constexpr (PREC == 0) {
        __shared__ float red[256];
        float mx = 0.f;
        for (int k = threadIdx.x; k < K; k += 256) mx = fmaxf(mx, fabsf(ld(k)));
        red[threadIdx.x] = mx;
        __syncthreads();
        for (int s = 128; s > 0; s >>= 1) {
            if ((int)threadIdx.x < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
            __syncthreads();
        }
        mx = red[0];
        int s = 0;
        if (mx >= 32768.0f && mx <= 3.0e38f) {
            int e;
            frexpf(mx, &e);                      // mx in [2^(e-1), 2^e)
            s = e - 15;                          // mx * 2^-s < 2^15
        }
        scale = ldexpf(1.0f, -s);
        if (threadIdx.x == 0) tscale[t] = ldexpf(1.0f, s);
    }
    for (int k = threadIdx.x; k < K; k += 256) {
        const float v = ld(k) * scale;
        uint16_t o;
        if constexpr (PREC == 0) o = __builtin_bit_cast(uint16_t, (_Float16)v);
        else o = (uint16_t)f32_to_bf16_rne(v);
        x16[row + k] = o;
    }
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
};
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

// Pick the variant that keeps the most of 256 CUs busy (Q4MI_PREFILL_CFG overrides).
int choose_cfg(int T, int N, int K) {
    static int forced = [] {
        const char* e = getenv("Q4MI_PREFILL_CFG");
        return e ? atoi(e) : -1;
    }();
    if (forced >= 0 && forced < kNumCfgs && K % (32 * kCfgs[forced].ks) == 0) return forced;
    const double eff[] = {1.0, 0.9, 0.9, 0.75, 0.8};   // relative per-workgroup efficiency
    double best = 1e300;
    int pick = 4;
    for (int i = 0; i < kNumCfgs; ++i) {
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
void launch_cfg(int64_t grid, hipStream_t st, const uint8_t* w, const uint16_t* x16, const float* ts, float* y,
                int T, int N, int K, int tiles_t) {
    constexpr TileCfg c = kCfgs[C];
    hipLaunchKernelGGL((prefill_kernel<c.bn, c.bt, c.wgn, c.wgt, c.ks, PREC>), dim3((unsigned)grid),
                       dim3(64 * c.wgn * c.wgt), 0, st, w, x16, ts, y, T, N, K, tiles_t);
}

template <int PREC>
void launch_prefill(int cfg, int64_t grid, hipStream_t st, const uint8_t* w, const uint16_t* x16, const float* ts,
                    float* y, int T, int N, int K, int tiles_t) {
    switch (cfg) {
        case 0: launch_cfg<0, PREC>(grid, st, w, x16, ts, y, T, N, K, tiles_t); break;
        case 1: launch_cfg<1, PREC>(grid, st, w, x16, ts, y, T, N, K, tiles_t); break;
        case 2: launch_cfg<2, PREC>(grid, st, w, x16, ts, y, T, N, K, tiles_t); break;
        case 3: launch_cfg<3, PREC>(grid, st, w, x16, ts, y, T, N, K, tiles_t); break;
        default: launch_cfg<4, PREC>(grid, st, w, x16, ts, y, T, N, K, tiles_t); break;
    }
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

}  // namespace

extern "C" size_t q4_gemm_prefill_workspace_bytes(int T, int64_t N, int64_t K) {
    if (T <= 0 || K <= 0) return 0;
    (void)N;
    return align256((size_t)T * K * 2) + align256((size_t)T * 4);
}

extern "C" int q4_gemm_prefill(const uint8_t* packed, const void* x, int x_dtype, float* y, int T, int64_t N,
                               int64_t K, int precision, void* workspace, size_t workspace_bytes, void* stream) {
    if (x_dtype != Q4MI_F32 && x_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (precision != 0 && precision != 1) return Q4MI_E_ARG;
    if (T < 0 || N < 0 || K <= 0 || N % 64 || K % 32) return Q4MI_E_SHAPE;
    if (N > 0x7FFFFFFF || K > 0x7FFFFFFF) return Q4MI_E_RANGE;
    if (T == 0 || N == 0) return Q4MI_OK;
    if (!packed || !x || !y) return Q4MI_E_ARG;
    const size_t need = q4_gemm_prefill_workspace_bytes(T, N, K);
    if (!workspace || workspace_bytes < need) return Q4MI_E_WORKSPACE;
    uint16_t* x16 = (uint16_t*)workspace;
    float* ts = (float*)((char*)workspace + align256((size_t)T * K * 2));
    const hipStream_t st = (hipStream_t)stream;
    const bool xf32 = x_dtype == Q4MI_F32;
    if (precision == 0) {
        if (xf32) hipLaunchKernelGGL((prefill_xprep<true, 0>), dim3(T), dim3(256), 0, st, x, x16, ts, (int)K);
        else hipLaunchKernelGGL((prefill_xprep<false, 0>), dim3(T), dim3(256), 0, st, x, x16, ts, (int)K);
    } else {
        if (xf32) hipLaunchKernelGGL((prefill_xprep<true, 1>), dim3(T), dim3(256), 0, st, x, x16, ts, (int)K);
        else hipLaunchKernelGGL((prefill_xprep<false, 1>), dim3(T), dim3(256), 0, st, x, x16, ts, (int)K);
    }
    if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
    const int cfg = choose_cfg(T, (int)N, (int)K);
    const int tiles_t = (int)ceil_div(T, kCfgs[cfg].bt);
    const int64_t grid = ceil_div(N, kCfgs[cfg].bn) * tiles_t;
    const float* tsp = precision == 0 ? ts : nullptr;
    if (precision == 0) launch_prefill<0>(cfg, grid, st, packed, x16, tsp, y, T, (int)N, (int)K, tiles_t);
    else launch_prefill<1>(cfg, grid, st, packed, x16, tsp, y, T, (int)N, (int)K, tiles_t);
    return launch_status();
}
