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
// Tiling: a 256-thread workgroup computes BN weight rows x BT tokens, its four
// waves 2x2 over that tile. Per 32-K step every wave of the group turns the
// mx codes of its 64-row group into 16-bit weights and stores them to LDS;
// activations are copied to LDS; both are double buffered so the global loads
// and the dequant of step k+1 overlap the MFMAs of step k (one barrier per
// step). LDS rows are 40 halves (80 B) so a 16-lane ds_read_b128 phase hits
// distinct banks.
#include "q4mi_device.h"
#include "q4mi_internal.h"

using namespace q4mi;

namespace {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
constexpr int kLdsStride = 40;     // halves per LDS row: 32 k + 8 pad
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

template <int BN, int BT, int PREC>
__global__ __launch_bounds__(256) void prefill_kernel(const uint8_t* __restrict__ packed,
                                                      const uint16_t* __restrict__ x16,
                                                      const float* __restrict__ tscale, float* __restrict__ y,
                                                      int T, int N, int K, int tiles_t) {
    constexpr int WN = BN / 2, WT = BT / 2;          // wave tile
    constexpr int FN = WN / 16, FT = WT / 16;        // 16-wide fragments per wave
    constexpr int RG = BN / 64;                      // mx row groups per workgroup tile
    constexpr int XCH = BT * 4 / 256;                // 16-byte activation chunks per thread
    typedef typename std::conditional<PREC == 0, f16x8, bf16x8>::type frag_t;

    __shared__ __attribute__((aligned(16))) uint16_t wl[2][BN * kLdsStride];
    __shared__ __attribute__((aligned(16))) uint16_t xl[2][BT * kLdsStride];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 1, wt = wave >> 1;
    const int bt = blockIdx.x % tiles_t, bn = blockIdx.x / tiles_t;
    const int n0 = bn * BN, t0 = bt * BT;
    const int KB = K >> 5;
    const int G = N >> 6;
    const int i16 = lane & 15, kg = lane >> 4;

    // this thread's mx row group (waves beyond RG have none) and activation chunks
    const bool has_w = wave < RG;
    const int rg = min(n0 / 64 + (has_w ? wave : 0), G - 1);         // clamp ragged N
    const uint8_t* wbase = packed + (int64_t)rg * KB * kTileBytes;
    const int coff = lane * 16, soff = kCodeBytes + i16 * 16;
    const uint16_t* xsrc[XCH];
    int xdst[XCH];
#pragma unroll
    for (int c = 0; c < XCH; ++c) {
        const int ch = tid + 256 * c, tok = ch >> 2, part = ch & 3;
        xsrc[c] = x16 + (int64_t)min(t0 + tok, T - 1) * K + part * 8;
        xdst[c] = tok * kLdsStride + part * 8;
    }
    const uint32_t nib2 = vgpr_const(kNib2);
    const uint32_t magic = vgpr_const(PREC == 0 ? kMagic1024 : kMagic128);

    f32x4 acc[FN][FT];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 wc = {}, ws = {};
    u32x4 xr[XCH];
    auto gload = [&](int ks) {
        if (has_w) {
            const uint8_t* tp = wbase + (int64_t)ks * kTileBytes;
            wc = load_nt_u32x4(tp + coff);
            ws = load_nt_u32x4(tp + soff);
        }
#pragma unroll
        for (int c = 0; c < XCH; ++c) xr[c] = *(const u32x4*)(xsrc[c] + ks * 32);
    };
    auto lstore = [&](int buf) {
        if (has_w) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const u32x4 v = dequant8<PREC>(wc[r], ws[r], nib2, magic);
                *(u32x4*)&wl[buf][(wave * 64 + r * 16 + i16) * kLdsStride + kg * 8] = v;
            }
        }
#pragma unroll
        for (int c = 0; c < XCH; ++c) *(u32x4*)&xl[buf][xdst[c]] = xr[c];
    };

    gload(0);
    lstore(0);
    __syncthreads();
    for (int ks = 0; ks < KB; ++ks) {
        const int buf = ks & 1;
        const bool more = ks + 1 < KB;
        if (more) gload(ks + 1);
        frag_t a[FN], b[FT];
#pragma unroll
        for (int i = 0; i < FN; ++i)
            a[i] = *(const frag_t*)&wl[buf][(wn * WN + i * 16 + i16) * kLdsStride + kg * 8];
#pragma unroll
        for (int j = 0; j < FT; ++j)
            b[j] = *(const frag_t*)&xl[buf][(wt * WT + j * 16 + i16) * kLdsStride + kg * 8];
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FT; ++j) acc[i][j] = mfma16(a[i], b[j], acc[i][j]);
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

struct TileChoice {
    int bn, bt;
};

// Pick the workgroup tile that keeps the most of 256 CUs busy for this shape.
TileChoice choose_tile(int T, int N) {
    const TileChoice c[] = {{256, 256}, {256, 128}, {128, 256}, {128, 128}};
    const double eff[] = {1.0, 0.92, 0.92, 0.8};   // per-workgroup MFMA efficiency guess by tile
    double best = 1e300;
    TileChoice pick = c[3];
    for (int i = 0; i < 4; ++i) {
        const int64_t wgs = ceil_div(N, c[i].bn) * ceil_div(T, c[i].bt);
        const int64_t rounds = ceil_div(wgs, 256);
        const double cost = (double)rounds * c[i].bn * c[i].bt / eff[i];
        if (cost < best) {
            best = cost;
            pick = c[i];
        }
    }
    return pick;
}

template <int BN, int BT>
void launch_tile(int prec, int64_t grid, hipStream_t st, const uint8_t* w, const uint16_t* x16, const float* ts,
                 float* y, int T, int N, int K, int tiles_t) {
    if (prec == 0)
        hipLaunchKernelGGL((prefill_kernel<BN, BT, 0>), dim3((unsigned)grid), dim3(256), 0, st, w, x16, ts, y, T,
                           N, K, tiles_t);
    else
        hipLaunchKernelGGL((prefill_kernel<BN, BT, 1>), dim3((unsigned)grid), dim3(256), 0, st, w, x16, ts, y, T,
                           N, K, tiles_t);
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
    const TileChoice tc = choose_tile(T, (int)N);
    const int tiles_t = (int)ceil_div(T, tc.bt);
    const int64_t grid = ceil_div(N, tc.bn) * tiles_t;
    const float* tsp = precision == 0 ? ts : nullptr;
    if (tc.bn == 256 && tc.bt == 256) launch_tile<256, 256>(precision, grid, st, packed, x16, tsp, y, T, (int)N, (int)K, tiles_t);
    else if (tc.bn == 256) launch_tile<256, 128>(precision, grid, st, packed, x16, tsp, y, T, (int)N, (int)K, tiles_t);
    else if (tc.bt == 256) launch_tile<128, 256>(precision, grid, st, packed, x16, tsp, y, T, (int)N, (int)K, tiles_t);
    else launch_tile<128, 128>(precision, grid, st, packed, x16, tsp, y, T, (int)N, (int)K, tiles_t);
    return launch_status();
}
