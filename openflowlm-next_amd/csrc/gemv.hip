// gemv.hip -- decode GEMV / skinny GEMM on the mx layout: Y[M][N] = X[M][K] . W^T,
// 1 <= M <= 16, fp32 accumulate (inner loop in gemv_core.h).
//
// Work item = one 64-row group over a K range, one 256-thread workgroup.
// K splits (S > 1, for matrices too short to fill 256 CUs): the GEMV kernel
// writes each split's partial sums to the workspace and a second, tiny kernel
// adds the S partials in split order, so the result does not depend on the
// order the workgroups ran in. (Finishing in the last-arriving workgroup
// instead needs device-scope fences, which on gfx950 write back and
// invalidate the L2 of every XCD -- far slower than the extra launch.)
#include <stdlib.h>

#include <algorithm>
#include <mutex>

#include "gemv_core.h"
#include "q4mi_internal.h"

using namespace q4mi;

namespace {

struct GemvParams {
    const uint8_t* packed;
    const void* x;
    float* y;
    int M;
    int S;
    int64_t N, K;
    float* part;      // [S][M][N] partial sums (S > 1)
    const float* res; // residual added to the result ([M][N], may alias y), or null
    const void* nw;   // NORM kernels: the RMSNorm weight [K] (x is the f32 residual stream)
    int nw_bf16;
    float eps;
    const float* acc_part;   // XN kernels: x = res (P.x) + the S planes of a split GEMV's partials
    int acc_S;
    float* x_out;            // XN kernels: that x, written by workgroup 0 (when not null)
    bool xn;                 // launch the XN instance
};


// y[t][n] = sum over s = 0..S-1 of part[s][t][n], in split order (+ res[t][n]).
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ part, float* y,
                                                           int64_t MN, int S, const float* res) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= MN) return;
    // loads batched sixteen splits at a time (one trip to memory for the plans' counts),
    // added in split order
    float s = 0.f;
    for (int q = 0; q < S; q += 16) {
        float t[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) t[u] = q + u < S ? part[(int64_t)(q + u) * MN + i] : 0.f;
#pragma unroll
        for (int u = 0; u < 16; ++u)
            if (q + u < S) s += t[u];
    }
    y[i] = res ? res[i] + s : s;
}

// WAVES waves per workgroup (4, 8 or 16): more waves put more tiles of a row group in
// flight, so fewer K splits fill the memory system.
// NORM: X = bf16(RMSNorm(x) * nw) formed per tile from the f32 row x (every workgroup
// first computes the rows' 1/rms exactly as q4_rmsnorm_add does), so the norm needs no
// launch and no bf16 copy of its own.
// XN (NORM on the rolling loop, one row of K <= 256 kAccRowJ): x is res (P.x) plus a split
// GEMV's partial-sum planes (P.acc_part, P.acc_S); each workgroup reduces them in
// split_reduce's order, normalises the row into LDS once, and workgroup 0 writes x to
// P.x_out, so the producer needs no reduce launch.
constexpr int kXnElems = 256 * kAccRowJ;

// F16S: the scale words hold fp16 d and m (q4_repack scale_mode 1; rolling loop, plain x).
template <int NTL, bool XF32, int WAVES, bool Q40 = false, bool NORM = false, bool STREAM = false, bool XN = false,
          bool F16S = false>
__global__ __launch_bounds__(64 * WAVES) void gemv_kernel(GemvParams P) {
    static_assert(!XN || (NORM && STREAM && NTL == 1 && !Q40), "XN: one row, norm, rolling loop");
    static_assert(!F16S || (STREAM && !NORM && !Q40), "fp16 scales: the rolling loop over plain activations");
    __shared__ float red[WAVES][4][NTL][64];
    __shared__ float rrow[NORM ? 4 * NTL : 1];
    __shared__ __attribute__((aligned(16))) __bf16 xs[XN ? kXnElems : 8];
    __shared__ float xf[XN ? kXnElems : 1];
    if constexpr (NORM && !XN) rms_inv_rows<4 * NTL>((const float*)P.x, P.M, P.K, P.eps, rrow);
    const int64_t item = blockIdx.x;
    const int S = P.S;
    const int64_t g = item / S;
    const int s = (int)(item % S);
    const int KB = (int)(P.K >> 5);
    const int kb0 = (int)((int64_t)s * KB / S), kb1 = (int)((int64_t)(s + 1) * KB / S);
    float acc[1][4][NTL];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < NTL; ++j) acc[0][r][j] = 0.f;
    if constexpr (XN) {
        const uint8_t* const gb[1] = {P.packed + g * KB * kTileBytes};
        const int kr = (kb1 - kb0) * 32;
        float* xo = blockIdx.x == 0 ? P.x_out : nullptr;
        if (P.nw_bf16)
            stage_norm_acc_row<1, 64 * WAVES>((const float*)P.x, P.acc_part, P.acc_S, P.K, P.K, P.eps, P.nw, (int64_t)kb0 * 32, kr,
                                  xs, xo, xf);
        else
            stage_norm_acc_row<2, 64 * WAVES>((const float*)P.x, P.acc_part, P.acc_S, P.K, P.K, P.eps, P.nw, (int64_t)kb0 * 32, kr,
                                  xs, xo, xf);
        gemv_rows_stream<1, false, 1, 4, WAVES, false, 0, DenseRows, true>(gb, P.x, DenseRows{P.M}, P.K, kb0, kb1, acc,
                                                                          NormIn{}, xs, kr);
    } else if constexpr (STREAM) {
        // K positions in flight: 4, or 3 where 16 waves (128 VGPRs each) hold 3-4 accumulator
        // sets or 2 with the f32 activation's two fragments (an in-flight register must not be
        // spilled)
        constexpr int kUnr = WAVES == 16 && (NTL >= 3 || (NTL == 2 && XF32)) ? 3 : 4;
        const uint8_t* const gb[1] = {P.packed + g * KB * (Q40 ? kQ0TileBytes : kTileBytes)};
        const NormIn nrm{P.nw, P.nw_bf16, rrow};
        if constexpr (NORM) {
            if (P.nw_bf16)
                gemv_rows_stream<NTL, false, 1, kUnr, WAVES, Q40, 1>(gb, P.x, DenseRows{P.M}, P.K, kb0, kb1, acc,
                                                                     nrm);
            else
                gemv_rows_stream<NTL, false, 1, 3, WAVES, Q40, 2>(gb, P.x, DenseRows{P.M}, P.K, kb0, kb1, acc, nrm);
        } else {
            gemv_rows_stream<NTL, XF32, 1, kUnr, WAVES, Q40, 0, DenseRows, false, F16S>(gb, P.x, DenseRows{P.M}, P.K,
                                                                                     kb0, kb1, acc);
        }
    } else {
        gemv_rows<NTL, XF32, DenseRows, WAVES, Q40, NORM>(P.packed, P.x, DenseRows{P.M}, P.K, g, kb0, kb1, acc[0],
                                                           NormIn{P.nw, P.nw_bf16, rrow});
    }
    if (S == 1) gemv_finish<NTL, WAVES>(acc[0], red, P.M, P.y, P.N, g, P.res);
    else gemv_finish<NTL, WAVES>(acc[0], red, P.M, P.part + (int64_t)s * P.M * P.N, P.N, g);
}

// gemv_kernel for 17..24 tokens: two 16-token blocks (gemv_rows_tb2) over the same work
// items and splits; block 1's rows are stored from y + 16 N (its partials from the split's
// token row 16).
template <int NTL2, bool XF32, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void gemv_tb2_kernel(GemvParams P) {
    __shared__ float red[WAVES][4][4][64];
    const int64_t item = blockIdx.x;
    const int S = P.S;
    const int64_t g = item / S;
    const int s = (int)(item % S);
    const int KB = (int)(P.K >> 5);
    const int kb0 = (int)((int64_t)s * KB / S), kb1 = (int)((int64_t)(s + 1) * KB / S);
    float acc0[4][4], acc1[4][NTL2];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc0[r][j] = 0.f;
#pragma unroll
        for (int j = 0; j < NTL2; ++j) acc1[r][j] = 0.f;
    }
    gemv_rows_tb2<NTL2, XF32, WAVES>(P.packed, P.x, P.M, P.K, g, kb0, kb1, acc0, acc1);
    float* y = S == 1 ? P.y : P.part + (int64_t)s * P.M * P.N;
    const float* res = S == 1 ? P.res : nullptr;
    gemv_finish<4, WAVES>(acc0, red, 16, y, P.N, g, res);
    __syncthreads();
    gemv_finish<NTL2, WAVES>(acc1, (float (*)[4][NTL2][64])red, P.M - 16, y + 16 * P.N, P.N, g,
                             res ? res + 16 * P.N : nullptr);
}

// The GEMV over the native Q4_K layout: split s takes super-blocks [sb0, sb1) of K / 256
// (each wave whole super-blocks), then stores as gemv_kernel.
template <int NTL, bool XF32>
__global__ __launch_bounds__(256) void q4k_gemv_kernel(GemvParams P) {
    __shared__ float red[kWaves][4][NTL][64];
    const int64_t item = blockIdx.x;
    const int S = P.S;
    const int64_t g = item / S;
    const int s = (int)(item % S);
    const int SB = (int)(P.K >> 8);
    const int sb0 = (int)((int64_t)s * SB / S), sb1 = (int)((int64_t)(s + 1) * SB / S);
    float acc[4][NTL];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < NTL; ++j) acc[r][j] = 0.f;
    q4k_rows<NTL, XF32>(P.packed, P.x, DenseRows{P.M}, P.K, g, sb0, sb1, acc);
    if (S == 1) gemv_finish<NTL>(acc, red, P.M, P.y, P.N, g, P.res);
    else gemv_finish<NTL>(acc, red, P.M, P.part + (int64_t)s * P.M * P.N, P.N, g);
}

// The GEMV over the native q8 layout: the same work items, splits and stores as gemv_kernel.
template <int NTL, bool XF32>
__global__ __launch_bounds__(256) void q8n_gemv_kernel(GemvParams P) {
    __shared__ float red[kWaves][4][NTL][64];
    const int64_t item = blockIdx.x;
    const int S = P.S;
    const int64_t g = item / S;
    const int s = (int)(item % S);
    const int KB = (int)(P.K >> 5);
    const int kb0 = (int)((int64_t)s * KB / S), kb1 = (int)((int64_t)(s + 1) * KB / S);
    float acc[4][NTL];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < NTL; ++j) acc[r][j] = 0.f;
    q8n_rows<NTL, XF32>(P.packed, P.x, DenseRows{P.M}, P.K, g, kb0, kb1, acc);
    if (S == 1) gemv_finish<NTL>(acc, red, P.M, P.y, P.N, g, P.res);
    else gemv_finish<NTL>(acc, red, P.M, P.part + (int64_t)s * P.M * P.N, P.N, g);
}

// The q8 GEMV as two q4_1 planes (hi, lo) of one matrix: one workgroup streams row group
// g of both (sharing the activation fragments) and stores y = hi . x + lo . x (S == 1, plus
// the residual when one is given) or this split's partial of that sum.
template <int NTL, bool XF32>
__global__ __launch_bounds__(256) void gemv_pair_kernel(GemvParams P, const uint8_t* lo) {
    __shared__ float red[kWaves][4][NTL][64];
    const int64_t item = blockIdx.x;
    const int S = P.S;
    const int64_t g = item / S;
    const int s = (int)(item % S);
    const int KB = (int)(P.K >> 5);
    const int kb0 = (int)((int64_t)s * KB / S), kb1 = (int)((int64_t)(s + 1) * KB / S);
    const uint8_t* const gb[2] = {P.packed + g * KB * kTileBytes, lo + g * KB * kTileBytes};
    float acc[2][4][NTL];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < NTL; ++j) acc[i][r][j] = 0.f;
    gemv_rows_multi<NTL, XF32, 2, 4>(gb, P.x, DenseRows{P.M}, P.K, kb0, kb1, acc);
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < NTL; ++j) acc[0][r][j] += acc[1][r][j];
    if (S == 1) gemv_finish<NTL>(acc[0], red, P.M, P.y, P.N, g, P.res);
    else gemv_finish<NTL>(acc[0], red, P.M, P.part + (int64_t)s * P.M * P.N, P.N, g);
}

// SwiGLU over a gate / up pair: one workgroup takes row group g of both matrices
// (sharing the activation fragments) over its K range. S == 1: h[t][f] = silu(gate) *
// up, stored f32 or bf16 (RNE); S > 1: this split's gate and up sums go to
// part[s][t][0, F) and [F, 2F), and swiglu_reduce_kernel finishes in split order.
struct SwigluParams {
    const uint8_t* gate;
    const uint8_t* up;
    const void* x;
    void* h;
    int h_bf16;
    int M;
    int S;
    int64_t F, K;
    float* part;
    const void* nw;   // NORM: the RMSNorm weight [K] (x is the f32 residual stream)
    int nw_bf16;
    float eps;
    const float* acc_part;   // XN: x = res (P.x) + these S partial planes, as in gemv_kernel
    int acc_S;
    float* x_out;
    bool xn;
};

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

__device__ __forceinline__ void store_h(void* h, bool bf16, int64_t i, float v) {
    if (bf16) ((uint16_t*)h)[i] = (uint16_t)f32_to_bf16_rne(v);
    else ((float*)h)[i] = v;
}

template <int NTL, bool XF32, bool NORM = false, int WAVES = kWaves, bool STREAM = false, bool XN = false>
__global__ __launch_bounds__(64 * WAVES) void gemv_swiglu_kernel(SwigluParams P) {
    static_assert(!XN || (NORM && STREAM && NTL == 1), "XN: one row, norm, rolling loop");
    __shared__ float red[WAVES][4][NTL][64];
    __shared__ float rrow[NORM ? 4 * NTL : 1];
    __shared__ __attribute__((aligned(16))) __bf16 xs[XN ? kXnElems : 8];
    __shared__ float xf[XN ? kXnElems : 1];
    if constexpr (NORM && !XN) rms_inv_rows<4 * NTL>((const float*)P.x, P.M, P.K, P.eps, rrow);
    const int64_t item = blockIdx.x;
    const int S = P.S;
    const int64_t g = item / S;
    const int s = (int)(item % S);
    const int KB = (int)(P.K >> 5);
    const int kb0 = (int)((int64_t)s * KB / S), kb1 = (int)((int64_t)(s + 1) * KB / S);
    const uint8_t* const gb[2] = {P.gate + g * KB * kTileBytes, P.up + g * KB * kTileBytes};
    float acc[2][4][NTL];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < NTL; ++j) acc[i][r][j] = 0.f;
    const NormIn nrm{P.nw, P.nw_bf16, rrow};
    constexpr int kUnr = NTL >= 3 ? 3 : 4;   // K positions in flight (two tiles each)
    if constexpr (XN) {
        const int kr = (kb1 - kb0) * 32;
        float* xo = blockIdx.x == 0 ? P.x_out : nullptr;
        if (P.nw_bf16)
            stage_norm_acc_row<1, 64 * WAVES>((const float*)P.x, P.acc_part, P.acc_S, P.K, P.K, P.eps, P.nw, (int64_t)kb0 * 32, kr,
                                  xs, xo, xf);
        else
            stage_norm_acc_row<2, 64 * WAVES>((const float*)P.x, P.acc_part, P.acc_S, P.K, P.K, P.eps, P.nw, (int64_t)kb0 * 32, kr,
                                  xs, xo, xf);
        gemv_rows_stream<1, false, 2, kUnr, WAVES, false, 0, DenseRows, true>(gb, P.x, DenseRows{P.M}, P.K, kb0, kb1,
                                                                             acc, NormIn{}, xs, kr);
    } else if constexpr (STREAM) {
        if constexpr (NORM) {
            if (P.nw_bf16)
                gemv_rows_stream<NTL, false, 2, kUnr, WAVES, false, 1>(gb, P.x, DenseRows{P.M}, P.K, kb0, kb1, acc,
                                                                       nrm);
            else
                gemv_rows_stream<NTL, false, 2, 2, WAVES, false, 2>(gb, P.x, DenseRows{P.M}, P.K, kb0, kb1, acc, nrm);
        } else {
            gemv_rows_stream<NTL, XF32, 2, kUnr, WAVES, false, 0>(gb, P.x, DenseRows{P.M}, P.K, kb0, kb1, acc);
        }
    } else {
        gemv_rows_multi<NTL, XF32, 2, 4, WAVES, NORM>(gb, P.x, DenseRows{P.M}, P.K, kb0, kb1, acc, nrm);
    }
    float vg[NTL], vu[NTL];
    wave_sum<NTL, WAVES>(acc[0], red, vg);
    __syncthreads();
    wave_sum<NTL, WAVES>(acc[1], red, vu);
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid >= 256) return;               // threads 0..255 own the row group's 64 rows
    const int64_t f = g * 64 + (tid >> 6) * 16 + (lane & 15);
#pragma unroll
    for (int j = 0; j < NTL; ++j) {
        const int tok = token_of(lane >> 4, j);
        if (tok >= P.M) continue;
        if (S == 1) {
            store_h(P.h, P.h_bf16, (int64_t)tok * P.F + f, silu(vg[j]) * vu[j]);
        } else {
            float* part = P.part + ((int64_t)s * P.M + tok) * 2 * P.F;
            part[f] = vg[j];
            part[P.F + f] = vu[j];
        }
    }
}

__global__ __launch_bounds__(256) void swiglu_reduce_kernel(const float* __restrict__ part, void* h, int h_bf16,
                                                            int M, int64_t F, int S) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)M * F) return;
    const int64_t t = i / F, f = i % F;
    float gs = 0.f, us = 0.f;
    int q = 0;
    for (; q + 4 <= S; q += 4) {               // loads batched, sums in split order
        float tg[4], tu[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float* p = part + ((int64_t)(q + u) * M + t) * 2 * F;
            tg[u] = p[f];
            tu[u] = p[F + f];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            gs += tg[u];
            us += tu[u];
        }
    }
    for (; q < S; ++q) {
        const float* p = part + ((int64_t)q * M + t) * 2 * F;
        gs += p[f];
        us += p[F + f];
    }
    store_h(h, h_bf16, i, silu(gs) * us);
}

// Workgroups to aim for when a matrix has few row groups.
// Q4MI_GEMV_TARGET_WGS (experiments): the workgroup count to split toward, else 0.
int64_t forced_target() {
    static int64_t t = [] {
        const char* e = getenv("Q4MI_GEMV_TARGET_WGS");
        const long v = e ? atol(e) : 0;
        return (int64_t)(v > 0 ? v : 0);
    }();
    return t;
}

constexpr int kMaxGemvTokens = 24;    // the plain GEMV; the q8 pair, SwiGLU, q8 and Q4_K kernels take 16
constexpr int64_t kMaxSplitGroups = 4096;                 // row groups a split call may have

// Splits that bring N/64 row groups toward `target` workgroups (keeping >= 8 blocks, two
// tiles per wave, per split).
int splits_toward(int64_t N, int64_t K, int64_t target) {
    const int64_t G = N / 64, KB = K / 32;
    if (G >= target || G > kMaxSplitGroups) return 1;
    int64_t S = ceil_div(target, G);
    const int64_t max_s = KB / 8;
    if (S > max_s) S = max_s;
    return (int)(S < 1 ? 1 : S);
}

// The q8 pair, native q8 and SwiGLU kernels (4 waves): about 1024 workgroups.
int choose_splits(int64_t N, int64_t K) {
    const int64_t t = forced_target();
    return splits_toward(N, K, t ? t : 1024);
}

// The plain GEMV's plan: K splits and waves per workgroup. Measured per Llama-3-8B shape in
// a same-process A/B (M = 1, graph replays over rotating copies, bit-identical outputs
// across plans up to the split order's fp32 rounding), against 1024 workgroups of 4 waves:
//   28672 x 4096 (448 row groups): unsplit, 8 waves       19.1 -> 15.9 us
//   14336 x 4096 (224):            unsplit, 16 waves      12.7 ->  9.6 us
//    6144 x 4096 (96):             unsplit, 16 waves       8.6 ->  8.4 us
//    4096 x 4096 (64):             4 splits, 8 waves       7.3 ->  7.0 us
//    1024 x 4096 (16):             16 splits, 8 waves      5.6 ->  5.2 us
//    4096 x 14336 (64):            16 splits, 4 waves (kept; 4 splits of 8 waves 12.9 us)
// More waves keep more of a row group's tiles in flight, so fewer splits (and reduce
// traffic) fill the memory system. From 1024 row groups on (lm_head) nothing changes.
// Q4MI_GEMV_TARGET_WGS and Q4MI_GEMV_WAVES override, for experiments.
struct GemvPlan {
    int S, waves;
};

GemvPlan plan_gemv(int64_t N, int64_t K) {
    static const int forced_waves = [] {
        const char* e = getenv("Q4MI_GEMV_WAVES");
        const int v = e ? atoi(e) : 0;
        return v == 4 || v == 8 || v == 16 ? v : 0;
    }();
    const int64_t G = N / 64, t = forced_target();
    if (t || forced_waves) return {splits_toward(N, K, t ? t : 1024), forced_waves ? forced_waves : 4};
    if (G >= 1024) return {1, 4};
    if (G >= 384) return {1, 8};
    if (K <= 8192 && G >= 96) return {1, 16};
    if (K <= 8192) return {splits_toward(N, K, 256), 8};
    return {splits_toward(N, K, 1024), 4};
}

// Native Q4_K: split on whole super-blocks. A wave takes whole super-blocks, so S is the
// smallest divisor of SB / 4 that reaches the workgroup target (every wave of every split
// then gets the same count), else SB / 4 (one per wave). From 256 row groups on there is
// no split: its reduce launch costs more than the longer waves (measured on the Llama-3-8B
// gate_up pair, 28672 x 4096: 15.9 us unsplit, 17.9 us in 4 splits).
constexpr int64_t kQ4kNoSplitGroups = 256;

int q4k_splits(int64_t N, int64_t K) {
    const int64_t G = N / 64, SB = K / 256;
    const int64_t t = forced_target(), target = t ? t : 1024;
    if (G >= target || G >= kQ4kNoSplitGroups || SB < 8) return 1;
    const int64_t want = ceil_div(target, G), per_wave = SB / 4;
    for (int64_t S = 1; S <= per_wave; ++S)
        if (per_wave % S == 0 && S >= want) return (int)S;
    return (int)per_wave;
}

// The SwiGLU kernel's plan. On the rolling pipeline (the default) it is the plain GEMV's
// plan for the 2F rows it streams (gate and up row groups side by side per work item), at
// most 8 waves; on the batched loop, swiglu_splits with 4 waves.
bool gemv_stream();
GemvPlan swiglu_plan(int64_t F, int64_t K);

// The SwiGLU kernel streams two row groups per work item, so it takes half the splits
// a plain GEMV of F rows would (measured on Llama-3-8B's 14336 x 4096 pair: 2 splits
// 1.10 ms per 32 layers, 5 splits 1.15, 3 splits 1.14, none 1.22).
int swiglu_splits(int64_t F, int64_t K) {
    const int s = choose_splits(F, K) / 2;
    return s < 1 ? 1 : s;
}

GemvPlan swiglu_plan(int64_t F, int64_t K) {
    if (!gemv_stream()) return {swiglu_splits(F, K), 4};
    GemvPlan p = plan_gemv(2 * F, K);
    p.waves = std::min(p.waves, 8);   // two row groups per position: 16 waves would spill
    return p;
}

size_t workspace_for(int M, int64_t N, int64_t K, int S) {
    (void)K;
    if (S <= 1) return 0;
    return (size_t)S * M * N * sizeof(float);
}

// Q4MI_GEMV_STREAM=0 selects the batched loop (gemv_rows) instead of the rolling
// pipeline (gemv_rows_stream), for experiments.
bool gemv_stream() {
    static const bool on = [] {
        const char* e = getenv("Q4MI_GEMV_STREAM");
        return !(e && e[0] == '0');
    }();
    return on;
}

template <int NTL, int WAVES, bool STREAM>
void launch_swiglu_ws(bool xf32, dim3 grid, hipStream_t st, const SwigluParams& P) {
    const dim3 block(64 * WAVES);
    if constexpr (STREAM && NTL == 1) {
        if (P.xn) {   // the row normalised into LDS (swiglu_impl checked that it applies)
            hipLaunchKernelGGL((gemv_swiglu_kernel<1, false, true, WAVES, true, true>), grid, block, 0, st, P);
            return;
        }
    }
    if (P.nw) hipLaunchKernelGGL((gemv_swiglu_kernel<NTL, false, true, WAVES, STREAM>), grid, block, 0, st, P);
    else if (xf32) hipLaunchKernelGGL((gemv_swiglu_kernel<NTL, true, false, WAVES, STREAM>), grid, block, 0, st, P);
    else hipLaunchKernelGGL((gemv_swiglu_kernel<NTL, false, false, WAVES, STREAM>), grid, block, 0, st, P);
}

template <int NTL>
void launch_swiglu(bool xf32, bool stream, int waves, dim3 grid, hipStream_t st, const SwigluParams& P) {
    if (!stream) launch_swiglu_ws<NTL, 4, false>(xf32, grid, st, P);
    else if (waves >= 8) launch_swiglu_ws<NTL, 8, true>(xf32, grid, st, P);
    else launch_swiglu_ws<NTL, 4, true>(xf32, grid, st, P);
}

template <int NTL>
void launch_pair(bool xf32, dim3 grid, hipStream_t st, const GemvParams& P, const uint8_t* lo) {
    if (xf32) hipLaunchKernelGGL((gemv_pair_kernel<NTL, true>), grid, dim3(256), 0, st, P, lo);
    else hipLaunchKernelGGL((gemv_pair_kernel<NTL, false>), grid, dim3(256), 0, st, P, lo);
}

template <int NTL, int WAVES, bool Q40, bool STREAM>
void launch_gemv_ws(bool xf32, dim3 grid, hipStream_t st, const GemvParams& P) {
    if constexpr (!Q40 && STREAM && NTL == 1) {
        if (P.xn) {   // the row normalised into LDS (gemv_impl checked that it applies)
            hipLaunchKernelGGL((gemv_kernel<1, false, WAVES, false, true, true, true>), grid, dim3(64 * WAVES), 0, st,
                               P);
            return;
        }
    }
    if constexpr (!Q40) {
        if (P.nw) {
            hipLaunchKernelGGL((gemv_kernel<NTL, false, WAVES, false, true, STREAM>), grid, dim3(64 * WAVES), 0, st,
                               P);
            return;
        }
    }
    if (xf32) hipLaunchKernelGGL((gemv_kernel<NTL, true, WAVES, Q40, false, STREAM>), grid, dim3(64 * WAVES), 0, st, P);
    else hipLaunchKernelGGL((gemv_kernel<NTL, false, WAVES, Q40, false, STREAM>), grid, dim3(64 * WAVES), 0, st, P);
}

template <int NTL, int WAVES, bool Q40>
void launch_gemv_w(bool xf32, dim3 grid, hipStream_t st, const GemvParams& P) {
    if (gemv_stream()) launch_gemv_ws<NTL, WAVES, Q40, true>(xf32, grid, st, P);
    else launch_gemv_ws<NTL, WAVES, Q40, false>(xf32, grid, st, P);
}

template <int NTL, bool Q40 = false>
void launch_gemv(bool xf32, int waves, dim3 grid, hipStream_t st, const GemvParams& P) {
    if (waves == 16) launch_gemv_w<NTL, 16, Q40>(xf32, grid, st, P);
    else if (waves == 8) launch_gemv_w<NTL, 8, Q40>(xf32, grid, st, P);
    else launch_gemv_w<NTL, 4, Q40>(xf32, grid, st, P);
}

// fp16 scale words: the rolling loop only (plain activations, M <= 16).
template <int NTL>
void launch_gemv_f16s(bool xf32, int waves, dim3 grid, hipStream_t st, const GemvParams& P) {
    const dim3 b(64 * waves);
    if (waves == 16) {
        if (xf32) hipLaunchKernelGGL((gemv_kernel<NTL, true, 16, false, false, true, false, true>), grid, b, 0, st, P);
        else hipLaunchKernelGGL((gemv_kernel<NTL, false, 16, false, false, true, false, true>), grid, b, 0, st, P);
    } else if (waves == 8) {
        if (xf32) hipLaunchKernelGGL((gemv_kernel<NTL, true, 8, false, false, true, false, true>), grid, b, 0, st, P);
        else hipLaunchKernelGGL((gemv_kernel<NTL, false, 8, false, false, true, false, true>), grid, b, 0, st, P);
    } else {
        if (xf32) hipLaunchKernelGGL((gemv_kernel<NTL, true, 4, false, false, true, false, true>), grid, b, 0, st, P);
        else hipLaunchKernelGGL((gemv_kernel<NTL, false, 4, false, false, true, false, true>), grid, b, 0, st, P);
    }
}

template <int NTL2, int WAVES>
void launch_tb2_w(bool xf32, dim3 grid, hipStream_t st, const GemvParams& P) {
    if (xf32) hipLaunchKernelGGL((gemv_tb2_kernel<NTL2, true, WAVES>), grid, dim3(64 * WAVES), 0, st, P);
    else hipLaunchKernelGGL((gemv_tb2_kernel<NTL2, false, WAVES>), grid, dim3(64 * WAVES), 0, st, P);
}

template <int NTL2>
void launch_tb2(bool xf32, int waves, dim3 grid, hipStream_t st, const GemvParams& P) {
    if (waves == 16) launch_tb2_w<NTL2, 16>(xf32, grid, st, P);
    else if (waves == 8) launch_tb2_w<NTL2, 8>(xf32, grid, st, P);
    else launch_tb2_w<NTL2, 4>(xf32, grid, st, P);
}



template <int NTL>
void launch_q4k(bool xf32, dim3 grid, hipStream_t st, const GemvParams& P) {
    if (xf32) hipLaunchKernelGGL((q4k_gemv_kernel<NTL, true>), grid, dim3(256), 0, st, P);
    else hipLaunchKernelGGL((q4k_gemv_kernel<NTL, false>), grid, dim3(256), 0, st, P);
}

template <int NTL>
void launch_q8n(bool xf32, dim3 grid, hipStream_t st, const GemvParams& P) {
    if (xf32) hipLaunchKernelGGL((q8n_gemv_kernel<NTL, true>), grid, dim3(256), 0, st, P);
    else hipLaunchKernelGGL((q8n_gemv_kernel<NTL, false>), grid, dim3(256), 0, st, P);
}

}  // namespace

// The plain GEMV and the q8 pair kernel share this query: it covers both plans.
extern "C" size_t q4_gemv_workspace_bytes(int M, int64_t N, int64_t K) {
    if (M < 1 || M > kMaxGemvTokens || N <= 0 || K <= 0 || N % 64 || K % 32) return 0;
    const size_t a = workspace_for(M, N, K, plan_gemv(N, K).S), b = workspace_for(M, N, K, choose_splits(N, K));
    return a > b ? a : b;
}

namespace {

struct NormSpec {
    const void* w = nullptr;   // RMSNorm weight [K]; null: x is the GEMV's input as given
    int w_bf16 = 0;
    float eps = 0.f;
    const float* acc_part = nullptr;   // the deferred reduction (gemv_kernel's XN): x = res + part
    int acc_S = 0;
    float* x_out = nullptr;            // non-null: a deferred-reduction call
};

// A split GEMV's workgroups store their partial sums to [ws, ws + ws_used) while other
// workgroups still read x and the deferred planes, workgroup 0 writes x_out, and the reduce
// launch then writes out (out_bytes) from the partials: none of those may share a byte with
// the partials, or the result depends on timing.
bool split_ws_conflict(const void* ws, int64_t ws_used, const void* x, int64_t x_bytes, const NormSpec& nrm,
                       const void* out, int64_t out_bytes, int M, int64_t K) {
    const int64_t row_bytes = (int64_t)M * K * 4;
    return overlaps(ws, ws_used, x, x_bytes) || overlaps(ws, ws_used, nrm.acc_part, nrm.acc_S * row_bytes) ||
           overlaps(ws, ws_used, nrm.x_out, row_bytes) || overlaps(ws, ws_used, out, out_bytes);
}

// x_out = res + the S partial planes [S][MK], in stage_norm_acc_row's order (S = 1: res +
// part; S > 1: split_reduce's; S = 0: res): the unfused form of the deferred reduction.
__global__ __launch_bounds__(256) void acc_reduce_kernel(const float* __restrict__ res, const float* __restrict__ part,
                                                         int S, int64_t MK, float* __restrict__ x_out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= MK) return;
    float x;
    if (S == 1) {
        x = res[i] + part[i];
    } else {
        // loads batched eight planes at a time (issued together), added in split order
        float sum = 0.f;
        for (int q = 0; q < S; q += 8) {
            float t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) t[u] = q + u < S ? part[(int64_t)(q + u) * MK + i] : 0.f;
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (q + u < S) sum += t[u];
        }
        x = S == 0 ? res[i] : res[i] + sum;
    }
    x_out[i] = x;
}

// CUs of the current device (256 when none is visible).
int cus_of_device() {
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

// The row normalised once into LDS by every workgroup (the XN kernels) applies: the rolling
// loop, one row, K <= 4096, and a grid of at most one workgroup per CU. Every workgroup
// reads the whole row (and a deferred reduction's planes) before its first tile; past one
// workgroup per CU those reads repeat and sit in front of each later workgroup's tiles
// (lm_head 128256 x 4096, 2004 workgroups: 67.0 against 65.8 us for the per-position
// normalisation with no planes, 82.8 against 65.8 + a reduce launch with 16; qkv 6144 x
// 4096, 96 workgroups: 9.8 against 10.5 us).
bool acc_fused(int M, int64_t K, int64_t workgroups) {
    return gemv_stream() && M == 1 && K <= kXnElems && workgroups <= cus_of_device();
}

// The plain norm GEMVs also normalise the row once into LDS where the fused deferred form
// applies (S = 0: x = res); Q4MI_NORM_XN=0 keeps them on the per-position normalisation.
// A decode step measured 1.472 against 1.519 ms: the row's loads go out together with the
// norm weight's in one trip, and the K loop then loads weights only.
bool norm_xn() {
    static const bool on = [] {
        const char* e = getenv("Q4MI_NORM_XN");
        return !(e && atoi(e) == 0);
    }();
    return on;
}

constexpr int kMaxAccSplits = 16;   // partial planes a deferred reduction takes

// Vocabulary-sized norm GEMVs (at least kRowNormWgs workgroups, several per CU) normalise the
// rows once, with q4_rmsnorm_add's kernel, into the workspace (bf16, after the split partials)
// and run the plain GEMV over them. Normalising per position inside such a GEMV repeats the
// rows' loads, the norm weight's and the 1/rms in every workgroup: lm_head 128256 x 4096 at
// M = 1 took 66.9 us that way against 48.8 us for the plain GEMV. The bits are the same: the
// per-position form is q4_rmsnorm_add's arithmetic. A workspace below
// q4_gemv_rmsnorm_workspace_bytes keeps the per-position form.
constexpr int64_t kRowNormWgs = 1024;

bool row_norm_first(int64_t N, int S) { return (N / 64) * S >= kRowNormWgs; }

size_t row_norm_offset(int M, int64_t N, int64_t K, int S) {
    return (workspace_for(M, N, K, S) + 255) & ~(size_t)255;
}

int gemv_impl(const uint8_t* packed, const void* x, int x_dtype, const float* res, float* y, int M, int64_t N,
              int64_t K, void* workspace, size_t workspace_bytes, void* stream, const uint8_t* lo = nullptr,
              bool q40 = false, NormSpec nrm = {}, bool f16s = false) {
    if (x_dtype != Q4MI_F32 && x_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (M < 0 || M > (lo || q40 || f16s ? 16 : kMaxGemvTokens)) return Q4MI_E_RANGE;
    if (N < 0 || K <= 0 || N % 64 || K % 32) return Q4MI_E_SHAPE;
    if (M == 0 || N == 0) return Q4MI_OK;   // nothing to compute
    if (!packed || !x || !y) return Q4MI_E_ARG;
    if (misaligned16(packed) || misaligned16(x) || misaligned16(y) || misaligned16(workspace)) return Q4MI_E_ARG;
    const GemvPlan plan = lo ? GemvPlan{choose_splits(N, K), 4} : plan_gemv(N, K);
    const int S = plan.S;
    if (S > 1) {   // the documented contract: at least what the query reports (checked before any launch)
        if (!workspace || workspace_bytes < q4_gemv_workspace_bytes(M, N, K)) return Q4MI_E_WORKSPACE;
        if (split_ws_conflict(workspace, (int64_t)workspace_for(M, N, K, S), x,
                              (int64_t)M * K * (x_dtype == Q4MI_F32 ? 4 : 2), nrm, y, (int64_t)M * N * 4, M, K))
            return Q4MI_E_ARG;
    }
    const bool fused = acc_fused(M, K, (N / 64) * S);
    // the vocabulary-sized form: the bf16 rows in the workspace, past the split partials
    uint8_t* xn_rows = nullptr;
    if (nrm.w && !fused && !lo && !q40 && !f16s && row_norm_first(N, S) && workspace) {
        const size_t off = row_norm_offset(M, N, K, S);
        const int64_t rb = (int64_t)M * K * 2, xb = (int64_t)M * K * 4;
        uint8_t* const xn = (uint8_t*)workspace + off;
        if (workspace_bytes >= off + (size_t)rb && !overlaps(xn, rb, x, xb) && !overlaps(xn, rb, y, (int64_t)M * N * 4) &&
            !overlaps(xn, rb, nrm.x_out, xb) && !overlaps(xn, rb, nrm.acc_part, (int64_t)nrm.acc_S * xb))
            xn_rows = xn;
    }
    if (xn_rows && nrm.x_out && K <= 256 * 16) {   // reduce and normalise in one launch
        const int rc = rmsnorm_planes((const float*)x, nrm.acc_part, nrm.acc_S, nrm.w, nrm.w_bf16 ? Q4MI_BF16 : Q4MI_F32,
                                      nrm.x_out, xn_rows, M, K, nrm.eps, stream);
        if (rc != Q4MI_OK) return rc;
        x = xn_rows;
        x_dtype = Q4MI_BF16;
        nrm = NormSpec{};
    }
    if (nrm.x_out && !fused) {   // deferred reduction, unfused: reduce into x_out, then the norm GEMV
        const int64_t MK = (int64_t)M * K;
        hipLaunchKernelGGL(acc_reduce_kernel, dim3((unsigned)ceil_div(MK, 256)), dim3(256), 0, (hipStream_t)stream,
                           (const float*)x, nrm.acc_part, nrm.acc_S, MK, nrm.x_out);
        if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
        x = nrm.x_out;
        nrm.x_out = nullptr;
        nrm.acc_part = nullptr;
        nrm.acc_S = 0;
    }
    if (xn_rows && nrm.w) {
        const int rc = q4_rmsnorm_add((const float*)x, nullptr, nrm.w, nrm.w_bf16 ? Q4MI_BF16 : Q4MI_F32, nullptr,
                                      xn_rows, Q4MI_BF16, M, K, nrm.eps, stream);
        if (rc != Q4MI_OK) return rc;
        x = xn_rows;
        x_dtype = Q4MI_BF16;
        nrm = NormSpec{};
    }
    GemvParams P{};
    P.packed = packed;
    P.x = x;
    P.y = y;
    P.M = M;
    P.S = S;
    P.N = N;
    P.K = K;
    P.res = res;
    P.nw = nrm.w;
    P.nw_bf16 = nrm.w_bf16;
    P.eps = nrm.eps;
    P.acc_part = nrm.acc_part;
    P.acc_S = nrm.acc_S;
    P.x_out = nrm.x_out;
    P.xn = nrm.x_out || (nrm.w && norm_xn() && fused);
    if (S > 1) P.part = (float*)workspace;
    const dim3 grid((unsigned)((N / 64) * S));
    const hipStream_t st = (hipStream_t)stream;
    const bool xf32 = x_dtype == Q4MI_F32;
    if (f16s) {
        switch ((M + 3) / 4) {
            case 1: launch_gemv_f16s<1>(xf32, plan.waves, grid, st, P); break;
            case 2: launch_gemv_f16s<2>(xf32, plan.waves, grid, st, P); break;
            case 3: launch_gemv_f16s<3>(xf32, plan.waves, grid, st, P); break;
            default: launch_gemv_f16s<4>(xf32, plan.waves, grid, st, P); break;
        }
    } else if (lo) {
        switch ((M + 3) / 4) {
            case 1: launch_pair<1>(xf32, grid, st, P, lo); break;
            case 2: launch_pair<2>(xf32, grid, st, P, lo); break;
            case 3: launch_pair<3>(xf32, grid, st, P, lo); break;
            default: launch_pair<4>(xf32, grid, st, P, lo); break;
        }
    } else if (q40) {
        const int waves = plan.waves;
        switch ((M + 3) / 4) {
            case 1: launch_gemv<1, true>(xf32, waves, grid, st, P); break;
            case 2: launch_gemv<2, true>(xf32, waves, grid, st, P); break;
            case 3: launch_gemv<3, true>(xf32, waves, grid, st, P); break;
            default: launch_gemv<4, true>(xf32, waves, grid, st, P); break;
        }
    } else {
        const int waves = plan.waves;
        switch ((M + 3) / 4) {
            case 1: launch_gemv<1>(xf32, waves, grid, st, P); break;
            case 2: launch_gemv<2>(xf32, waves, grid, st, P); break;
            case 3: launch_gemv<3>(xf32, waves, grid, st, P); break;
            case 4: launch_gemv<4>(xf32, waves, grid, st, P); break;
            case 5: launch_tb2<1>(xf32, waves, grid, st, P); break;
            default: launch_tb2<2>(xf32, waves, grid, st, P); break;
        }
    }
    if (S > 1) {
        if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
        const int64_t MN = (int64_t)M * N;
        hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)ceil_div(MN, 256)), dim3(256), 0, st, P.part, y, MN,
                           S, res);
    }
    return launch_status();
}

}  // namespace

extern "C" int q4_gemv(const uint8_t* packed, const void* x, int x_dtype, float* y, int M, int64_t N, int64_t K,
                       void* workspace, size_t workspace_bytes, void* stream) {
    return gemv_impl(packed, x, x_dtype, nullptr, y, M, N, K, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// q4_gemv_noalloc: q4_gemv with its K-split partial sums in a file-scope device array
// instead of a caller workspace, for callers that cannot allocate device memory.
//
// The partials of a split call are [S][M][N] f32; both split plans (plan_gemv, choose_splits)
// keep S * N/64 below 2048 for every N, so with M <= 16 they never exceed 2046 * 64 * 16 * 4 =
// 8,380,416 bytes, and Q4MI_NOALLOC_SCRATCH_BYTES (8 MiB) covers every shape. The gemv
// kernel writes every partial it later reduces, so nothing needs clearing between calls.
// Each device holds its own copy of the array; its address is read once per device
// (hipGetSymbolAddress, with that device current) and kept here. Calls that overlap on
// one device (other streams, other host threads) share the array and race.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[Q4MI_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up on its first use there.
int scratch_for_current_device(void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return Q4MI_E_LAUNCH;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return Q4MI_E_LAUNCH;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return Q4MI_OK;
}

}  // namespace

extern "C" int q4_gemv_noalloc(const uint8_t* packed, const void* x, int x_dtype, float* y, int M, int64_t N,
                               int64_t K, void* stream) {
    if (x_dtype != Q4MI_F32 && x_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (M < 0 || M > 16) return Q4MI_E_RANGE;
    if (N < 0 || K <= 0 || N % 64 || K % 32) return Q4MI_E_SHAPE;
    if (M == 0 || N == 0) return Q4MI_OK;
    const size_t need = q4_gemv_workspace_bytes(M, N, K);
    if (need > (size_t)Q4MI_NOALLOC_SCRATCH_BYTES) return Q4MI_E_WORKSPACE;
    void* ws = nullptr;
    if (need > 0) {
        const int st = scratch_for_current_device(&ws);
        if (st != Q4MI_OK) return st;
    }
    return gemv_impl(packed, x, x_dtype, nullptr, y, M, N, K, ws, need, stream);
}

extern "C" int q4_gemv_residual(const uint8_t* packed, const void* x, int x_dtype, const float* residual, float* y,
                                int M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes, void* stream) {
    if (!residual && M > 0 && N > 0) return Q4MI_E_ARG;
    return gemv_impl(packed, x, x_dtype, residual, y, M, N, K, workspace, workspace_bytes, stream);
}

extern "C" int q4_gemv_q8(const uint8_t* hi, const uint8_t* lo, const void* x, int x_dtype, const float* residual,
                          float* y, int M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
                          void* stream) {
    if (M > 0 && N > 0 && (!lo || misaligned16(lo))) return Q4MI_E_ARG;
    return gemv_impl(hi, x, x_dtype, residual, y, M, N, K, workspace, workspace_bytes, stream, lo);
}

// The GEMV over fp16 scale words (q4_repack scale_mode 1): q4_gemv's work items, plan,
// workspace and arithmetic, d and m converted from fp16 instead of bf16.
extern "C" int q4_gemv_fp16s(const uint8_t* packed, const void* x, int x_dtype, const float* residual, float* y,
                             int M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes, void* stream) {
    return gemv_impl(packed, x, x_dtype, residual, y, M, N, K, workspace, workspace_bytes, stream, nullptr, false,
                     NormSpec{}, true);
}

// The mx0 (Q4_0-native) GEMV: q4_gemv's work items, plan and workspace over 1152 B tiles.
extern "C" int q4_gemv_q40(const uint8_t* packed, const void* x, int x_dtype, const float* residual, float* y, int M,
                           int64_t N, int64_t K, void* workspace, size_t workspace_bytes, void* stream) {
    return gemv_impl(packed, x, x_dtype, residual, y, M, N, K, workspace, workspace_bytes, stream, nullptr, true);
}

// Norm-fused forms: X = bf16(RMSNorm(x) * norm_w) from the f32 residual stream x, the same
// bits as q4_rmsnorm_add (bf16 out, no add) followed by q4_gemv / q4_gemv_swiglu.
static int norm_args(const float* x, const void* norm_w, int norm_w_dtype, float eps, int M, int64_t K,
                     NormSpec* out) {
    if (norm_w_dtype != Q4MI_F32 && norm_w_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (!(eps >= 0.0f)) return Q4MI_E_ARG;
    if (M > 16) return Q4MI_E_RANGE;
    if (K > 16384) return Q4MI_E_RANGE;
    if (M > 0 && (!x || !norm_w || misaligned16(norm_w))) return Q4MI_E_ARG;
    out->w = norm_w;
    out->w_bf16 = norm_w_dtype == Q4MI_BF16;
    out->eps = eps;
    return Q4MI_OK;
}

extern "C" int q4_gemv_rmsnorm(const uint8_t* packed, const float* x, const void* norm_w, int norm_w_dtype, float eps,
                               float* y, int M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
                               void* stream) {
    NormSpec nrm;
    const int a = norm_args(x, norm_w, norm_w_dtype, eps, M, K, &nrm);
    if (a != Q4MI_OK) return a;
    return gemv_impl(packed, x, Q4MI_F32, nullptr, y, M, N, K, workspace, workspace_bytes, stream, nullptr, false,
                     nrm);
}

extern "C" size_t q4_gemv_rmsnorm_workspace_bytes(int M, int64_t N, int64_t K) {
    const size_t base = q4_gemv_workspace_bytes(M, N, K);
    if (base == 0 && (M < 1 || M > kMaxGemvTokens || N <= 0 || K <= 0 || N % 64 || K % 32)) return 0;
    const int S = plan_gemv(N, K).S;
    if (!row_norm_first(N, S)) return base;
    const size_t need = row_norm_offset(M, N, K, S) + (size_t)M * K * 2;
    return need > base ? need : base;
}

extern "C" size_t q4_gemv_swiglu_workspace_bytes(int M, int64_t F, int64_t K) {
    if (M < 1 || M > 16 || F <= 0 || K <= 0 || F % 64 || K % 32) return 0;
    const int S = std::max(swiglu_splits(F, K), swiglu_plan(F, K).S);   // either loop's plan
    return S > 1 ? (size_t)S * M * 2 * F * sizeof(float) : 0;
}

static int swiglu_impl(const uint8_t* gate, const uint8_t* up, const void* x, int x_dtype, void* h, int h_dtype,
                       int M, int64_t F, int64_t K, void* workspace, size_t workspace_bytes, void* stream,
                       NormSpec nrm = {}) {
    if (x_dtype != Q4MI_F32 && x_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (h_dtype != Q4MI_F32 && h_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (M < 0 || M > 16) return Q4MI_E_RANGE;
    if (F < 0 || K <= 0 || F % 64 || K % 32) return Q4MI_E_SHAPE;
    if (M == 0 || F == 0) return Q4MI_OK;
    if (!gate || !up || !x || !h) return Q4MI_E_ARG;
    if (misaligned16(gate) || misaligned16(up) || misaligned16(x) || misaligned16(workspace)) return Q4MI_E_ARG;
    if (((uintptr_t)h & (h_dtype == Q4MI_BF16 ? 1 : 3)) != 0) return Q4MI_E_ARG;
    const GemvPlan plan = swiglu_plan(F, K);
    const int S = plan.S;
    if (S > 1) {   // checked before any launch
        if (!workspace || workspace_bytes < (size_t)S * M * 2 * F * sizeof(float)) return Q4MI_E_WORKSPACE;
        if (split_ws_conflict(workspace, (int64_t)S * M * 2 * F * 4, x, (int64_t)M * K * (x_dtype == Q4MI_F32 ? 4 : 2),
                              nrm, h, (int64_t)M * F * (h_dtype == Q4MI_BF16 ? 2 : 4), M, K))
            return Q4MI_E_ARG;
    }
    const bool fused = acc_fused(M, K, (F / 64) * S);
    if (nrm.x_out && !fused) {   // deferred reduction, unfused: reduce into x_out, then the norm GEMV
        const int64_t MK = (int64_t)M * K;
        hipLaunchKernelGGL(acc_reduce_kernel, dim3((unsigned)ceil_div(MK, 256)), dim3(256), 0, (hipStream_t)stream,
                           (const float*)x, nrm.acc_part, nrm.acc_S, MK, nrm.x_out);
        if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
        x = nrm.x_out;
        nrm.x_out = nullptr;
        nrm.acc_part = nullptr;
        nrm.acc_S = 0;
    }
    SwigluParams P{};
    P.gate = gate;
    P.up = up;
    P.x = x;
    P.h = h;
    P.h_bf16 = h_dtype == Q4MI_BF16;
    P.M = M;
    P.S = S;
    P.F = F;
    P.K = K;
    P.nw = nrm.w;
    P.nw_bf16 = nrm.w_bf16;
    P.eps = nrm.eps;
    P.acc_part = nrm.acc_part;
    P.acc_S = nrm.acc_S;
    P.x_out = nrm.x_out;
    P.xn = nrm.x_out || (nrm.w && norm_xn() && fused);
    if (S > 1) P.part = (float*)workspace;
    const dim3 grid((unsigned)((F / 64) * S));
    const hipStream_t st = (hipStream_t)stream;
    const bool xf32 = x_dtype == Q4MI_F32;
    const bool sm = gemv_stream();
    switch ((M + 3) / 4) {
        case 1: launch_swiglu<1>(xf32, sm, plan.waves, grid, st, P); break;
        case 2: launch_swiglu<2>(xf32, sm, plan.waves, grid, st, P); break;
        case 3: launch_swiglu<3>(xf32, sm, plan.waves, grid, st, P); break;
        default: launch_swiglu<4>(xf32, sm, plan.waves, grid, st, P); break;
    }
    if (S > 1) {
        if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
        const int64_t MF = (int64_t)M * F;
        hipLaunchKernelGGL(swiglu_reduce_kernel, dim3((unsigned)ceil_div(MF, 256)), dim3(256), 0, st, P.part, h,
                           P.h_bf16, M, F, S);
    }
    return launch_status();
}

extern "C" int q4_gemv_swiglu(const uint8_t* gate, const uint8_t* up, const void* x, int x_dtype, void* h,
                              int h_dtype, int M, int64_t F, int64_t K, void* workspace, size_t workspace_bytes,
                              void* stream) {
    return swiglu_impl(gate, up, x, x_dtype, h, h_dtype, M, F, K, workspace, workspace_bytes, stream);
}

extern "C" int q4_gemv_swiglu_rmsnorm(const uint8_t* gate, const uint8_t* up, const float* x, const void* norm_w,
                                      int norm_w_dtype, float eps, void* h, int h_dtype, int M, int64_t F, int64_t K,
                                      void* workspace, size_t workspace_bytes, void* stream) {
    NormSpec nrm;
    const int a = norm_args(x, norm_w, norm_w_dtype, eps, M, K, &nrm);
    if (a != Q4MI_OK) return a;
    return swiglu_impl(gate, up, x, Q4MI_F32, h, h_dtype, M, F, K, workspace, workspace_bytes, stream, nrm);
}

// ---------------------------------------------------------------------------
// The K-split reduction deferred to the consumer: q4_gemv_partials leaves a split GEMV's
// partial sums; the norm-fused GEMVs' _acc forms add them to the residual stream in
// split_reduce's order (so the result is the one q4_gemv_residual + the norm GEMV give),
// write that residual to x_out, and normalise it, with no reduce launch in between.

extern "C" int q4_gemv_split_count(int64_t N, int64_t K) {
    if (N <= 0 || K <= 0 || N % 64 || K % 32) return 0;
    return plan_gemv(N, K).S;
}

extern "C" int q4_gemv_partials(const uint8_t* packed, const void* x, int x_dtype, float* part, int S, int M,
                                int64_t N, int64_t K, void* stream) {
    if (x_dtype != Q4MI_F32 && x_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (M < 0 || M > 16) return Q4MI_E_RANGE;
    if (N < 0 || K <= 0 || N % 64 || K % 32) return Q4MI_E_SHAPE;
    if (S < 1 || S > kMaxAccSplits || S > K / 32) return Q4MI_E_RANGE;
    if (M == 0 || N == 0) return Q4MI_OK;
    if (!packed || !x || !part) return Q4MI_E_ARG;
    if (misaligned16(packed) || misaligned16(x) || misaligned16(part)) return Q4MI_E_ARG;
    GemvParams P{};
    P.packed = packed;
    P.x = x;
    P.y = part;       // S = 1: the unsplit store
    P.part = part;    // S > 1: plane s at part + s M N
    P.M = M;
    P.S = S;
    P.N = N;
    P.K = K;
    // the plain plan's waves when S is its split count (then the planes add up, in split
    // order, to q4_gemv's result bit for bit); other counts take 8
    const GemvPlan plan = plan_gemv(N, K);
    const int waves = S == plan.S ? plan.waves : 8;
    const dim3 grid((unsigned)((N / 64) * S));
    const hipStream_t st = (hipStream_t)stream;
    const bool xf32 = x_dtype == Q4MI_F32;
    switch ((M + 3) / 4) {
        case 1: launch_gemv<1>(xf32, waves, grid, st, P); break;
        case 2: launch_gemv<2>(xf32, waves, grid, st, P); break;
        case 3: launch_gemv<3>(xf32, waves, grid, st, P); break;
        default: launch_gemv<4>(xf32, waves, grid, st, P); break;
    }
    return launch_status();
}

// out / out_bytes: the GEMV's own output (y or h), written while other workgroups still
// read res and the planes.
static int acc_args(const float* res, const float* part, int S, const float* x_out, const void* out,
                    int64_t out_bytes, int M, int64_t K, NormSpec* nrm) {
    if (S < 0 || S > kMaxAccSplits) return Q4MI_E_RANGE;
    if (M == 0) return Q4MI_OK;
    if (!x_out || (S > 0 && !part)) return Q4MI_E_ARG;
    // workgroup 0 writes x_out while the others read res and the planes
    const int64_t row_bytes = (int64_t)M * K * 4, part_bytes = S > 0 ? S * row_bytes : 0;
    if (overlaps(x_out, row_bytes, res, row_bytes) || overlaps(x_out, row_bytes, part, part_bytes) ||
        overlaps(out, out_bytes, res, row_bytes) || overlaps(out, out_bytes, part, part_bytes) ||
        overlaps(out, out_bytes, x_out, row_bytes))
        return Q4MI_E_ARG;
    if (misaligned16(x_out) || (S > 0 && misaligned16(part))) return Q4MI_E_ARG;
    nrm->acc_part = part;
    nrm->acc_S = S;
    nrm->x_out = (float*)x_out;
    return Q4MI_OK;
}

extern "C" int q4_gemv_rmsnorm_acc(const uint8_t* packed, const float* res, const float* part, int S,
                                   const void* norm_w, int norm_w_dtype, float eps, float* x_out, float* y, int M,
                                   int64_t N, int64_t K, void* workspace, size_t workspace_bytes, void* stream) {
    NormSpec nrm;
    int a = norm_args(res, norm_w, norm_w_dtype, eps, M, K, &nrm);
    if (a != Q4MI_OK) return a;
    if ((a = acc_args(res, part, S, x_out, y, (int64_t)M * N * 4, M, K, &nrm)) != Q4MI_OK) return a;
    return gemv_impl(packed, res, Q4MI_F32, nullptr, y, M, N, K, workspace, workspace_bytes, stream, nullptr, false,
                     nrm);
}

extern "C" int q4_gemv_swiglu_rmsnorm_acc(const uint8_t* gate, const uint8_t* up, const float* res, const float* part,
                                          int S, const void* norm_w, int norm_w_dtype, float eps, float* x_out,
                                          void* h, int h_dtype, int M, int64_t F, int64_t K, void* workspace,
                                          size_t workspace_bytes, void* stream) {
    NormSpec nrm;
    int a = norm_args(res, norm_w, norm_w_dtype, eps, M, K, &nrm);
    if (a != Q4MI_OK) return a;
    if ((a = acc_args(res, part, S, x_out, h, (int64_t)M * F * (h_dtype == Q4MI_BF16 ? 2 : 4), M, K, &nrm)) !=
        Q4MI_OK)
        return a;
    return swiglu_impl(gate, up, res, Q4MI_F32, h, h_dtype, M, F, K, workspace, workspace_bytes, stream, nrm);
}

extern "C" size_t q4_gemv_q4k_workspace_bytes(int M, int64_t N, int64_t K) {
    if (M < 1 || M > 16 || N <= 0 || K <= 0 || N % 64 || K % 256) return 0;
    return workspace_for(M, N, K, q4k_splits(N, K));
}

extern "C" int q4_gemv_q4k(const uint8_t* packed, const void* x, int x_dtype, const float* residual, float* y, int M,
                           int64_t N, int64_t K, void* workspace, size_t workspace_bytes, void* stream) {
    if (x_dtype != Q4MI_F32 && x_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (M < 0 || M > 16) return Q4MI_E_RANGE;
    if (N < 0 || K <= 0 || N % 64 || K % 256) return Q4MI_E_SHAPE;
    if (M == 0 || N == 0) return Q4MI_OK;
    if (!packed || !x || !y) return Q4MI_E_ARG;
    if (misaligned16(packed) || misaligned16(x) || misaligned16(y) || misaligned16(workspace)) return Q4MI_E_ARG;
    const int S = q4k_splits(N, K);
    GemvParams P{};
    P.packed = packed;
    P.x = x;
    P.y = y;
    P.M = M;
    P.S = S;
    P.N = N;
    P.K = K;
    P.res = residual;
    if (S > 1) {
        if (!workspace || workspace_bytes < workspace_for(M, N, K, S)) return Q4MI_E_WORKSPACE;
        P.part = (float*)workspace;
    }
    const dim3 grid((unsigned)((N / 64) * S));
    const hipStream_t st = (hipStream_t)stream;
    const bool xf32 = x_dtype == Q4MI_F32;
    switch ((M + 3) / 4) {
        case 1: launch_q4k<1>(xf32, grid, st, P); break;
        case 2: launch_q4k<2>(xf32, grid, st, P); break;
        case 3: launch_q4k<3>(xf32, grid, st, P); break;
        default: launch_q4k<4>(xf32, grid, st, P); break;
    }
    if (S > 1) {
        if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
        const int64_t MN = (int64_t)M * N;
        hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)ceil_div(MN, 256)), dim3(256), 0, st, P.part, y, MN,
                           S, residual);
    }
    return launch_status();
}

extern "C" size_t q4_gemv_q8_native_workspace_bytes(int M, int64_t N, int64_t K) {
    return q4_gemv_workspace_bytes(M, N, K);
}

extern "C" int q4_gemv_q8_native(const uint8_t* packed, const void* x, int x_dtype, const float* residual, float* y,
                                 int M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes, void* stream) {
    if (x_dtype != Q4MI_F32 && x_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (M < 0 || M > 16) return Q4MI_E_RANGE;
    if (N < 0 || K <= 0 || N % 64 || K % 32) return Q4MI_E_SHAPE;
    if (M == 0 || N == 0) return Q4MI_OK;
    if (!packed || !x || !y) return Q4MI_E_ARG;
    if (misaligned16(packed) || misaligned16(x) || misaligned16(y) || misaligned16(workspace)) return Q4MI_E_ARG;
    const int S = choose_splits(N, K);
    GemvParams P{};
    P.packed = packed;
    P.x = x;
    P.y = y;
    P.M = M;
    P.S = S;
    P.N = N;
    P.K = K;
    P.res = residual;
    if (S > 1) {
        if (!workspace || workspace_bytes < workspace_for(M, N, K, S)) return Q4MI_E_WORKSPACE;
        P.part = (float*)workspace;
    }
    const dim3 grid((unsigned)((N / 64) * S));
    const hipStream_t st = (hipStream_t)stream;
    const bool xf32 = x_dtype == Q4MI_F32;
    switch ((M + 3) / 4) {
        case 1: launch_q8n<1>(xf32, grid, st, P); break;
        case 2: launch_q8n<2>(xf32, grid, st, P); break;
        case 3: launch_q8n<3>(xf32, grid, st, P); break;
        default: launch_q8n<4>(xf32, grid, st, P); break;
    }
    if (S > 1) {
        if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
        const int64_t MN = (int64_t)M * N;
        hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)ceil_div(MN, 256)), dim3(256), 0, st, P.part, y, MN,
                           S, residual);
    }
    return launch_status();
}
