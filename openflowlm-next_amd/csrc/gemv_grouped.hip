// gemv_grouped.hip -- many decode GEMVs in one launch: one workgroup per 64-row group of
// any matrix in a descriptor table (q4_gemv_grouped), the inner loop of gemv_core.h.
//
// Built on its own so that its MFMA accumulators can be kept in VGPRs (the build's
// per-source flags): here that measured faster (the Llama-3-8B sweep at M = 1: 197.1 ->
// 193.6 us for 8 layers), while the same flag on the single-matrix kernels of gemv.hip
// measured slower (native Q4_K gate_up 14.9 -> 21.0 us).
#include <stdlib.h>

#include "gemv_core.h"
#include "q4mi_internal.h"

using namespace q4mi;

namespace {

// K positions in flight per wave on the rolling loop. Same-process A/B over the 225
// Llama-3-8B matrices (graph-free back-to-back launches, bit-identical outputs), µs:
//   M = 1: batched 685.8, depth 4 684.6, 6 698.8, 8 680.1
//   M = 4: 741.0, 740.2, 753.0, 732.9;  M = 16: 1066.7, 1067.6, 1109.3, 1055.6
constexpr int kGroupedUnr = 8;

// F16S: every matrix's scale words hold fp16 d and m (q4_repack scale_mode 1).
template <int NTL, bool XF32, bool STREAM, bool F16S = false>
__global__ __launch_bounds__(256) void gemv_grouped_kernel(const q4_gemv_desc* __restrict__ descs, int count, int M) {
    static_assert(!F16S || STREAM, "fp16 scales: the rolling loop");
    __shared__ float red[kWaves][4][NTL][64];
    const int64_t item = blockIdx.x;
    int lo = 0, hi = count - 1;
    while (lo < hi) {               // last descriptor with item_begin <= item
        const int mid = (lo + hi + 1) >> 1;
        if (descs[mid].item_begin <= item) lo = mid;
        else hi = mid - 1;
    }
    const q4_gemv_desc D = descs[lo];
    const int64_t g = item - D.item_begin;
    if (g < 0 || g >= (D.N >> 6)) return;   // inconsistent total_items: the whole workgroup leaves
    float acc[4][NTL];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < NTL; ++j) acc[r][j] = 0.f;
    if constexpr (STREAM) {
        float acc1[1][4][NTL];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < NTL; ++j) acc1[0][r][j] = 0.f;
        const uint8_t* const gb[1] = {D.packed + g * (D.K >> 5) * kTileBytes};
        gemv_rows_stream<NTL, XF32, 1, kGroupedUnr, kWaves, false, 0, DenseRows, false, F16S>(
            gb, D.x, DenseRows{M}, D.K, 0, (int)(D.K >> 5), acc1);
        gemv_finish<NTL>(acc1[0], red, M, D.y, D.N, g);
    } else {
        gemv_rows<NTL, XF32>(D.packed, D.x, DenseRows{M}, D.K, g, 0, (int)(D.K >> 5), acc);
        gemv_finish<NTL>(acc, red, M, D.y, D.N, g);
    }
}

// NG consecutive 64-row groups of one matrix per workgroup, the token fragment of each K
// position loaded once and shared by the NG groups' tiles (gemv_rows_stream over NG row
// groups). Per group the waves visit the same positions in the same order with the same
// arithmetic as gemv_grouped_kernel's, and the finish sums the waves in the same order, so
// every output is bit-identical to it. Workgroups whose NG items straddle two matrices (or
// the end) take their items one at a time.
template <int NTL, bool XF32, int NG, int UNR>
__global__ __launch_bounds__(256) void gemv_grouped_ng_kernel(const q4_gemv_desc* __restrict__ descs, int count,
                                                              int M, int64_t total_items) {
    __shared__ float red[kWaves][4][NTL][64];
    auto find = [&](int64_t item) {
        int lo = 0, hi = count - 1;
        while (lo < hi) {           // last descriptor with item_begin <= item
            const int mid = (lo + hi + 1) >> 1;
            if (descs[mid].item_begin <= item) lo = mid;
            else hi = mid - 1;
        }
        return lo;
    };
    const int64_t item0 = (int64_t)blockIdx.x * NG;
    const q4_gemv_desc D = descs[find(item0)];
    const int64_t g0 = item0 - D.item_begin;
    if (g0 < 0) return;
    const int KB = (int)(D.K >> 5);
    if (g0 + NG <= (D.N >> 6) && item0 + NG <= total_items) {
        float acc[NG][4][NTL];
#pragma unroll
        for (int i = 0; i < NG; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int j = 0; j < NTL; ++j) acc[i][r][j] = 0.f;
        const uint8_t* gb[NG];
#pragma unroll
        for (int i = 0; i < NG; ++i) gb[i] = D.packed + (g0 + i) * KB * kTileBytes;
        gemv_rows_stream<NTL, XF32, NG, UNR, kWaves, false, 0, DenseRows>(gb, D.x, DenseRows{M}, D.K, 0, KB, acc);
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            if (i) __syncthreads();                 // red is rewritten by the next finish
            gemv_finish<NTL>(acc[i], red, M, D.y, D.N, g0 + i);
        }
        return;
    }
    for (int i = 0; i < NG; ++i) {                  // straddling workgroup: item by item
        const int64_t item = item0 + i;
        if (item >= total_items) break;
        const q4_gemv_desc E = descs[find(item)];
        const int64_t g = item - E.item_begin;
        if (g < 0 || g >= (E.N >> 6)) break;
        float acc1[1][4][NTL];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < NTL; ++j) acc1[0][r][j] = 0.f;
        const uint8_t* const gb1[1] = {E.packed + g * (E.K >> 5) * kTileBytes};
        gemv_rows_stream<NTL, XF32, 1, kGroupedUnr, kWaves, false, 0, DenseRows>(gb1, E.x, DenseRows{M}, E.K, 0,
                                                                                 (int)(E.K >> 5), acc1);
        if (i) __syncthreads();
        gemv_finish<NTL>(acc1[0], red, M, E.y, E.N, g);
    }
}

template <int NTL, bool XF32, int NG, int UNR>
void launch_ng(dim3 grid, hipStream_t st, const q4_gemv_desc* d, int count, int M) {
    const int64_t items = grid.x;
    hipLaunchKernelGGL((gemv_grouped_ng_kernel<NTL, XF32, NG, UNR>), dim3((unsigned)((items + NG - 1) / NG)),
                       dim3(256), 0, st, d, count, M, items);
}

// Q4MI_GROUPED_STREAM=0 keeps the batched loop (experiments).
bool grouped_stream() {
    static const bool on = [] {
        const char* e = getenv("Q4MI_GROUPED_STREAM");
        return !(e && e[0] == '0');
    }();
    return on;
}

template <int NTL, bool STREAM>
void launch_grouped_s(bool xf32, dim3 grid, hipStream_t st, const q4_gemv_desc* d, int count, int M) {
    if (xf32) hipLaunchKernelGGL((gemv_grouped_kernel<NTL, true, STREAM>), grid, dim3(256), 0, st, d, count, M);
    else hipLaunchKernelGGL((gemv_grouped_kernel<NTL, false, STREAM>), grid, dim3(256), 0, st, d, count, M);
}

template <int NTL>
void launch_grouped(bool xf32, bool f16s, dim3 grid, hipStream_t st, const q4_gemv_desc* d, int count, int M) {
    // M = 2..16 on bf16 x: the fragment shared by 2 (M <= 8, 4 positions in flight) or 4
    // (M > 8, 2 in flight) row groups. Same-process sweeps over the 225 Llama-3-8B matrices
    // (ms, against the one-group kernel): M = 2 0.716 / 0.759, M = 4 0.744 / 0.759, M = 8
    // 0.810 / 0.881, M = 12 0.877 / 0.992, M = 16 0.920 / 1.072. Four groups at M <= 8, or
    // two at M > 8, measured slower than the choice here; M = 1 keeps the one-group kernel.
    if (M > 1 && !f16s && !xf32) {
        if constexpr (NTL <= 2) launch_ng<NTL, false, 2, 4>(grid, st, d, count, M);
        else launch_ng<NTL, false, 4, 2>(grid, st, d, count, M);
        return;
    }
    if (f16s) {
        if (xf32) hipLaunchKernelGGL((gemv_grouped_kernel<NTL, true, true, true>), grid, dim3(256), 0, st, d, count, M);
        else hipLaunchKernelGGL((gemv_grouped_kernel<NTL, false, true, true>), grid, dim3(256), 0, st, d, count, M);
    } else if (grouped_stream()) {
        launch_grouped_s<NTL, true>(xf32, grid, st, d, count, M);
    } else {
        launch_grouped_s<NTL, false>(xf32, grid, st, d, count, M);
    }
}

int grouped_impl(const q4_gemv_desc* descs, int count, int64_t total_items, int M, int x_dtype, void* stream,
                 bool f16s) {
    if (!descs || count <= 0 || total_items <= 0) return Q4MI_E_ARG;
    if (x_dtype != Q4MI_F32 && x_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (M < 1 || M > 16) return Q4MI_E_RANGE;
    if (total_items > 0x7FFFFFFF) return Q4MI_E_RANGE;
    const dim3 grid((unsigned)total_items);
    const hipStream_t st = (hipStream_t)stream;
    const bool xf32 = x_dtype == Q4MI_F32;
    switch ((M + 3) / 4) {
        case 1: launch_grouped<1>(xf32, f16s, grid, st, descs, count, M); break;
        case 2: launch_grouped<2>(xf32, f16s, grid, st, descs, count, M); break;
        case 3: launch_grouped<3>(xf32, f16s, grid, st, descs, count, M); break;
        default: launch_grouped<4>(xf32, f16s, grid, st, descs, count, M); break;
    }
    return launch_status();
}

}  // namespace

extern "C" int q4_gemv_grouped(const q4_gemv_desc* descs, int count, int64_t total_items, int M, int x_dtype,
                               void* stream) {
    return grouped_impl(descs, count, total_items, M, x_dtype, stream, false);
}

// The same sweep over matrices packed with fp16 scale words (q4_repack scale_mode 1).
extern "C" int q4_gemv_grouped_fp16s(const q4_gemv_desc* descs, int count, int64_t total_items, int M, int x_dtype,
                                     void* stream) {
    return grouped_impl(descs, count, total_items, M, x_dtype, stream, true);
}
