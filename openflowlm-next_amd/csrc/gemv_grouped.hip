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
