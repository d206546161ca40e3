// peaks.hip -- on-box reference points for the roofline fractions: the HBM read rate a
// plain streaming kernel reaches, and the dense fp16 MFMA rate of a loop that does nothing
// else. Neither is on the reference's path; the bench reports both beside the vendor peaks
// (8 TB/s, 2.5 PFLOP/s) so a fraction of nameplate can be read against what this box
// sustains.
#include "q4mi_device.h"
#include "q4mi_internal.h"

using namespace q4mi;

namespace {

constexpr int kReadUnroll = 8;   // 16-byte loads in flight per lane

// Workgroup b reads its contiguous share of the buffer in 16-byte non-temporal loads, 8 per
// lane in flight, and folds every word into an xor that one lane per wave stores (so no
// load can be dropped). 256 threads.
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ p, int64_t n16, int64_t per_wg,
                                                          uint32_t* __restrict__ out) {
    const int64_t beg = (int64_t)blockIdx.x * per_wg;
    const int64_t end = beg + per_wg < n16 ? beg + per_wg : n16;
    uint32_t acc = 0;
    for (int64_t i = beg + threadIdx.x; i < end; i += 256 * kReadUnroll) {
        u32x4 v[kReadUnroll];
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u) {
            const int64_t j = i + (int64_t)u * 256;
            v[u] = j < end ? load_nt_u32x4(p + j) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o);
    if ((threadIdx.x & 63) == 0) out[blockIdx.x * 4 + (threadIdx.x >> 6)] = acc;
}

// Each wave runs `iters` rounds of 8 independent v_mfma_f32_16x16x32_f16 chains, then stores
// its accumulators' sum per lane. 256 threads: one wave per SIMD per workgroup.
// Constant operands (ops == NULL): every MFMA multiplies the same A and B, made from the lane
// id. Operand sets (ops != NULL): each lane loads 8 A and 8 B fragments (ops[lane][16] of
// f16x8) and the 8 x 8 MFMAs of an unrolled round pair A set (u + c) % 8 with B set c, so
// consecutive MFMAs see different operands: the multipliers toggle as on real data.
template <bool SETS>
__global__ __launch_bounds__(256) void mfma_probe_kernel(int iters, const f16x8* __restrict__ ops,
                                                         float* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    f16x8 a[8], b[8];
    if constexpr (SETS) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            a[i] = ops[lane * 16 + i];
            b[i] = ops[lane * 16 + 8 + i];
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            a[0][e] = (_Float16)((lane + e) & 7) * (_Float16)0.125f;
            b[0][e] = (_Float16)((lane * 3 + e) & 7) * (_Float16)0.0625f;
        }
    }
    f32x4 acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < iters; ++i) {
        if constexpr (SETS) {
#pragma unroll
            for (int u = 0; u < 8; ++u)
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[(u + c) & 7], b[c], acc[c], 0, 0, 0);
        } else {
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0], b[0], acc[c], 0, 0, 0);
        }
    }
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

}  // namespace

extern "C" size_t q4_probe_stream_read_out_bytes(int workgroups) {
    return workgroups > 0 ? (size_t)workgroups * 4 * sizeof(uint32_t) : 0;
}

extern "C" int q4_probe_stream_read(const void* buf, size_t bytes, int workgroups, uint32_t* out, void* stream) {
    if (workgroups < 1 || workgroups > 65536) return Q4MI_E_RANGE;
    if (bytes % 16) return Q4MI_E_SHAPE;
    if (bytes == 0) return Q4MI_OK;
    if (!buf || !out || misaligned16(buf)) return Q4MI_E_ARG;
    const int64_t n16 = (int64_t)(bytes / 16);
    const int64_t per_wg = ceil_div(n16, workgroups);
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)workgroups), dim3(256), 0, (hipStream_t)stream,
                       (const u32x4*)buf, n16, per_wg, out);
    return launch_status();
}

extern "C" int q4_probe_mfma(int workgroups, int iters, const void* operands, float* out, void* stream) {
    if (workgroups < 1 || workgroups > 65536 || iters < 1) return Q4MI_E_RANGE;
    if (!out || misaligned16(operands)) return Q4MI_E_ARG;
    if (operands)
        hipLaunchKernelGGL(mfma_probe_kernel<true>, dim3((unsigned)workgroups), dim3(256), 0, (hipStream_t)stream,
                           iters, (const f16x8*)operands, out);
    else
        hipLaunchKernelGGL(mfma_probe_kernel<false>, dim3((unsigned)workgroups), dim3(256), 0, (hipStream_t)stream,
                           iters, (const f16x8*)nullptr, out);
    return launch_status();
}
