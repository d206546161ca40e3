// norm_core.h -- the RMSNorm arithmetic shared by the norm kernels (norm.hip) and the GEMVs
// that normalise their activation row themselves (gemv.hip), so both give the same bits.
//
//   r  = 1 / sqrt(mean(v^2) + eps): the lane sums of v^2 in fp64 over i = lane + 256 j
//        (j ascending), each wave's sum as two f32 halves through a DPP tree, the four
//        waves' sums added as (w0 + w1) + (w2 + w3), the root in fp64, rounded to f32;
//   xn = (v * r) * w, rounded to bf16 (RNE) when the consumer takes bf16.
// (The reference's ln design, designs/ln/ln.py:1-6, and its host twin rms_vec,
// src/open_qwen36/block_host.cpp:42-47: double sum of squares, float r, x * r * w.)
#pragma once

#include "q4mi_device.h"

namespace q4mi {

// Wave sum of an f32 in every lane: DPP steps within rows (xor 1, xor 2 quad permutes,
// the half-row and row mirrors), row broadcasts into lane 63, then readlane. Every lane's
// addends arrive in the same tree order, so the result is deterministic.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                                    0xF, false));
}
__device__ __forceinline__ float wave_sum_f32(float v) {
    v = dpp_add<0xB1, 0xF>(v);        // quad_perm [1,0,3,2]
    v = dpp_add<0x4E, 0xF>(v);        // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xF>(v);       // row_half_mirror
    v = dpp_add<0x140, 0xF>(v);       // row_mirror
    v = dpp_add<0x142, 0xA>(v);       // row_bcast:15 -> rows 1, 3
    v = dpp_add<0x143, 0xC>(v);       // row_bcast:31 -> rows 2, 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// A wave's sum of its lanes' fp64 partial sums of squares (exact lane sums as hi + lo f32).
__device__ __forceinline__ double wave_sum_ss(double ss) {
    const float hi = (float)ss, lo = (float)(ss - (double)hi);
    return (double)wave_sum_f32(hi) + (double)wave_sum_f32(lo);
}

// r from the four waves' sums.
__device__ __forceinline__ float inv_rms(const double (&part)[4], int64_t N, float eps) {
    const double tot = (part[0] + part[1]) + (part[2] + part[3]);
    return (float)(1.0 / sqrt(tot / (double)N + (double)eps));
}

// r of rows 0..M-1 of x [M][N] (N <= 16384) into r_out[m], by the workgroup's first 256
// threads (every thread calls it: barriers inside; M <= MAXM).
template <int MAXM>
__device__ __forceinline__ void rms_inv_rows(const float* __restrict__ x, int M, int64_t N, float eps,
                                             float* r_out) {
    __shared__ double part[MAXM][4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (wave < 4) {
        for (int m = 0; m < M; ++m) {
            const float* xr = x + (int64_t)m * N;
            double ss = 0.0;
#pragma unroll 16
            for (int64_t i = tid; i < N; i += 256) {
                const float v = xr[i];
                ss += (double)v * (double)v;
            }
            const double ws = wave_sum_ss(ss);
            if (lane == 0) part[m][wave] = ws;
        }
    }
    __syncthreads();
    if (tid < M) r_out[tid] = inv_rms(part[tid], N, eps);
    __syncthreads();
}

// The normalised bf16 of 8 consecutive activations a[0..3], b[0..3] with weights wv:
// ((x * r) * w) rounded to bf16.
__device__ __forceinline__ bf16x8 norm_bf16x8_of(f32x4 a, f32x4 b, const float (&wv)[8], float r) {
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float v0 = e < 2 ? a[2 * e] : b[2 * e - 4], v1 = e < 2 ? a[2 * e + 1] : b[2 * e - 3];
        o[e] = f32_to_bf16_rne(v0 * r * wv[2 * e]) | (f32_to_bf16_rne(v1 * r * wv[2 * e + 1]) << 16);
    }
    return __builtin_bit_cast(bf16x8, o);
}

// 8 bf16 norm weights (one 16-byte word) as f32.
__device__ __forceinline__ void norm_w_of_bf16(u32x4 ww, float (&wv)[8]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) wv[2 * e] = bf16_lo_to_f32(ww[e]), wv[2 * e + 1] = bf16_hi_to_f32(ww[e]);
}

// The normalised bf16 of 8 consecutive activations: ((x * r) * w) rounded to bf16.
__device__ __forceinline__ bf16x8 norm_bf16x8(const float* __restrict__ x, const void* __restrict__ w, int w_bf16,
                                              float r) {
    const f32x4 a = load_global<f32x4>(x), b = load_global<f32x4>(x + 4);
    float wv[8];
    if (w_bf16) {
        norm_w_of_bf16(load_global<u32x4>(w), wv);
    } else {
        const f32x4 c = load_global<f32x4>(w), d = load_global<f32x4>((const float*)w + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) wv[e] = c[e], wv[e + 4] = d[e];
    }
    return norm_bf16x8_of(a, b, wv, r);
}

}  // namespace q4mi
