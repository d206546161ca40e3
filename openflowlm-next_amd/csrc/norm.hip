// norm.hip -- the activation producer in front of a GEMV: the residual add and the
// RMSNorm, with the normalised row stored as the next projection's bf16 (or f32) input.
//
//   y  = x + add                         (f32; add optional, y optional, y may be x)
//   r  = 1 / sqrt(mean(y^2) + eps)       (sum of squares and the root in fp64)
//   xn = (y * r) * w                     (f32, then RNE to bf16 when asked)
//
// The reference's ln design (open_kernels/designs/ln/ln.py:1-6: y = x + add,
// xn = bf16(y * rsqrt(mean(y^2) + 1e-6) * w)) and its host twin rms_vec
// (src/open_qwen36/block_host.cpp:42-47: double sum of squares, float r, x * r * w).
// One 256-thread workgroup per row. Rows up to 16384 values are read once into
// registers (the loads issue together; y is stored only after all of x is read, so y
// may be x); longer rows take a two-pass kernel.
#include "norm_core.h"
#include "q4mi_internal.h"

using namespace q4mi;

namespace {

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// PER: values each thread keeps in registers (N <= 256 PER); the row is read once, and
// y is written only after every read of x, so y may be x.
template <int PER>
__global__ __launch_bounds__(256) void rmsnorm_add_kernel(const float* x, const float* __restrict__ add,
                                                          const void* __restrict__ w, int w_bf16, float* y,
                                                          void* __restrict__ xn, int xn_bf16, int64_t N,
                                                          float eps) {
    __shared__ double part[4];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const float* xr = x + row * N;
    const float* ar = add ? add + row * N : nullptr;
    float v[PER], wv[PER];
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {            // x, add and w all issued before the reduction
        const int64_t i = tid + 256 * j;
        v[j] = i < N ? (ar ? xr[i] + ar[i] : xr[i]) : 0.0f;
        wv[j] = i >= N ? 0.0f
                       : (w_bf16 ? bf16_hi_to_f32((uint32_t)((const uint16_t*)w)[i] << 16) : ((const float*)w)[i]);
    }
#pragma unroll
    for (int j = 0; j < PER; ++j) ss += (double)v[j] * (double)v[j];
    // the wave tree adds the lane sums as two f32 halves (hi + lo)
    const double ws = wave_sum_ss(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ws;
    __syncthreads();
    if (y) {
        float* yr = y + row * N;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int64_t i = tid + 256 * j;
            if (i < N) yr[i] = v[j];
        }
    }
    const float r = inv_rms(part, N, eps);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int64_t i = tid + 256 * j;
        if (i >= N) break;
        const float o = v[j] * r * wv[j];
        if (xn_bf16) ((uint16_t*)xn)[row * N + i] = (uint16_t)f32_to_bf16_rne(o);
        else ((float*)xn)[row * N + i] = o;
    }
}

// Rows longer than 256 * 64 values: two passes over memory (y must not be x here).
__global__ __launch_bounds__(256) void rmsnorm_add_long_kernel(const float* __restrict__ x,
                                                               const float* __restrict__ add,
                                                               const void* __restrict__ w, int w_bf16,
                                                               float* __restrict__ y, void* __restrict__ xn,
                                                               int xn_bf16, int64_t N, float eps) {
    __shared__ double part[4];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const float* xr = x + row * N;
    const float* ar = add ? add + row * N : nullptr;
    double ss = 0.0;
    for (int64_t i = tid; i < N; i += 256) {
        const float v = ar ? xr[i] + ar[i] : xr[i];
        ss += (double)v * (double)v;
    }
    ss = wave_sum_f64(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    const double tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float r = (float)(1.0 / sqrt(tot / (double)N + (double)eps));
    for (int64_t i = tid; i < N; i += 256) {
        const float v = ar ? xr[i] + ar[i] : xr[i];
        if (y) y[row * N + i] = v;
        const float wi = w_bf16 ? bf16_hi_to_f32((uint32_t)((const uint16_t*)w)[i] << 16) : ((const float*)w)[i];
        const float o = v * r * wi;
        if (xn_bf16) ((uint16_t*)xn)[row * N + i] = (uint16_t)f32_to_bf16_rne(o);
        else ((float*)xn)[row * N + i] = o;
    }
}

// x = res + the S partial planes of a split GEMV (planes MN floats apart; acc_reduce_kernel's
// sum: S = 1 res + p0, S > 1 res + (((0 + p0) + p1) + ...), S = 0 res), stored to x_out, then
// rmsnorm_add_kernel's normalisation of x into xn: one launch for the reduce and the norm
// in front of a vocabulary-sized norm GEMV. The planes' loads go out four at a time.
template <int PER>
__global__ __launch_bounds__(256) void rmsnorm_planes_kernel(const float* __restrict__ res, const float* __restrict__ part,
                                                             int S, int64_t MN, const void* __restrict__ w, int w_bf16,
                                                             float* __restrict__ x_out, void* __restrict__ xn, int xn_bf16,
                                                             int64_t N, float eps) {
    __shared__ double part_ss[4];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const float* rr = res + row * N;
    const float* pr = part + row * N;
    float v[PER], wv[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int64_t i = tid + 256 * j;
        v[j] = i < N ? rr[i] : 0.0f;
        wv[j] = i >= N ? 0.0f
                       : (w_bf16 ? bf16_hi_to_f32((uint32_t)((const uint16_t*)w)[i] << 16) : ((const float*)w)[i]);
    }
    if (S == 1) {
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int64_t i = tid + 256 * j;
            if (i < N) v[j] = v[j] + pr[i];
        }
    } else if (S > 1) {
        float sum[PER];
#pragma unroll
        for (int j = 0; j < PER; ++j) sum[j] = 0.0f;
        for (int q = 0; q < S; q += 4) {
            float t[4][PER];
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int j = 0; j < PER; ++j) {
                    const int64_t i = tid + 256 * j;
                    t[u][j] = q + u < S && i < N ? pr[(int64_t)(q + u) * MN + i] : 0.0f;
                }
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (q + u < S) {
#pragma unroll
                    for (int j = 0; j < PER; ++j) sum[j] += t[u][j];
                }
        }
#pragma unroll
        for (int j = 0; j < PER; ++j) v[j] = v[j] + sum[j];
    }
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int64_t i = tid + 256 * j;
        if (i >= N) v[j] = 0.0f;
        ss += (double)v[j] * (double)v[j];
    }
    const double wsum = wave_sum_ss(ss);
    if ((tid & 63) == 0) part_ss[tid >> 6] = wsum;
    __syncthreads();
    float* xo = x_out + row * N;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int64_t i = tid + 256 * j;
        if (i < N) xo[i] = v[j];
    }
    const float r = inv_rms(part_ss, N, eps);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int64_t i = tid + 256 * j;
        if (i >= N) break;
        const float o = v[j] * r * wv[j];
        if (xn_bf16) ((uint16_t*)xn)[row * N + i] = (uint16_t)f32_to_bf16_rne(o);
        else ((float*)xn)[row * N + i] = o;
    }
}

}  // namespace

extern "C" int q4_rmsnorm_add(const float* x, const float* add, const void* w, int w_dtype, float* y, void* xn,
                              int xn_dtype, int M, int64_t N, float eps, void* stream) {
    if ((w_dtype != Q4MI_F32 && w_dtype != Q4MI_BF16) || (xn_dtype != Q4MI_F32 && xn_dtype != Q4MI_BF16))
        return Q4MI_E_ARG;
    if (M < 0 || M > 65535) return Q4MI_E_RANGE;
    if (N <= 0) return Q4MI_E_SHAPE;
    if (M == 0) return Q4MI_OK;
    if (!x || !w || !xn) return Q4MI_E_ARG;
    if (!(eps >= 0.0f)) return Q4MI_E_ARG;
    const hipStream_t st = (hipStream_t)stream;
    const int wb = w_dtype == Q4MI_BF16, xb = xn_dtype == Q4MI_BF16;
    const dim3 grid((unsigned)M), block(256);
    if (N <= 256 * 8)
        hipLaunchKernelGGL(rmsnorm_add_kernel<8>, grid, block, 0, st, x, add, w, wb, y, xn, xb, N, eps);
    else if (N <= 256 * 16)
        hipLaunchKernelGGL(rmsnorm_add_kernel<16>, grid, block, 0, st, x, add, w, wb, y, xn, xb, N, eps);
    else if (N <= 256 * 32)
        hipLaunchKernelGGL(rmsnorm_add_kernel<32>, grid, block, 0, st, x, add, w, wb, y, xn, xb, N, eps);
    else if (N <= 256 * 64)
        hipLaunchKernelGGL(rmsnorm_add_kernel<64>, grid, block, 0, st, x, add, w, wb, y, xn, xb, N, eps);
    else if (y == x)
        return Q4MI_E_ARG;          // rows this long are read twice: y must not overwrite x
    else
        hipLaunchKernelGGL(rmsnorm_add_long_kernel, grid, block, 0, st, x, add, w, wb, y, xn, xb, N, eps);
    return launch_status();
}

namespace q4mi {

int rmsnorm_planes(const float* res, const float* part, int S, const void* w, int w_dtype, float* x_out, void* xn,
                   int M, int64_t N, float eps, void* stream) {
    if (M <= 0 || N <= 0 || N > 256 * 16 || S < 0) return Q4MI_E_RANGE;
    const hipStream_t st = (hipStream_t)stream;
    const int wb = w_dtype == Q4MI_BF16;
    const int64_t MN = (int64_t)M * N;
    if (N <= 256 * 8)
        hipLaunchKernelGGL(rmsnorm_planes_kernel<8>, dim3((unsigned)M), dim3(256), 0, st, res, part, S, MN, w, wb,
                           x_out, xn, 1, N, eps);
    else
        hipLaunchKernelGGL(rmsnorm_planes_kernel<16>, dim3((unsigned)M), dim3(256), 0, st, res, part, S, MN, w, wb,
                           x_out, xn, 1, N, eps);
    return launch_status();
}

}  // namespace q4mi
