// moe.hip -- routed MoE expert block for decode tokens on the mx layout:
//   out[t] = sum_j w[t][j] * down_e( silu(gate_e . x_t) * (up_e . x_t) ),  e = ids[t][j]
//
// The reference runs each expert "slot" of NT gathered tokens through
// h = bf16(silu(gate x) * (up x)), y = down h on the NPU (moe_batch.h:98-202)
// after the host gathers tokens per expert and before it scatters y with the
// router weights (Core::moe_block, core.cpp:5150-5245). Here the gather and
// the scatter run on the device, in three launches:
//   1. gate/up: workgroup (expert e, 64-row group of F). It finds the (token,
//      slot) pairs routed to e by a ballot compaction of ids (pair order, so
//      the result is deterministic), streams e's 64 gate rows and the 64 up
//      rows next to them once for all those tokens (gemv_core.h, activations
//      gathered by row index), and writes h = silu(g) * u in fp32 per pair.
//      Workgroups of experts no token picked leave after the scan.
//   2. down: workgroup (expert e, 64-row group of H): y_pair = down_e h_pair,
//      h read as fp32 (split into two bf16 halves for the MFMA).
//   3. combine: out[t] = sum_j w[t][j] y_pair[t][j] in slot order j.
// h stays fp32 (the fp64 replica's semantics, model/replica.py:131-140); the
// reference kernel's bf16 rounding of h would cost ~2^-9 relative.
#include "gemv_core.h"
#include "q4mi_internal.h"

using namespace q4mi;

namespace {

constexpr int kMaxPairs = 4096;     // T * topk per call

// The pairs p = t * topk + j with ids[p] == e, ascending, into `list`; returns
// their count (all 256 threads call it; barriers inside).
__device__ int collect_pairs(const int32_t* __restrict__ ids, int P, int e, int* list) {
    __shared__ int wave_cnt[4];
    __shared__ int base;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) base = 0;
    __syncthreads();
    for (int p0 = 0; p0 < P; p0 += 256) {
        const int p = p0 + tid;
        const bool hit = p < P && ids[p] == e;
        const uint64_t mask = __ballot(hit);
        const int within = __popcll(mask & ((1ull << lane) - 1ull));
        if (lane == 0) wave_cnt[wave] = __popcll(mask);
        __syncthreads();
        int off = base;
        for (int w = 0; w < wave; ++w) off += wave_cnt[w];
        if (hit) list[off + within] = p;
        __syncthreads();
        if (tid == 0) base += wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
        __syncthreads();
    }
    return base;
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

template <int NTL, bool XF32>
__device__ __forceinline__ void up_chunk(const uint8_t* wexp, const void* x, int H, int F, int rgp, const int* rows,
                                         const int* pairs, int M, float (*red)[4][4][64], float* __restrict__ hbuf) {
    // the gate rows (row group 2 rgp) and the up rows next to them (2 rgp + 1) in one stream
    float acc[2][4][NTL];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < NTL; ++j) acc[i][r][j] = 0.f;
    const int KB = H >> 5;
    const uint8_t* const gb[2] = {wexp + (int64_t)(2 * rgp) * KB * kTileBytes,
                                  wexp + (int64_t)(2 * rgp + 1) * KB * kTileBytes};
    gemv_rows_multi<NTL, XF32, 2, 4>(gb, x, GatherRows{rows, M}, H, 0, KB, acc);
    float (*rd)[4][NTL][64] = (float (*)[4][NTL][64])red;
    float vg[NTL], vu[NTL];
    wave_sum<NTL>(acc[0], rd, vg);
    __syncthreads();
    wave_sum<NTL>(acc[1], rd, vu);
    const int tid = threadIdx.x, lane = tid & 63, r = tid >> 6, i16 = lane & 15, kg = lane >> 4;
    const int64_t f = (int64_t)rgp * 64 + r * 16 + i16;
#pragma unroll
    for (int j = 0; j < NTL; ++j) {
        const int tok = token_of(kg, j);
        if (tok < M) hbuf[(int64_t)pairs[tok] * F + f] = silu(vg[j]) * vu[j];
    }
}

// MAXNTL: accumulators per row (chunks of 4 * MAXNTL routed tokens). The register
// allocation follows the largest instance a kernel holds: MAXNTL = 1 needs 132 VGPRs for
// gate/up and 156 for down (3 waves per SIMD), MAXNTL = 4 188 and 224 (2 waves). An expert
// with more than 4 * MAXNTL tokens streams its rows once per chunk.
template <bool XF32, int MAXNTL>
__global__ __launch_bounds__(256) void moe_up_kernel(const uint8_t* __restrict__ gate_up, const void* __restrict__ x,
                                                     const int32_t* __restrict__ ids, int P, int topk, int H, int F,
                                                     float* __restrict__ hbuf) {
    __shared__ int list[kMaxPairs];
    __shared__ int rows[16];
    __shared__ float red[4][4][4][64];
    const int fg = F >> 6;
    const int e = blockIdx.x / fg, rgp = blockIdx.x % fg;
    const int cnt = collect_pairs(ids, P, e, list);
    if (cnt == 0) return;
    const uint8_t* wexp = gate_up + (int64_t)e * (2 * F / 64) * (H / 32) * kTileBytes;
    for (int c0 = 0; c0 < cnt; c0 += 4 * MAXNTL) {
        const int M = min(4 * MAXNTL, cnt - c0);
        if (threadIdx.x < 16) rows[threadIdx.x] = list[c0 + min((int)threadIdx.x, M - 1)] / topk;
        __syncthreads();
        if constexpr (MAXNTL == 1) {
            up_chunk<1, XF32>(wexp, x, H, F, rgp, rows, list + c0, M, red, hbuf);
        } else {
            switch ((M + 3) / 4) {
                case 1: up_chunk<1, XF32>(wexp, x, H, F, rgp, rows, list + c0, M, red, hbuf); break;
                case 2: up_chunk<2, XF32>(wexp, x, H, F, rgp, rows, list + c0, M, red, hbuf); break;
                case 3: up_chunk<3, XF32>(wexp, x, H, F, rgp, rows, list + c0, M, red, hbuf); break;
                default: up_chunk<4, XF32>(wexp, x, H, F, rgp, rows, list + c0, M, red, hbuf); break;
            }
        }
        __syncthreads();
    }
}

// NG 64-row groups of H per down workgroup (4 when H % 256 == 0, else 1): K = F is short,
// so one group alone is latency-bound.
template <int NTL, int NG>
__device__ __forceinline__ void down_chunk(const uint8_t* wexp, const float* hbuf, int H, int F, int rg0,
                                           const int* pairs, int M, float (*red)[4][4][64], float* __restrict__ ypair) {
    float acc[NG][4][NTL];
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < NTL; ++j) acc[i][r][j] = 0.f;
    const int KB = F >> 5;
    const uint8_t* gb[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) gb[i] = wexp + (int64_t)(rg0 + i) * KB * kTileBytes;
    gemv_rows_multi<NTL, true, NG, NG == 1 ? 4 : 2>(gb, hbuf, GatherRows{pairs, M}, F, 0, KB, acc);
    float (*rd)[4][NTL][64] = (float (*)[4][NTL][64])red;
    const int tid = threadIdx.x, lane = tid & 63, r = tid >> 6, i16 = lane & 15, kg = lane >> 4;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        float v[NTL];
        if (i) __syncthreads();
        wave_sum<NTL>(acc[i], rd, v);
        const int64_t n = (int64_t)(rg0 + i) * 64 + r * 16 + i16;
#pragma unroll
        for (int j = 0; j < NTL; ++j) {
            const int tok = token_of(kg, j);
            if (tok < M) ypair[(int64_t)pairs[tok] * H + n] = v[j];
        }
    }
}

template <int NG, int MAXNTL>
__global__ __launch_bounds__(256) void moe_down_kernel(const uint8_t* __restrict__ down,
                                                       const float* __restrict__ hbuf,
                                                       const int32_t* __restrict__ ids, int P, int H, int F,
                                                       float* __restrict__ ypair) {
    __shared__ int list[kMaxPairs];
    __shared__ float red[4][4][4][64];
    const int hg = H >> 6, wg_per_e = hg / NG;
    const int e = blockIdx.x / wg_per_e, rg0 = (blockIdx.x % wg_per_e) * NG;
    const int cnt = collect_pairs(ids, P, e, list);
    if (cnt == 0) return;
    const uint8_t* wexp = down + (int64_t)e * (H / 64) * (F / 32) * kTileBytes;
    for (int c0 = 0; c0 < cnt; c0 += 4 * MAXNTL) {
        const int M = min(4 * MAXNTL, cnt - c0);
        if constexpr (MAXNTL == 1) {
            down_chunk<1, NG>(wexp, hbuf, H, F, rg0, list + c0, M, red, ypair);
        } else {
            switch ((M + 3) / 4) {
                case 1: down_chunk<1, NG>(wexp, hbuf, H, F, rg0, list + c0, M, red, ypair); break;
                case 2: down_chunk<2, NG>(wexp, hbuf, H, F, rg0, list + c0, M, red, ypair); break;
                case 3: down_chunk<3, NG>(wexp, hbuf, H, F, rg0, list + c0, M, red, ypair); break;
                default: down_chunk<4, NG>(wexp, hbuf, H, F, rg0, list + c0, M, red, ypair); break;
            }
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ ypair,
                                                          const int32_t* __restrict__ ids,
                                                          const float* __restrict__ w, int T, int topk, int E, int H,
                                                          float* __restrict__ out) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)T * H) return;
    const int64_t t = idx / H, n = idx % H;
    float s = 0.f;
    for (int j = 0; j < topk; ++j) {
        const int64_t p = t * topk + j;
        const int e = ids[p];
        if (e >= 0 && e < E) s += w[p] * ypair[p * H + n];
    }
    out[idx] = s;
}

// The block output with the residual and the gated shared expert folded into the combine,
// one workgroup per token (moe_fin, designs/moe_combine/moe_fin.py:1-4 and
// designs/moe_experts/moe_fin.cc: out = xres + sum_j w y + sigmoid(xm . sgw) * shared):
//   g = sigmoid(x[t] . sgw) (sgw bf16 [H], the dot product in fp32, fixed reduction order),
//   out[t][n] = (res[t][n] + sum_j w[t][j] y_pair[t][j][n]) + g shared[t][n].
// res may be null (no residual) and may alias out; shared null leaves the gate out.
template <bool XF32>
__global__ __launch_bounds__(256) void moe_fin_kernel(const float* __restrict__ ypair, const int32_t* __restrict__ ids,
                                                      const float* __restrict__ w, int topk, int E, int H,
                                                      const void* __restrict__ x, const uint16_t* __restrict__ sgw,
                                                      const float* __restrict__ shared, const float* res, float* out) {
    __shared__ float red[4];
    const int64_t t = blockIdx.x;
    float g = 0.f;
    if (shared) {
        float dot = 0.f;
        for (int h = threadIdx.x; h < H; h += 256) {
            const float xv = XF32 ? ((const float*)x)[t * H + h]
                                  : bf16_hi_to_f32((uint32_t)((const uint16_t*)x)[t * H + h] << 16);
            dot = __builtin_fmaf(xv, bf16_hi_to_f32((uint32_t)sgw[h] << 16), dot);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) dot += __shfl_xor(dot, o);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = dot;
        __syncthreads();
        dot = (red[0] + red[1]) + (red[2] + red[3]);
        g = 1.0f / (1.0f + expf(-dot));
    }
    for (int n = threadIdx.x; n < H; n += 256) {
        float s = 0.f;
        for (int j = 0; j < topk; ++j) {
            const int64_t p = t * topk + j;
            const int e = ids[p];
            if (e >= 0 && e < E) s += w[p] * ypair[p * H + n];
        }
        float v = res ? res[t * H + n] + s : s;
        if (shared) v = __builtin_fmaf(g, shared[t * H + n], v);
        out[t * H + n] = v;
    }
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

}  // namespace

extern "C" size_t q4_moe_workspace_bytes(int T, int E, int topk, int H, int F) {
    (void)E;
    if (T <= 0 || topk <= 0 || H <= 0 || F <= 0) return 0;
    const size_t P = (size_t)T * topk;
    return align256(P * F * 4) + align256(P * H * 4);
}

// The expert kernels, then the plain combine (fin == false) or the finish with residual and
// gated shared expert (fin == true).
static int moe_impl(const uint8_t* gate_up, const uint8_t* down, const void* x, int x_dtype, const int32_t* topk_ids,
                    const float* topk_w, float* out, int T, int E, int topk, int64_t H, int64_t F, void* workspace,
                    size_t workspace_bytes, void* stream, bool fin, const float* residual, const float* shared,
                    const uint16_t* shared_gate_w) {
    if (x_dtype != Q4MI_F32 && x_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (fin && (!shared) != (!shared_gate_w)) return Q4MI_E_ARG;
    if (H <= 0 || F <= 0 || H % 64 || F % 64) return Q4MI_E_SHAPE;
    if (H > (1 << 24) || F > (1 << 24)) return Q4MI_E_RANGE;
    if (T < 0 || E <= 0 || topk <= 0 || topk > 16 || (int64_t)T * topk > kMaxPairs) return Q4MI_E_RANGE;
    if (T == 0) return Q4MI_OK;
    if (!gate_up || !down || !x || !topk_ids || !topk_w || !out) return Q4MI_E_ARG;
    if (misaligned16(gate_up) || misaligned16(down) || misaligned16(x) || misaligned16(out) || misaligned16(workspace))
        return Q4MI_E_ARG;
    const size_t need = q4_moe_workspace_bytes(T, E, topk, (int)H, (int)F);
    if (!workspace || workspace_bytes < need) return Q4MI_E_WORKSPACE;
    const int P = T * topk;
    float* hbuf = (float*)workspace;
    float* ypair = (float*)((char*)workspace + align256((size_t)P * F * 4));
    const hipStream_t st = (hipStream_t)stream;
    const int ng = H % 256 == 0 ? 4 : 1;
    const dim3 gu((unsigned)(E * (F / 64))), dn((unsigned)(E * (H / (64 * ng))));
    // At most 2 routed pairs per expert on average (decode batches): the one-accumulator
    // instances, whose lower register use runs 3 waves per SIMD (config 4, 16 tokens x top-8
    // of 128 experts: 66.7 -> 63.7 us, bit-identical). Larger batches stream each expert's
    // rows once per 16 tokens instead of once per 4.
    const bool few = P <= 2 * E;
    if (x_dtype == Q4MI_F32) {
        if (few)
            hipLaunchKernelGGL((moe_up_kernel<true, 1>), gu, dim3(256), 0, st, gate_up, x, topk_ids, P, topk, (int)H,
                               (int)F, hbuf);
        else
            hipLaunchKernelGGL((moe_up_kernel<true, 4>), gu, dim3(256), 0, st, gate_up, x, topk_ids, P, topk, (int)H,
                               (int)F, hbuf);
    } else {
        if (few)
            hipLaunchKernelGGL((moe_up_kernel<false, 1>), gu, dim3(256), 0, st, gate_up, x, topk_ids, P, topk,
                               (int)H, (int)F, hbuf);
        else
            hipLaunchKernelGGL((moe_up_kernel<false, 4>), gu, dim3(256), 0, st, gate_up, x, topk_ids, P, topk,
                               (int)H, (int)F, hbuf);
    }
    if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
    if (ng == 4) {
        if (few)
            hipLaunchKernelGGL((moe_down_kernel<4, 1>), dn, dim3(256), 0, st, down, hbuf, topk_ids, P, (int)H, (int)F,
                               ypair);
        else
            hipLaunchKernelGGL((moe_down_kernel<4, 4>), dn, dim3(256), 0, st, down, hbuf, topk_ids, P, (int)H, (int)F,
                               ypair);
    } else {
        if (few)
            hipLaunchKernelGGL((moe_down_kernel<1, 1>), dn, dim3(256), 0, st, down, hbuf, topk_ids, P, (int)H, (int)F,
                               ypair);
        else
            hipLaunchKernelGGL((moe_down_kernel<1, 4>), dn, dim3(256), 0, st, down, hbuf, topk_ids, P, (int)H, (int)F,
                               ypair);
    }
    if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
    if (fin) {
        if (x_dtype == Q4MI_F32)
            hipLaunchKernelGGL(moe_fin_kernel<true>, dim3((unsigned)T), dim3(256), 0, st, ypair, topk_ids, topk_w, topk,
                               E, (int)H, x, shared_gate_w, shared, residual, out);
        else
            hipLaunchKernelGGL(moe_fin_kernel<false>, dim3((unsigned)T), dim3(256), 0, st, ypair, topk_ids, topk_w,
                               topk, E, (int)H, x, shared_gate_w, shared, residual, out);
        return launch_status();
    }
    const int64_t tot = (int64_t)T * H;
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)ceil_div(tot, 256)), dim3(256), 0, st, ypair, topk_ids,
                       topk_w, T, topk, E, (int)H, out);
    return launch_status();
}

extern "C" int q4_moe_gemv(const uint8_t* gate_up, const uint8_t* down, const void* x, int x_dtype,
                           const int32_t* topk_ids, const float* topk_w, float* out, int T, int E, int topk,
                           int64_t H, int64_t F, void* workspace, size_t workspace_bytes, void* stream) {
    return moe_impl(gate_up, down, x, x_dtype, topk_ids, topk_w, out, T, E, topk, H, F, workspace, workspace_bytes,
                    stream, false, nullptr, nullptr, nullptr);
}

extern "C" int q4_moe_gemv_fin(const uint8_t* gate_up, const uint8_t* down, const void* x, int x_dtype,
                               const int32_t* topk_ids, const float* topk_w, const float* residual,
                               const float* shared, const uint16_t* shared_gate_w, float* out, int T, int E, int topk,
                               int64_t H, int64_t F, void* workspace, size_t workspace_bytes, void* stream) {
    if ((residual && misaligned16(residual)) || (shared && misaligned16(shared))) return Q4MI_E_ARG;
    return moe_impl(gate_up, down, x, x_dtype, topk_ids, topk_w, out, T, E, topk, H, F, workspace, workspace_bytes,
                    stream, true, residual, shared, shared_gate_w);
}
