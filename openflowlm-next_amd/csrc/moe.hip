// moe.hip -- routed MoE expert block for decode tokens on the mx layout:
//   out[t] = sum_j w[t][j] * down_e( silu(gate_e . x_t) * (up_e . x_t) ),  e = ids[t][j]
//
// The reference runs each expert "slot" of NT gathered tokens through
// h = bf16(silu(gate x) * (up x)), y = down h on the NPU (moe_batch.h:98-202)
// after the host gathers tokens per expert and before it scatters y with the
// router weights (Core::moe_block, core.cpp:5150-5245). Here the gather and
// the scatter run on the device, in three launches:
//   1. gate/up: workgroup (a, 64-row group of F), for the a-th routed expert e in
//      ascending order (found from an LDS bitmap of ids, so the workgroups of the
//      routed experts lead the grid and the rest leave at once). It finds the
//      (token, slot) pairs routed to e by a ballot compaction of ids (pair order,
//      so the result is deterministic), streams e's 64 gate rows and the 64 up
//      rows next to them once for all those tokens (gemv_core.h, activations
//      gathered by row index), and writes h = silu(g) * u in fp32 per pair.
//   2. down: workgroup (a, 64-row groups of H): y_pair = down_e h_pair, h read
//      as fp32 (split into two bf16 halves for the MFMA).
//   3. combine: out[t] = sum_j w[t][j] y_pair[t][j] in slot order j.
// h stays fp32 (the fp64 replica's semantics, model/replica.py:131-140); the
// reference kernel's bf16 rounding of h would cost ~2^-9 relative.
#include "gemv_core.h"
#include "q4mi_internal.h"

using namespace q4mi;

namespace {

constexpr int kMaxPairs = 4096;     // T * topk per call
constexpr int kMaxExperts = 8192;   // one bit each in LDS, one 32-expert word per thread

// Waves per workgroup, K positions in flight per wave and 64-row groups of H per down
// workgroup. Measured at config 4 (128 experts, top-8 of 16 tokens, H 2048, F 768, bf16 x;
// 84 routed experts, graph replays over 4 expert pools), per call: 4 waves, 2 positions (up),
// 4 waves, 2 positions, 4 groups (down) 56.9 us; 4 positions in up 58.5 us; 3 in down
// 59.6 us; 8 waves per workgroup 73 us; 2 row-group pairs per up workgroup 65 us; 2 or 1
// groups per down workgroup 64 / 71 us.
constexpr int kUpWaves = 4, kUpUnr = 2;
constexpr int kDnWaves = 4, kDnUnr = 2, kDnGroups = 4;

// The a-th expert, in ascending order, that at least one pair is routed to; -1 when fewer
// than a + 1 are. Every thread of the workgroup calls it (barriers inside) and gets the
// same answer: the routed experts are marked in an LDS bitmap, each thread counts one
// 32-expert word, and a block-wide prefix sum of the counts finds the word and bit. The
// expert kernels map their workgroups onto this list, so the workgroups of routed experts
// come first in the grid and the rest leave at once. The ids are also left in sids (LDS, P
// entries) for collect_pairs, so the routing reads them from memory once.
template <int WAVES>
__device__ int active_expert(const int32_t* __restrict__ ids, int P, int E, int a, int* sids) {
    __shared__ uint32_t bits[kMaxExperts / 32];
    __shared__ int wsum[WAVES];
    __shared__ int found;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = (E + 31) >> 5;
    for (int i = tid; i < nw; i += 64 * WAVES) bits[i] = 0u;
    if (tid == 0) found = -1;
    __syncthreads();
    // up to one id per thread (decode batches): one pass; more (4096 pairs at T = 512 take 16
    // per thread): kR ids per thread issued together, not one trip to memory per id
    constexpr int kR = 8;
    if (P <= 64 * WAVES) {
        if (tid < P) {
            const int e = ids[tid];
            sids[tid] = e;
            if (e >= 0 && e < E) atomicOr(&bits[e >> 5], 1u << (e & 31));
        }
    } else {
        for (int p0 = 0; p0 < P; p0 += 64 * WAVES * kR) {
            int ev[kR];
#pragma unroll
            for (int j = 0; j < kR; ++j) {
                const int p = p0 + tid + 64 * WAVES * j;
                ev[j] = p < P ? ids[p] : -1;
            }
#pragma unroll
            for (int j = 0; j < kR; ++j) {
                const int p = p0 + tid + 64 * WAVES * j;
                if (p < P) sids[p] = ev[j];
                if (ev[j] >= 0 && ev[j] < E) atomicOr(&bits[ev[j] >> 5], 1u << (ev[j] & 31));
            }
        }
    }
    __syncthreads();
    const uint32_t w = tid < nw ? bits[tid] : 0u;
    const int c = __popc(w);
    int incl = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o);
        if (lane >= o) incl += v;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int excl = incl - c;
    for (int i = 0; i < wave; ++i) excl += wsum[i];
    if (a >= excl && a < excl + c) {
        uint32_t m = w;
        for (int i = excl; i < a; ++i) m &= m - 1u;     // drop the lower set bits
        found = tid * 32 + __builtin_ctz(m);
    }
    __syncthreads();
    return found;
}

// collect_pairs for P > 64 WAVES: thread t takes the kMaxPairs / (64 WAVES) consecutive
// pairs from t times that on (read as 16-byte vectors), so a block-wide prefix sum of the
// threads' counts orders the matches, in one pass for any P <= kMaxPairs.
template <int WAVES>
__device__ int collect_pairs_runs(const int* sids, int P, int e, int* list) {
    constexpr int kPer = kMaxPairs / (64 * WAVES);
    static_assert(kPer % 4 == 0, "whole 16-byte groups per thread");
    __shared__ int wave_cnt[WAVES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, i0 = tid * kPer;
    int v[kPer];
#pragma unroll
    for (int q = 0; q < kPer / 4; ++q) {
        if (i0 + 4 * q < P) {               // entries from P on (inside the array) are masked below
            const int4 g = *(const int4*)(sids + i0 + 4 * q);
            v[4 * q] = g.x, v[4 * q + 1] = g.y, v[4 * q + 2] = g.z, v[4 * q + 3] = g.w;
        } else {
            v[4 * q] = v[4 * q + 1] = v[4 * q + 2] = v[4 * q + 3] = -1;
        }
    }
    int c = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) c += i0 + j < P && v[j] == e;
    int incl = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o);
        if (lane >= o) incl += t;
    }
    if (lane == 63) wave_cnt[wave] = incl;
    __syncthreads();
    int r = incl - c, total = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
        if (w < wave) r += wave_cnt[w];
        total += wave_cnt[w];
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j)
        if (i0 + j < P && v[j] == e) list[r++] = i0 + j;
    __syncthreads();                        // list complete; wave_cnt free for the next call
    return total;
}

// The pairs p = t * topk + j with ids[p] == e, ascending, into `list`; returns their count
// (every thread calls it; barriers inside). sids: the ids as active_expert left them in LDS.
// Up to one pair per thread (decode batches): a ballot compaction; more: collect_pairs_runs.
template <int WAVES>
__device__ int collect_pairs(const int* sids, int P, int e, int* list) {
    if (P > 64 * WAVES) return collect_pairs_runs<WAVES>(sids, P, e, list);
    __shared__ int wave_cnt[WAVES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool hit = tid < P && sids[tid] == e;
    const uint64_t mask = __ballot(hit);
    const int within = __popcll(mask & ((1ull << lane) - 1ull));
    if (lane == 0) wave_cnt[wave] = __popcll(mask);
    __syncthreads();
    int off = 0, total = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
        if (w < wave) off += wave_cnt[w];
        total += wave_cnt[w];
    }
    if (hit) list[off + within] = tid;
    __syncthreads();                        // list complete; wave_cnt free for the next call
    return total;
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

template <int NTL, bool XF32, int WAVES, int UNR>
__device__ __forceinline__ void up_chunk(const uint8_t* wexp, const void* x, int H, int F, int rgp, const int* rows,
                                         const int* pairs, int M, float* red, float* __restrict__ hbuf) {
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
    gemv_rows_pipe<NTL, XF32, 2, UNR, WAVES>(gb, x, GatherRows{rows, M}, H, 0, KB, acc);
    float (*rd)[4][NTL][64] = (float (*)[4][NTL][64])red;
    float vg[NTL], vu[NTL];
    wave_sum<NTL, WAVES>(acc[0], rd, vg);
    __syncthreads();
    wave_sum<NTL, WAVES>(acc[1], rd, vu);
    const int tid = threadIdx.x, lane = tid & 63, r = tid >> 6, i16 = lane & 15, kg = lane >> 4;
    if (r >= 4) return;
    const int64_t f = (int64_t)rgp * 64 + r * 16 + i16;
#pragma unroll
    for (int j = 0; j < NTL; ++j) {
        const int tok = token_of(kg, j);
        if (tok < M) hbuf[(int64_t)pairs[tok] * F + f] = silu(vg[j]) * vu[j];
    }
}

// The shared expert of a block (q4_moe_gemv_shared): a dense expert every token goes
// through, its gate/up [2 Fs, H] interleaved as the routed experts' and its down [H, Fs].
// Its workgroups lead the expert kernels' grids: workgroup (chunk c, row group) covers the
// tokens [4 MAXNTL c, 4 MAXNTL (c + 1)), its h goes to hs [T][Fs] and its y to ys [T][H].
struct SharedExpert {
    const uint8_t* w = nullptr;   // gate/up (up kernel) or down (down kernel); null: none
    float* out = nullptr;         // hs (up kernel) or ys (down kernel)
    const float* h = nullptr;     // hs (down kernel)
    int Fs = 0, T = 0, wgs = 0;   // wgs: the leading workgroups that take it
};

// Workgroup (a, rgp): the a-th routed expert's gate/up row-group pair rgp, for all the
// pairs routed to it. MAXNTL: accumulators per row (chunks of 4 * MAXNTL routed tokens);
// the register allocation follows the largest instance a kernel holds, so batches of at
// most 2 pairs per expert on average take the one-accumulator instance. An expert with
// more than 4 * MAXNTL pairs streams its rows once per chunk. The shared expert's
// workgroups (sh.wgs of them) come first.
template <bool XF32, int MAXNTL>
__global__ __launch_bounds__(64 * kUpWaves) void moe_up_kernel(const uint8_t* __restrict__ gate_up,
                                                               const void* __restrict__ x,
                                                               const int32_t* __restrict__ ids, int P, int E,
                                                               int topk, int H, int F, float* __restrict__ hbuf,
                                                               SharedExpert sh) {
    __shared__ int list[kMaxPairs];
    __shared__ int rows[16];
    __shared__ float red[kUpWaves * 4 * MAXNTL * 64];
    if ((int)blockIdx.x < sh.wgs) {   // the shared expert: every token, chunk by chunk
        const int fgs = sh.Fs >> 6, rgp = blockIdx.x % fgs, c0 = (blockIdx.x / fgs) * 4 * MAXNTL;
        const int M = min(4 * MAXNTL, sh.T - c0);
        if (threadIdx.x < 16) {
            rows[threadIdx.x] = c0 + min((int)threadIdx.x, M - 1);
            list[threadIdx.x] = c0 + threadIdx.x;
        }
        __syncthreads();
        switch ((M + 3) / 4) {
            case 1: up_chunk<1, XF32, kUpWaves, kUpUnr>(sh.w, x, H, sh.Fs, rgp, rows, list, M, red, sh.out); break;
            case 2: up_chunk<MAXNTL < 2 ? 1 : 2, XF32, kUpWaves, kUpUnr>(sh.w, x, H, sh.Fs, rgp, rows, list, M, red,
                                                                         sh.out); break;
            case 3: up_chunk<MAXNTL < 3 ? 1 : 3, XF32, kUpWaves, kUpUnr>(sh.w, x, H, sh.Fs, rgp, rows, list, M, red,
                                                                         sh.out); break;
            default: up_chunk<MAXNTL, XF32, kUpWaves, kUpUnr>(sh.w, x, H, sh.Fs, rgp, rows, list, M, red, sh.out);
        }
        return;
    }
    const int fg = F >> 6, b = (int)blockIdx.x - sh.wgs;
    __shared__ __attribute__((aligned(16))) int sids[kMaxPairs];
    const int e = active_expert<kUpWaves>(ids, P, E, b / fg, sids);
    if (e < 0) return;
    const int rgp = b % fg;
    const int cnt = collect_pairs<kUpWaves>(sids, P, e, list);
    const uint8_t* wexp = gate_up + (int64_t)e * (2 * F / 64) * (H / 32) * kTileBytes;
    for (int c0 = 0; c0 < cnt; c0 += 4 * MAXNTL) {
        const int M = min(4 * MAXNTL, cnt - c0);
        if (threadIdx.x < 16) rows[threadIdx.x] = list[c0 + min((int)threadIdx.x, M - 1)] / topk;
        __syncthreads();
        if constexpr (MAXNTL == 1) {
            up_chunk<1, XF32, kUpWaves, kUpUnr>(wexp, x, H, F, rgp, rows, list + c0, M, red, hbuf);
        } else {
            switch ((M + 3) / 4) {
                case 1: up_chunk<1, XF32, kUpWaves, kUpUnr>(wexp, x, H, F, rgp, rows, list + c0, M, red, hbuf); break;
                case 2: up_chunk<2, XF32, kUpWaves, kUpUnr>(wexp, x, H, F, rgp, rows, list + c0, M, red, hbuf); break;
                case 3: up_chunk<3, XF32, kUpWaves, kUpUnr>(wexp, x, H, F, rgp, rows, list + c0, M, red, hbuf); break;
                default: up_chunk<4, XF32, kUpWaves, kUpUnr>(wexp, x, H, F, rgp, rows, list + c0, M, red, hbuf); break;
            }
        }
        __syncthreads();
    }
}

// NG 64-row groups of H per down workgroup: K = F is short, so one group alone is
// latency-bound.
template <int NTL, int NG, int WAVES, int UNR>
__device__ __forceinline__ void down_chunk(const uint8_t* wexp, const float* hbuf, int H, int F, int rg0,
                                           const int* pairs, int M, float* red, float* __restrict__ ypair) {
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
    gemv_rows_pipe<NTL, true, NG, UNR, WAVES>(gb, hbuf, GatherRows{pairs, M}, F, 0, KB, acc);
    float (*rd)[4][NTL][64] = (float (*)[4][NTL][64])red;
    const int tid = threadIdx.x, lane = tid & 63, r = tid >> 6, i16 = lane & 15, kg = lane >> 4;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        float v[NTL];
        if (i) __syncthreads();
        wave_sum<NTL, WAVES>(acc[i], rd, v);
        const int64_t n = (int64_t)(rg0 + i) * 64 + r * 16 + i16;
        if (r < 4) {
#pragma unroll
            for (int j = 0; j < NTL; ++j) {
                const int tok = token_of(kg, j);
                if (tok < M) ypair[(int64_t)pairs[tok] * H + n] = v[j];
            }
        }
    }
}

// Workgroup (a, g): NG row groups of H from g * NG of the a-th routed expert's down matrix.
// The shared expert's workgroups (sh.wgs, token chunk by row-group span) come first.
template <int NG, int MAXNTL>
__global__ __launch_bounds__(64 * kDnWaves) void moe_down_kernel(const uint8_t* __restrict__ down,
                                                                 const float* __restrict__ hbuf,
                                                                 const int32_t* __restrict__ ids, int P, int E, int H,
                                                                 int F, float* __restrict__ ypair, SharedExpert sh) {
    __shared__ int list[kMaxPairs];
    __shared__ float red[kDnWaves * 4 * MAXNTL * 64];
    const int wg_per_e = (H >> 6) / NG;
    if ((int)blockIdx.x < sh.wgs) {   // the shared expert: y_s = down_s h_s for a chunk of tokens
        const int rg0 = (blockIdx.x % wg_per_e) * NG, c0 = (blockIdx.x / wg_per_e) * 4 * MAXNTL;
        const int M = min(4 * MAXNTL, sh.T - c0);
        if (threadIdx.x < 16) list[threadIdx.x] = c0 + threadIdx.x;
        __syncthreads();
        switch ((M + 3) / 4) {
            case 1: down_chunk<1, NG, kDnWaves, kDnUnr>(sh.w, sh.h, H, sh.Fs, rg0, list, M, red, sh.out); break;
            case 2: down_chunk<MAXNTL < 2 ? 1 : 2, NG, kDnWaves, kDnUnr>(sh.w, sh.h, H, sh.Fs, rg0, list, M, red,
                                                                         sh.out); break;
            case 3: down_chunk<MAXNTL < 3 ? 1 : 3, NG, kDnWaves, kDnUnr>(sh.w, sh.h, H, sh.Fs, rg0, list, M, red,
                                                                         sh.out); break;
            default: down_chunk<MAXNTL, NG, kDnWaves, kDnUnr>(sh.w, sh.h, H, sh.Fs, rg0, list, M, red, sh.out);
        }
        return;
    }
    const int b = (int)blockIdx.x - sh.wgs;
    __shared__ __attribute__((aligned(16))) int sids[kMaxPairs];
    const int e = active_expert<kDnWaves>(ids, P, E, b / wg_per_e, sids);
    if (e < 0) return;
    const int rg0 = (b % wg_per_e) * NG;
    const int cnt = collect_pairs<kDnWaves>(sids, P, e, list);
    const uint8_t* wexp = down + (int64_t)e * (H / 64) * (F / 32) * kTileBytes;
    for (int c0 = 0; c0 < cnt; c0 += 4 * MAXNTL) {
        const int M = min(4 * MAXNTL, cnt - c0);
        if constexpr (MAXNTL == 1) {
            down_chunk<1, NG, kDnWaves, kDnUnr>(wexp, hbuf, H, F, rg0, list + c0, M, red, ypair);
        } else {
            switch ((M + 3) / 4) {
                case 1: down_chunk<1, NG, kDnWaves, kDnUnr>(wexp, hbuf, H, F, rg0, list + c0, M, red, ypair); break;
                case 2: down_chunk<2, NG, kDnWaves, kDnUnr>(wexp, hbuf, H, F, rg0, list + c0, M, red, ypair); break;
                case 3: down_chunk<3, NG, kDnWaves, kDnUnr>(wexp, hbuf, H, F, rg0, list + c0, M, red, ypair); break;
                default: down_chunk<4, NG, kDnWaves, kDnUnr>(wexp, hbuf, H, F, rg0, list + c0, M, red, ypair); break;
            }
        }
        __syncthreads();
    }
}

// out[t][n..n+3] = sum_j w[t][j] y_pair[t][j][n..n+3], slot order j (H % 4 == 0). Workgroup
// (chunk of 1024 n, token t): the token's ids and weights are uniform, and the slots' y loads
// are all issued before the sum.
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ ypair,
                                                          const int32_t* __restrict__ ids,
                                                          const float* __restrict__ w, int topk, int E, int H,
                                                          float* __restrict__ out) {
    const int64_t t = blockIdx.y, n = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (n >= H) return;
    f32x4 y[16];
#pragma unroll
    for (int j = 0; j < 16; ++j)
        if (j < topk) y[j] = load_global<f32x4>(ypair + (t * topk + j) * H + n);
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        if (j < topk) {
            const int e = ids[t * topk + j];
            if (e >= 0 && e < E) {
                const float wp = w[t * topk + j];
#pragma unroll
                for (int c = 0; c < 4; ++c) s[c] += wp * y[j][c];
            }
        }
    }
    *(f32x4*)(out + t * H + n) = s;
}

// The block output with the residual and the gated shared expert folded into the combine
// (moe_fin, designs/moe_combine/moe_fin.py:1-4 and designs/moe_experts/moe_fin.cc:
// out = xres + sum_j w y + sigmoid(xm . sgw) * shared). Workgroup (chunk of 1024 n, token t),
// as moe_combine_kernel:
//   g = sigmoid(x[t] . sgw) (sgw bf16 [H], the dot product in fp32 in a fixed order, so every
//       workgroup of a token forms the same g),
//   out[t][n] = (res[t][n] + sum_j w[t][j] y_pair[t][j][n]) + g shared[t][n],
// the routed sum formed exactly as moe_combine_kernel forms it. res may be null (no
// residual) and may alias out; shared null leaves the gate out.
template <bool XF32>
__global__ __launch_bounds__(256) void moe_fin_kernel(const float* __restrict__ ypair, const int32_t* __restrict__ ids,
                                                      const float* __restrict__ w, int topk, int E, int H,
                                                      const void* __restrict__ x, const uint16_t* __restrict__ sgw,
                                                      const float* __restrict__ shared, const float* res, float* out) {
    __shared__ float red[4];
    const int64_t t = blockIdx.y, n = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
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
    if (n >= H) return;
    f32x4 y[16];
#pragma unroll
    for (int j = 0; j < 16; ++j)
        if (j < topk) y[j] = load_global<f32x4>(ypair + (t * topk + j) * H + n);
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        if (j < topk) {
            const int e = ids[t * topk + j];
            if (e >= 0 && e < E) {
                const float wp = w[t * topk + j];
#pragma unroll
                for (int c = 0; c < 4; ++c) s[c] += wp * y[j][c];
            }
        }
    }
    f32x4 v = s;
    if (res) v = *(const f32x4*)(res + t * H + n) + s;
    if (shared) {
        const f32x4 sv = *(const f32x4*)(shared + t * H + n);
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = __builtin_fmaf(g, sv[c], v[c]);
    }
    *(f32x4*)(out + t * H + n) = v;
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

}  // namespace

extern "C" size_t q4_moe_workspace_bytes(int T, int E, int topk, int H, int F) {
    (void)E;
    if (T <= 0 || topk <= 0 || H <= 0 || F <= 0) return 0;
    const size_t P = (size_t)T * topk;
    return align256(P * F * 4) + align256(P * H * 4);
}

extern "C" size_t q4_moe_shared_workspace_bytes(int T, int E, int topk, int H, int F, int Fs) {
    if (Fs <= 0) return 0;
    const size_t base = q4_moe_workspace_bytes(T, E, topk, H, F);
    return base ? base + align256((size_t)T * Fs * 4) + align256((size_t)T * H * 4) : 0;
}

// The expert kernels, then the plain combine (fin == false) or the finish with residual and
// gated shared expert (fin == true). With shared_gu / shared_dn the shared expert (inner size
// Fs) runs inside the expert kernels and its output, in the workspace, is the finish's
// `shared`.
static int moe_impl(const uint8_t* gate_up, const uint8_t* down, const void* x, int x_dtype, const int32_t* topk_ids,
                    const float* topk_w, float* out, int T, int E, int topk, int64_t H, int64_t F, void* workspace,
                    size_t workspace_bytes, void* stream, bool fin, const float* residual, const float* shared,
                    const uint16_t* shared_gate_w, const uint8_t* shared_gu = nullptr,
                    const uint8_t* shared_dn = nullptr, int64_t Fs = 0) {
    if (x_dtype != Q4MI_F32 && x_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (fin && !shared_gu && (!shared) != (!shared_gate_w)) return Q4MI_E_ARG;
    if (H <= 0 || F <= 0 || H % 64 || F % 64) return Q4MI_E_SHAPE;
    if (H > (1 << 24) || F > (1 << 24)) return Q4MI_E_RANGE;
    if (T < 0 || E <= 0 || E > kMaxExperts || topk <= 0 || topk > 16 || (int64_t)T * topk > kMaxPairs)
        return Q4MI_E_RANGE;
    const bool with_shared = shared_gu != nullptr;
    if (with_shared && (Fs <= 0 || Fs % 64)) return Q4MI_E_SHAPE;
    if (with_shared && Fs > (1 << 24)) return Q4MI_E_RANGE;
    if (T == 0) return Q4MI_OK;
    if (!gate_up || !down || !x || !topk_ids || !topk_w || !out) return Q4MI_E_ARG;
    if (misaligned16(gate_up) || misaligned16(down) || misaligned16(x) || misaligned16(out) || misaligned16(workspace))
        return Q4MI_E_ARG;
    if (with_shared && (!shared_dn || misaligned16(shared_gu) || misaligned16(shared_dn))) return Q4MI_E_ARG;
    const size_t need = with_shared ? q4_moe_shared_workspace_bytes(T, E, topk, (int)H, (int)F, (int)Fs)
                                    : q4_moe_workspace_bytes(T, E, topk, (int)H, (int)F);
    if (!workspace || workspace_bytes < need) return Q4MI_E_WORKSPACE;
    const int P = T * topk;
    float* hbuf = (float*)workspace;
    float* ypair = (float*)((char*)workspace + align256((size_t)P * F * 4));
    const hipStream_t st = (hipStream_t)stream;
    // Workgroups for every expert that could be routed (at most min(E, P)); those past the
    // routed count leave at once.
    const int64_t routed_max = E < P ? E : P;
    const int ng = H % (64 * kDnGroups) == 0 ? kDnGroups : 1;
    // At most 2 routed pairs per expert on average (decode batches): the one-accumulator
    // instances, whose lower register use keeps more waves per SIMD. Larger batches stream
    // each expert's rows once per 16 tokens instead of once per 4.
    const bool few = P <= 2 * E;
    SharedExpert su{}, sd{};
    if (with_shared) {   // its buffers follow the routed ones; T / (4 MAXNTL) token chunks
        const int chunks = (int)ceil_div(T, few ? 4 : 16);
        float* hs = (float*)((char*)ypair + align256((size_t)P * H * 4));
        float* ys = (float*)((char*)hs + align256((size_t)T * Fs * 4));
        su = SharedExpert{shared_gu, hs, nullptr, (int)Fs, T, chunks * (int)(Fs / 64)};
        sd = SharedExpert{shared_dn, ys, hs, (int)Fs, T, chunks * (int)(H / (64 * ng))};
        shared = ys;
    }
    const dim3 gu((unsigned)(su.wgs + routed_max * (F / 64))), dn((unsigned)(sd.wgs + routed_max * (H / (64 * ng))));
    const dim3 bu(64 * kUpWaves), bd(64 * kDnWaves);
    if (x_dtype == Q4MI_F32) {
        if (few)
            hipLaunchKernelGGL((moe_up_kernel<true, 1>), gu, bu, 0, st, gate_up, x, topk_ids, P, E, topk, (int)H,
                               (int)F, hbuf, su);
        else
            hipLaunchKernelGGL((moe_up_kernel<true, 4>), gu, bu, 0, st, gate_up, x, topk_ids, P, E, topk, (int)H,
                               (int)F, hbuf, su);
    } else {
        if (few)
            hipLaunchKernelGGL((moe_up_kernel<false, 1>), gu, bu, 0, st, gate_up, x, topk_ids, P, E, topk, (int)H,
                               (int)F, hbuf, su);
        else
            hipLaunchKernelGGL((moe_up_kernel<false, 4>), gu, bu, 0, st, gate_up, x, topk_ids, P, E, topk, (int)H,
                               (int)F, hbuf, su);
    }
    if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
    if (ng == kDnGroups) {
        if (few)
            hipLaunchKernelGGL((moe_down_kernel<kDnGroups, 1>), dn, bd, 0, st, down, hbuf, topk_ids, P, E, (int)H,
                               (int)F, ypair, sd);
        else
            hipLaunchKernelGGL((moe_down_kernel<kDnGroups, 4>), dn, bd, 0, st, down, hbuf, topk_ids, P, E, (int)H,
                               (int)F, ypair, sd);
    } else {
        if (few)
            hipLaunchKernelGGL((moe_down_kernel<1, 1>), dn, bd, 0, st, down, hbuf, topk_ids, P, E, (int)H, (int)F,
                               ypair, sd);
        else
            hipLaunchKernelGGL((moe_down_kernel<1, 4>), dn, bd, 0, st, down, hbuf, topk_ids, P, E, (int)H, (int)F,
                               ypair, sd);
    }
    if (launch_status() != Q4MI_OK) return Q4MI_E_LAUNCH;
    if (fin) {
        const dim3 grid((unsigned)ceil_div(H / 4, 256), (unsigned)T);
        if (x_dtype == Q4MI_F32)
            hipLaunchKernelGGL(moe_fin_kernel<true>, grid, dim3(256), 0, st, ypair, topk_ids, topk_w, topk, E, (int)H,
                               x, shared_gate_w, shared, residual, out);
        else
            hipLaunchKernelGGL(moe_fin_kernel<false>, grid, dim3(256), 0, st, ypair, topk_ids, topk_w, topk, E,
                               (int)H, x, shared_gate_w, shared, residual, out);
        return launch_status();
    }
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)ceil_div(H / 4, 256), (unsigned)T), dim3(256), 0, st, ypair,
                       topk_ids, topk_w, topk, E, (int)H, out);
    return launch_status();
}

extern "C" int q4_moe_gemv(const uint8_t* gate_up, const uint8_t* down, const void* x, int x_dtype,
                           const int32_t* topk_ids, const float* topk_w, float* out, int T, int E, int topk,
                           int64_t H, int64_t F, void* workspace, size_t workspace_bytes, void* stream) {
    return moe_impl(gate_up, down, x, x_dtype, topk_ids, topk_w, out, T, E, topk, H, F, workspace, workspace_bytes,
                    stream, false, nullptr, nullptr, nullptr);
}

extern "C" int q4_moe_gemv_shared(const uint8_t* gate_up, const uint8_t* down, const uint8_t* shared_gate_up,
                                  const uint8_t* shared_down, int64_t Fs, const uint16_t* shared_gate_w,
                                  const void* x, int x_dtype, const int32_t* topk_ids, const float* topk_w,
                                  const float* residual, float* out, int T, int E, int topk, int64_t H, int64_t F,
                                  void* workspace, size_t workspace_bytes, void* stream) {
    if (!shared_gate_up || !shared_down || !shared_gate_w) return Q4MI_E_ARG;
    if (residual && misaligned16(residual)) return Q4MI_E_ARG;
    // out [T][H] may alias the residual, nothing else the kernels read or the workspace
    const int64_t row_bytes = (int64_t)T * H * 4;
    if (out && workspace && overlaps(out, row_bytes, workspace, (int64_t)workspace_bytes)) return Q4MI_E_ARG;
    return moe_impl(gate_up, down, x, x_dtype, topk_ids, topk_w, out, T, E, topk, H, F, workspace, workspace_bytes,
                    stream, true, residual, nullptr, shared_gate_w, shared_gate_up, shared_down, Fs);
}

extern "C" int q4_moe_gemv_fin(const uint8_t* gate_up, const uint8_t* down, const void* x, int x_dtype,
                               const int32_t* topk_ids, const float* topk_w, const float* residual,
                               const float* shared, const uint16_t* shared_gate_w, float* out, int T, int E, int topk,
                               int64_t H, int64_t F, void* workspace, size_t workspace_bytes, void* stream) {
    if ((residual && misaligned16(residual)) || (shared && misaligned16(shared))) return Q4MI_E_ARG;
    return moe_impl(gate_up, down, x, x_dtype, topk_ids, topk_w, out, T, E, topk, H, F, workspace, workspace_bytes,
                    stream, true, residual, shared, shared_gate_w);
}
