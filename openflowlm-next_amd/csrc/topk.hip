// topk.hip -- the lm_head's sampling epilogue: for each token row of logits, the k largest
// (value descending, the lower id first on a tie), as ids and values; k = 1 is the greedy
// argmax. Plus q4_lm_head_topk, the lm_head GEMV followed by it on one stream.
//
// Reference semantics followed:
//   greedy: Sampler::sample_greedy (src/common/modules/sampler.cpp:355-430) over
//     Engine::logits_view's bf16 logits (src/open_qwen36/engine.cpp:125-131), stated
//     for the tests as argmax_bf16 (src/open_qwen36/cli.cpp:103-113): each f32 logit
//     rounded to bf16 (RNE, the plain formula), an f32 subnormal read as 0, strict '>'
//     from -inf so the lowest id wins a tie and an all -inf / NaN row gives id 0; rows
//     past the real vocabulary read as -inf.
//   top-k: Sampler::sampler_topk_apply (sampler.cpp:222-245): value descending, lower id
//     first when the values are equal.
//
// Every (value, id) becomes one uint64 key whose unsigned order is that order:
//   high word: the value's bits made monotone (sign set -> all bits flipped, else the
//   sign bit set), with -0 read as +0 and NaN as 0, below every number; low word: ~id.
// Padding slots are key 0, below every real key. Each lane holds 4 keys. For k <= 8 a
// block of 4 waves takes 1024 logits: each lane sorts its 4 keys in registers, each
// wave pops its k largest with k pairs of DPP wave reductions, and wave 0 merges the
// four wave lists the same way. For larger k a block of 16 waves takes 4096: each wave
// runs a bitonic network over its 256 keys and the top-64 lists merge 16 -> 4 -> 1 with
// the network's last two stages. Blocks emit k keys each; the same kernel then runs over those keys
// until one block per token remains, which writes ids and values.
#include "q4mi_device.h"
#include "q4mi_internal.h"

using namespace q4mi;

namespace {

constexpr int kLanes = 64, kWaves = 4, kThreads = kLanes * kWaves, kPerLane = 4;
constexpr int kChunk = kThreads * kPerLane;     // 1024 inputs per block
constexpr int kMaxK = 64;

__device__ __forceinline__ uint32_t monotone(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float from_monotone(uint32_t k) {
    return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// mode 0: the f32 logit; mode 1: what the sampler sees (bf16 RNE, f32 subnormal -> 0).
__device__ __forceinline__ uint64_t logit_key(float v, uint32_t id, int mode) {
    if (mode == 1) {
        const uint32_t u = __builtin_bit_cast(uint32_t, v);
        v = ((u & 0x7F800000u) == 0) ? 0.0f : __builtin_bit_cast(float, f32_to_bf16_rne(v) << 16);
    }
    if (v == 0.0f) v = 0.0f;                          // -0 ties with +0
    const uint32_t hi = (v != v) ? 0u : monotone(v);  // NaN below every number
    return ((uint64_t)hi << 32) | (uint32_t)~id;
}

// Wave-wide unsigned max / min with the result in every lane: DPP steps (xor 1 and 2
// within quads, half-row and row mirrors, then the row broadcasts of lanes 15 and 31)
// leave the total in lane 63, which readlane hands to the whole wave.
template <bool MAX>
__device__ __forceinline__ uint32_t dpp_step(uint32_t v, uint32_t o) {
    return MAX ? (o > v ? o : v) : (o < v ? o : v);
}

template <bool MAX>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v) {
    v = dpp_step<MAX>(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false));
    v = dpp_step<MAX>(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false));
    v = dpp_step<MAX>(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x141, 0xF, 0xF, false));
    v = dpp_step<MAX>(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x140, 0xF, 0xF, false));
    v = dpp_step<MAX>(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xA, 0xF, false));
    v = dpp_step<MAX>(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xC, 0xF, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Sort N keys descending in registers (bitonic network, all indices compile-time).
template <int N>
__device__ __forceinline__ void sort_desc(uint64_t (&a)[N]) {
#pragma unroll
    for (int s = 2; s <= N; s <<= 1)
#pragma unroll
        for (int j = s >> 1; j > 0; j >>= 1)
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const int l = i ^ j;
                if (l > i) {
                    const bool desc = (i & s) == 0;
                    const uint64_t x = a[i], y = a[l];
                    const bool swap = desc ? (x < y) : (x > y);
                    a[i] = swap ? y : x;
                    a[l] = swap ? x : y;
                }
            }
}

// Pop the k largest keys of the wave (each lane's a[] sorted descending): lane t < k
// returns the t-th largest, or 0 when the wave held fewer than t + 1 real keys. Each
// pop is two 32-bit wave reductions: the largest value, then the lowest id holding it
// (a padding slot is value 0 with id 0xFFFFFFFF; a NaN is value 0 with its own id).
template <int N>
__device__ __forceinline__ uint64_t wave_pop(uint64_t (&a)[N], int k, int lane) {
    uint64_t mine = 0;
    for (int t = 0; t < k; ++t) {
        const uint32_t hv = (uint32_t)(a[0] >> 32), hid = ~(uint32_t)a[0];
        const uint32_t mv = wave_reduce_u32<true>(hv);
        const uint32_t mid = wave_reduce_u32<false>(hv == mv ? hid : 0xFFFFFFFFu);
        if (mv == 0 && mid == 0xFFFFFFFFu) break;          // only padding left (wave-uniform)
        if (lane == t) mine = ((uint64_t)mv << 32) | (uint32_t)~mid;
        if (hv == mv && hid == mid) {                       // the one lane that held it
#pragma unroll
            for (int i = 0; i + 1 < N; ++i) a[i] = a[i + 1];
            a[N - 1] = 0;
        }
    }
    return mine;
}

// Exchange a 32-bit value with lane ^ M (M = 1, 2: DPP quad permutes; 4..16: ds_swizzle's
// xor mode; 32: ds_bpermute).
template <int M>
__device__ __forceinline__ uint32_t xchg(uint32_t v, int lane) {
    if constexpr (M == 1)
        return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false);
    else if constexpr (M == 2)
        return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false);
    else if constexpr (M < 32)
        return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, (M << 10) | 0x1F);
    else
        return (uint32_t)__builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, (int)v);
}

// One stage (size S, distance J) of the bitonic network over the wave's 256 keys, key e
// = 4 lane + r held in a[r]: position e keeps the larger of (e, e ^ J) when it is the
// lower of the pair and its S-run sorts descending ((e & S) == 0), else the smaller.
template <int S, int J>
__device__ __forceinline__ void bitonic_stage(uint64_t (&a)[4], int lane) {
    if constexpr (J >= 4) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint64_t o = ((uint64_t)xchg<J / 4>((uint32_t)(a[r] >> 32), lane) << 32) |
                               xchg<J / 4>((uint32_t)a[r], lane);
            const int e = 4 * lane + r;
            const bool keep_max = ((e & J) == 0) == ((e & S) == 0);
            const uint64_t hi = o > a[r] ? o : a[r], lo = o > a[r] ? a[r] : o;
            a[r] = keep_max ? hi : lo;
        }
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if ((r & J) == 0) {
                const bool desc = ((4 * lane + r) & S) == 0;
                const uint64_t x = a[r], y = a[r ^ J];
                const bool swap = desc ? (x < y) : (x > y);
                a[r] = swap ? y : x;
                a[r ^ J] = swap ? x : y;
            }
        }
    }
}

template <int S, int J>
__device__ __forceinline__ void bitonic_merge(uint64_t (&a)[4], int lane) {
    bitonic_stage<S, J>(a, lane);
    if constexpr (J > 1) bitonic_merge<S, J / 2>(a, lane);
}

// Stages S0, 2 S0, ..., 256: with S0 = 2 a full descending sort of the wave's 256 keys;
// with S0 = 128 the merge of two bitonic 128-runs (desc then asc halves) into one.
template <int S0>
__device__ __forceinline__ void bitonic256(uint64_t (&a)[4], int lane) {
    bitonic_merge<S0, S0 / 2>(a, lane);
    if constexpr (S0 < 256) bitonic256<S0 * 2>(a, lane);
}

// The k > 8 block: 16 waves over 4096 inputs. Each wave brings its 256 keys to a
// descending order -- logits with the full network; keys of an earlier pass, which
// arrive as sorted runs of 64, with only the last two stages (odd runs read reversed,
// so each pair of runs is a bitonic 128-run). The waves' top-64 lists are merged four
// at a time with the same two stages: 16 -> 4 -> 1. Non-final passes write their
// sorted top 64 (a superset of the top k); the final pass writes the first k as ids and
// values. Cost does not depend on k.
constexpr int kSortWaves = 16, kSortThreads = kSortWaves * kLanes, kSortChunk = kSortThreads * kPerLane;

__device__ __forceinline__ void merge4(uint64_t (&a)[4], const uint64_t (*lists)[kLanes], int lane) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int e = 4 * lane + r;
        a[r] = lists[e >> 6][e & 63];
    }
    bitonic256<128>(a, lane);
}

__device__ __forceinline__ void put_top64(const uint64_t (&a)[4], uint64_t* list, bool reversed, int lane) {
    if (lane < 16) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int e = 4 * lane + r;
            list[reversed ? 63 - e : e] = a[r];
        }
    }
}

template <bool KEYS, bool FINAL>
__global__ __launch_bounds__(kSortThreads) void topk_sort_kernel(const void* __restrict__ in, int64_t ld, int64_t n,
                                                                 int k, int mode, uint64_t* __restrict__ out_keys,
                                                                 int32_t* __restrict__ ids,
                                                                 float* __restrict__ vals) {
    __shared__ uint64_t l1[kSortWaves][kLanes], l2[4][kLanes];
    const int lane = threadIdx.x & (kLanes - 1), wave = threadIdx.x / kLanes;
    const int64_t s = blockIdx.x, m = blockIdx.y;
    const int64_t base = s * kSortChunk + wave * (kLanes * kPerLane);
    uint64_t a[kPerLane];
    if constexpr (KEYS) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int e = 4 * lane + r;                      // run e >> 6 of this wave, odd runs reversed
            const int64_t i = base + (e & ~63) + (((e >> 6) & 1) ? 63 - (e & 63) : (e & 63));
            a[r] = i < n ? ((const uint64_t*)in)[m * ld + i] : 0;
        }
        bitonic256<128>(a, lane);
    } else {
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {
            const int64_t i = base + j * kLanes + lane;      // coalesced
            a[j] = i < n ? logit_key(((const float*)in)[m * ld + i], (uint32_t)i, mode) : 0;
        }
        bitonic256<2>(a, lane);
    }
    put_top64(a, l1[wave], wave & 1, lane);
    __syncthreads();
    if (wave < 4) {
        merge4(a, l1 + 4 * wave, lane);
        put_top64(a, l2[wave], wave & 1, lane);
    }
    __syncthreads();
    if (wave != 0) return;
    merge4(a, l2, lane);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int e = 4 * lane + r;
        const uint64_t key = a[r];
        if constexpr (FINAL) {
            if (e < k) {
                ids[m * k + e] = key ? (int32_t)~(uint32_t)key : -1;
                if (vals) vals[m * k + e] = key ? from_monotone((uint32_t)(key >> 32)) : -__builtin_inff();
            }
        } else if (e < 64) {
            out_keys[(m * gridDim.x + s) * 64 + e] = key;
        }
    }
}

// One block: inputs [s*1024, min(n, (s+1)*1024)) of token row m -> its k largest keys.
// KEYS: the inputs are keys of an earlier pass (uint64[M][n]); else f32 logits (row
// stride ld). FINAL: write ids / values; else keys to out_keys[m][s][k].
template <bool KEYS, bool FINAL>
__global__ __launch_bounds__(kThreads) void topk_kernel(const void* __restrict__ in, int64_t ld, int64_t n,
                                                        int k, int mode, uint64_t* __restrict__ out_keys,
                                                        int32_t* __restrict__ ids, float* __restrict__ vals) {
    __shared__ uint64_t lists[kWaves][kLanes];
    const int lane = threadIdx.x & (kLanes - 1), wave = threadIdx.x / kLanes;
    const int64_t s = blockIdx.x, m = blockIdx.y;
    const int64_t base = s * kChunk + wave * (kLanes * kPerLane);
    uint64_t a[kPerLane];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
        const int64_t i = base + j * kLanes + lane;          // coalesced: 64 consecutive per j
        if (i < n) {
            if constexpr (KEYS)
                a[j] = ((const uint64_t*)in)[m * ld + i];
            else
                a[j] = logit_key(((const float*)in)[m * ld + i], (uint32_t)i, mode);
        } else {
            a[j] = 0;
        }
    }
    sort_desc(a);
    lists[wave][lane] = wave_pop(a, k, lane);
    __syncthreads();
    if (wave != 0) return;
    uint64_t b[kWaves];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) b[w] = lists[w][lane];
    sort_desc(b);
    const uint64_t key = wave_pop(b, k, lane);
    if (lane < k) {
        if constexpr (FINAL) {
            ids[m * k + lane] = key ? (int32_t)~(uint32_t)key : -1;
            if (vals) vals[m * k + lane] = key ? from_monotone((uint32_t)(key >> 32)) : -__builtin_inff();
        } else {
            out_keys[(m * gridDim.x + s) * k + lane] = key;
        }
    }
}

constexpr int kPopMaxK = 8;     // k above this: the sorting-network block

// Pass geometry: inputs per block and keys each non-final block writes.
struct TopkPlan {
    bool pop;
    int64_t chunk;
    int out;
};

inline TopkPlan topk_plan(int k) {
    return k <= kPopMaxK ? TopkPlan{true, kChunk, k} : TopkPlan{false, kSortChunk, 64};
}

template <bool KEYS>
void launch_topk(const TopkPlan& p, bool final_pass, dim3 grid, hipStream_t st, const void* in, int64_t ld,
                 int64_t n, int k, int mode, uint64_t* out_keys, int32_t* ids, float* vals) {
    if (p.pop) {
        if (final_pass)
            hipLaunchKernelGGL((topk_kernel<KEYS, true>), grid, dim3(kThreads), 0, st, in, ld, n, k, mode, out_keys,
                               ids, vals);
        else
            hipLaunchKernelGGL((topk_kernel<KEYS, false>), grid, dim3(kThreads), 0, st, in, ld, n, k, mode,
                               out_keys, ids, vals);
    } else {
        if (final_pass)
            hipLaunchKernelGGL((topk_sort_kernel<KEYS, true>), grid, dim3(kSortThreads), 0, st, in, ld, n, k, mode,
                               out_keys, ids, vals);
        else
            hipLaunchKernelGGL((topk_sort_kernel<KEYS, false>), grid, dim3(kSortThreads), 0, st, in, ld, n, k,
                               mode, out_keys, ids, vals);
    }
}

inline size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// Two key buffers, ping-ponged: the first pass's output, and the second's (every later
// pass writes fewer keys than the one two before it).
size_t topk_ws(int M, int64_t n, int k) {
    const TopkPlan p = topk_plan(k);
    const int64_t s1 = ceil_div(n, p.chunk);
    if (s1 <= 1) return 0;
    const int64_t s2 = ceil_div(s1 * p.out, p.chunk);
    return align256((size_t)M * s1 * p.out * 8) + (s2 > 1 ? align256((size_t)M * s2 * p.out * 8) : 0);
}

}  // namespace

extern "C" size_t q4_topk_workspace_bytes(int M, int64_t n, int k) {
    if (M <= 0 || n <= 0 || k < 1 || k > kMaxK) return 0;
    return topk_ws(M, n, k);
}

extern "C" int q4_logits_topk(const float* logits, int64_t ld, int M, int64_t n, int k, int mode, int32_t* ids,
                              float* vals, void* workspace, size_t workspace_bytes, void* stream) {
    if (k < 1 || k > kMaxK || (mode != 0 && mode != 1)) return Q4MI_E_RANGE;
    if (M < 0 || M > 65535) return Q4MI_E_RANGE;
    if (M == 0) return Q4MI_OK;
    if (n <= 0 || ld < n) return Q4MI_E_SHAPE;
    if (!logits || !ids) return Q4MI_E_ARG;
    if ((uintptr_t)workspace & 7) return Q4MI_E_ARG;
    const size_t need = topk_ws(M, n, k);
    if (need && (!workspace || workspace_bytes < need)) return Q4MI_E_WORKSPACE;
    const hipStream_t st = (hipStream_t)stream;
    const TopkPlan p = topk_plan(k);
    int64_t s = ceil_div(n, p.chunk);
    uint64_t* buf[2] = {(uint64_t*)workspace,
                        need ? (uint64_t*)((char*)workspace + align256((size_t)M * s * p.out * 8)) : nullptr};
    launch_topk<false>(p, s == 1, dim3((unsigned)s, (unsigned)M), st, logits, ld, n, k, mode, buf[0], ids, vals);
    int cur = 0;
    while (s > 1) {                 // reduce the keys of s blocks per token until one block is left
        const int64_t len = s * p.out;
        s = ceil_div(len, p.chunk);
        launch_topk<true>(p, s == 1, dim3((unsigned)s, (unsigned)M), st, buf[cur], len, len, k, mode, buf[cur ^ 1],
                          ids, vals);
        cur ^= 1;
    }
    return launch_status();
}

extern "C" size_t q4_lm_head_workspace_bytes(int M, int64_t N, int64_t K, int k) {
    if (M <= 0 || M > 16 || N <= 0 || k < 1 || k > kMaxK) return 0;
    return align256(q4_gemv_workspace_bytes(M, N, K)) + topk_ws(M, N, k);
}

extern "C" int q4_lm_head_topk(const uint8_t* packed, const void* x, int x_dtype, float* logits, int M, int64_t N,
                               int64_t K, int64_t n_valid, int k, int mode, int32_t* ids, float* vals,
                               void* workspace, size_t workspace_bytes, void* stream) {
    if (n_valid <= 0 || n_valid > N) return Q4MI_E_SHAPE;
    if (k < 1 || k > kMaxK || (mode != 0 && mode != 1)) return Q4MI_E_RANGE;
    if (M < 0 || M > 16) return Q4MI_E_RANGE;
    if (M == 0) return Q4MI_OK;
    if (!ids) return Q4MI_E_ARG;
    const size_t gws = q4_gemv_workspace_bytes(M, N, K);
    const size_t need = align256(gws) + topk_ws(M, n_valid, k);
    if (need && (!workspace || workspace_bytes < need)) return Q4MI_E_WORKSPACE;
    int rc = q4_gemv(packed, x, x_dtype, logits, M, N, K, gws ? workspace : nullptr, gws, stream);
    if (rc != Q4MI_OK) return rc;
    void* tws = need > align256(gws) ? (void*)((char*)workspace + align256(gws)) : nullptr;
    return q4_logits_topk(logits, N, M, n_valid, k, mode, ids, vals, tws, need - align256(gws), stream);
}
