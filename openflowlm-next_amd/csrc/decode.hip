// decode.hip -- the decoder layer's GEMV chain between two attentions, M = 1, in one launch:
//
//   x' = x + W_o a                          (a: the attention output, bf16)
//   h  = bf16(silu(W_g n') * (W_u n'))      n' = bf16(RMSNorm(x') * w_post)
//   x" = x' + W_d h
//   q  = W_qkv n"                           n" = bf16(RMSNorm(x") * w_next) (the next layer's)
//
// The reference runs a whole dense layer as one dispatch and one instruction stream
// (open_kernels/designs/dense/dx.py:1-5: ln -> q|k|v -> attention -> o -> ln(+res) ->
// up|gate -> silu*up -> down -> +res). Here the span between two attentions (attention is
// not on this path) is one persistent launch of one 512-thread workgroup per CU, four
// phases separated by grid barriers:
//
//   1. o      items (64-row group, K split): partial planes po[So][H]
//   2. gate/up items (64-row group of F, whole K), the norm of x + po in the prelude: h
//   3. down   items (64-row group, K split of F), h's K range staged in LDS: planes pd[Sd][H]
//   4. qkv    items (QNG row groups, K split), the norm of x' + pd in the prelude: pq[Sq][NQ]
//
// A barrier's cost is hidden behind weight traffic: before a workgroup waits for the
// previous phase, it issues the first K positions of its next item's weight loads (they do
// not depend on anything), so HBM keeps streaming while the phases hand over. o's and
// qkv's items are short enough for all of their positions to be in flight at the wait.
//
// Hand-over, without cache-wide fences (an agent-scope release fence writes back the XCD's
// whole L2, which measured ~8 us per hand-over here):
// - The values one phase hands to the next (po, h, x', pd) are stored write-through at
//   device scope (relaxed agent-scope atomic stores, `sc1`); each wave then waits for its
//   stores to complete (vmcnt 0) before the workgroup barrier, and thread 0 adds one arrival
//   (relaxed, agent scope) to one of 16 counters of that hand-over (workgroup w: counter
//   w % 16, each counter on its own 256 bytes, so the 256 arrivals are not serialised on
//   one address).
// - A waiting workgroup's first wave polls the 16 counters (one device-scope load per lane,
//   s_sleep between polls) until they sum to the grid, then the workgroup barrier releases
//   its waves. Its reads of the handed-over values are ordinary loads: no workgroup reads
//   them earlier in the launch (each buffer is read only after its hand-over), so no cache
//   holds an older copy (caches are invalidated at kernel start), and the stores have
//   reached the device's coherence point before the arrival was issued.
// - Every wait is bounded (kSpinLimit polls, about a second): a wait that runs out raises
//   the flag word and goes on, so the grid always drains (the results are then not to be
//   used).
// - The counters return to zero off the critical path, so a graph replays with no memset
//   and no workgroup waits for a last atomic before it exits: workgroup 0 zeroes hand-overs
//   1 and 2 (which the previous call left counted) before its arrival at hand-over 0, and
//   hand-over 0 after its first down item (every wait on hand-over 0 is over once it has
//   passed hand-over 1). A workgroup arrives at hand-over h + 1 only after hand-over h is
//   complete (a workgroup with no item in a phase still waits for that phase's hand-over),
//   so no arrival at hand-over 1 or 2 can come before workgroup 0's zeroing, which its own
//   first arrival waits for.
// - A wave's stores count in its vmcnt, so a store issued ahead of a weight stream holds the
//   stream's first wait until the store is acknowledged. Workgroup 0's extra stores (the
//   zeroing, x', x") therefore come after its streams, and the loads a norm prelude can
//   issue early (the residual row, the norm weight; x' is complete from hand-over 1 on) go
//   out with the primed weights, before the wait.
// The grid is at most one workgroup per CU (checked against the occupancy the runtime
// reports), so every workgroup is resident while others wait for it.
//
// Sums are deterministic: each output is one workgroup's (fixed wave-sum order), each plane
// sum is added in split order by its consumer (seg_norm_row).
#include <stdlib.h>

#include <algorithm>

#include "gemv_core.h"
#include "q4mi_internal.h"

using namespace q4mi;

namespace {

constexpr int kSegWaves = 8;
constexpr int kSegThreads = 64 * kSegWaves;
constexpr int kSegXs = 16384;               // bf16 activations staged per workgroup (LDS)
constexpr int kSegRow = 256 * kAccRowJ;     // the longest row stage_norm_acc_row normalises
constexpr uint32_t kSpinLimit = 1u << 20;   // polls before a grid wait gives up
// The workspace's first kSyncBytes: hand-over h (0..2), counter j (0..15) at word
// (16 h + j) * 64; the time-out flag at word 49 * 64.
constexpr int kSlots = 16, kSlotWords = 64;
constexpr int kFlagWord = 49 * kSlotWords;
constexpr size_t kSyncBytes = 50 * kSlotWords * 4;

struct SegParams {
    const uint8_t* o;          // [H, H] mx
    const uint8_t* gate;       // [F, H] mx
    const uint8_t* up;         // [F, H] mx
    const uint8_t* down;       // [H, F] mx
    const uint8_t* qkv;        // [NQ, H] mx, or null: phases 1-3 only
    const uint16_t* attn;      // bf16 [H]
    const float* x;            // f32 [H], the residual stream in (may be x_next)
    float* xmid;               // f32 [H]: x' (workgroup 0 writes it)
    float* xnext;              // f32 [H]: x" (workgroup 0 writes it; qkv given)
    const void* nw_post;       // RMSNorm weight in front of gate/up [H]
    const void* nw_next;       // the next layer's RMSNorm weight in front of qkv [H]
    float eps;
    uint16_t* h;               // bf16 [F] (workspace)
    float* po;                 // [So][H] (workspace)
    float* pd;                 // [Sd][H]
    float* pq;                 // [Sq][NQ]
    uint32_t* sync;            // counters (kSyncBytes, see kSlots)
    int H, F, NQ;
    int So, Sd, Sq;
};

// The rolling weight pipeline of gemv_rows_stream (XS form: activations staged in LDS) for
// one K range [kb0, kb1) over NG row groups, split in two so the first UNR positions can be
// issued before the workgroup waits for its activations: prime() issues them, run() waits,
// computes and keeps UNR positions in flight to the end. Wave w takes positions kb0 + w,
// kb0 + w + 8, ...; every wave of an item has at least one (the host's splits leave >= 8
// positions per item). Positions of the last chunk past the wave's count re-load its last
// tile and are not accumulated. Same arithmetic and order as gemv_rows_stream.
// XG: the activations come from a bf16 row in global memory instead (xg, position t at
// t * 32), one more load per position, so no staging pass sits in front of the stream.
template <int NG, int UNR, bool XG = false>
struct SegStream {
    static constexpr int L = 2 * NG + (XG ? 1 : 0);     // loads per position
    static_assert((UNR - 1) * L <= 63, "vmcnt holds 6 bits");
    const uint8_t* gb[NG];
    const uint16_t* xg = nullptr;
    int first, cnt;
    u32x4 c[UNR][NG], s[UNR][NG], xr[UNR];

    __device__ __forceinline__ void setup(const uint8_t* const (&gbase)[NG], int kb0, int kb1) {
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
        for (int i = 0; i < NG; ++i) gb[i] = gbase[i];
        first = __builtin_amdgcn_readfirstlane(kb0 + wave);
        cnt = __builtin_amdgcn_readfirstlane((kb1 - first + kSegWaves - 1) / kSegWaves);
    }
    __device__ __forceinline__ void issue(int b, int slot) {
        const int lane = threadIdx.x & 63;
        const uint32_t coff = lane * 16, soff = kCodeBytes + (lane & 15) * 16;
        const uint32_t toff = (uint32_t)(first + kSegWaves * min(b, cnt - 1)) * kTileBytes;
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            pipe_load_w(c[slot][i], gb[i], toff + coff);
            pipe_load_w(s[slot][i], gb[i], toff + soff);
        }
        if constexpr (XG)
            pipe_load_x(xr[slot], xg + (int64_t)(first + kSegWaves * min(b, cnt - 1)) * 32 + (lane >> 4) * 8);
    }
    __device__ __forceinline__ void prime() {
#pragma unroll
        for (int u = 0; u < UNR; ++u) issue(u, u);
    }
    // xs: the activations of positions [xkb, ...) as bf16 in LDS (position t at (t - xkb) * 32),
    // unless XG
    __device__ __forceinline__ void run(const __bf16* xs, int xkb, float (&acc)[NG][4][1]) {
        const int lane = threadIdx.x & 63;
        const CodeConsts kc = code_consts();
        const __bf16* xsl = xs + (lane >> 4) * 8 - (int64_t)xkb * 32;
        auto land = [&](int slot) {
#pragma unroll
            for (int i = 0; i < NG; ++i) {
                pipe_landed(c[slot][i]);
                pipe_landed(s[slot][i]);
            }
            if constexpr (XG) pipe_landed(xr[slot]);
        };
        auto pos = [&](int u, int b) {
            bf16x8 xh;
            if constexpr (XG) xh = __builtin_bit_cast(bf16x8, xr[u]);
            else xh = *(const bf16x8*)(xsl + (int64_t)(first + kSegWaves * b) * 32);
            tile_math<1, false, false, NG>(c[u], s[u], xh, xh, kc, acc);
        };
        int b0 = 0;
        for (; b0 + UNR < cnt; b0 += UNR) {
#pragma unroll
            for (int u = 0; u < UNR; ++u) {
                __builtin_amdgcn_s_waitcnt(pipe_wait_imm((UNR - 1) * L));
                land(u);
                pos(u, b0 + u);
                issue(b0 + u + UNR, u);
            }
        }
        static_for<0, UNR>([&](auto U) {
            constexpr int u = decltype(U)::value;
            __builtin_amdgcn_s_waitcnt(pipe_wait_imm((UNR - 1 - u) * L));
            land(u);
            if (b0 + u < cnt) pos(u, b0 + u);
        });
    }
};

template <int NG>
__device__ __forceinline__ void zero_acc(float (&acc)[NG][4][1]) {
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][r][0] = 0.f;
}

// A relaxed device-scope store: written through to the device's coherence point.
__device__ __forceinline__ void store_dev(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// This workgroup's hand-over stores are complete; one arrival at hand-over `hop`.
__device__ __forceinline__ void grid_arrive(uint32_t* sync, int hop) {
    __builtin_amdgcn_s_waitcnt(pipe_wait_imm(0));        // this wave's stores performed
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_fetch_add(sync + (hop * kSlots + (int)(blockIdx.x % kSlots)) * kSlotWords, 1u,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Until every workgroup of the grid has arrived at hand-over `hop` (bounded: a wait that runs
// out raises the flag and goes on). The first wave polls, one counter per lane.
__device__ __forceinline__ void grid_wait(uint32_t* sync, int hop) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        uint32_t* const slot = sync + (hop * kSlots + (lane & (kSlots - 1))) * kSlotWords;
        for (uint32_t polls = 0;; ++polls) {
            uint32_t v = lane < kSlots ? __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
#pragma unroll
            for (int m = 1; m < kSlots; m <<= 1) v += __shfl_xor(v, m);
            if (__builtin_amdgcn_readfirstlane(v) >= gridDim.x) break;
            if (polls >= kSpinLimit) {
                if (lane == 0) store_dev(sync + kFlagWord, 1u);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
}

// Zero hand-over hop's counters (lanes of the first wave, one counter each).
__device__ __forceinline__ void zero_hop(uint32_t* sync, int hop) {
    if (threadIdx.x < kSlots) store_dev(sync + (hop * kSlots + (int)threadIdx.x) * kSlotWords, 0u);
}

// Store the NG row groups' sums (rows n0[i] .. + 64) into y (thread t < 256 of lane group
// kg = 0 owns row 16 (t >> 6) + (t & 15) of a group; wave_sum's order).
// DEV: handed to the next phase (device-scope stores).
template <bool DEV, int NG>
__device__ __forceinline__ void store_rows(float (&acc)[NG][4][1], float (*red)[4][1][64], float* y,
                                           const int64_t (&n0)[NG]) {
    const int tid = threadIdx.x, lane = tid & 63;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        float v[1];
        wave_sum<1, kSegWaves>(acc[i], red, v);
        if (tid < 256 && (lane >> 4) == 0) {
            float* const p = y + n0[i] + (tid >> 6) * 16 + (lane & 15);
            if constexpr (DEV) store_dev(p, v[0]);
            else *p = v[0];
        }
        __syncthreads();
    }
}

// The row x = res + planes that seg_norm_row left in xf, stored by workgroup 0.
template <bool DEV>
__device__ __forceinline__ void store_row(const float* xf, float* dst, int n) {
    for (int i = threadIdx.x; i < n; i += kSegThreads) {
        if constexpr (DEV) store_dev(dst + i, xf[i]);
        else dst[i] = xf[i];
    }
}

// Copy n bf16 values from global memory into LDS.
__device__ __forceinline__ void stage_bf16(const uint16_t* __restrict__ src, int n, __bf16* xs) {
    uint16_t* d = (uint16_t*)xs;
    for (int i = threadIdx.x * 8; i < n; i += kSegThreads * 8) *(u32x4*)(d + i) = *(const u32x4*)(src + i);
    __syncthreads();
}

// What a norm prelude can load before its hand-over wait: res (thread t's elements t + 512 e,
// e < 8) and the norm weight (threads t < 256: elements t + 256 j, the ones it scales).
struct SegRowPre {
    static constexpr int E = kSegRow / kSegThreads;
    float r0[E];
    float wv[kAccRowJ];
};

template <int NW>
__device__ __forceinline__ void seg_row_pre(const float* __restrict__ res, const void* __restrict__ w, int K,
                                            SegRowPre& pre) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int e = 0; e < SegRowPre::E; ++e) pre.r0[e] = res[min(tid + kSegThreads * e, K - 1)];
    if (tid < 256) {                                  // waves 0-3: the scaling threads
#pragma unroll
        for (int j = 0; j < kAccRowJ; ++j) {
            const int i = min(tid + 256 * j, K - 1);
            pre.wv[j] = NW == 1 ? __uint_as_float((uint32_t)((const uint16_t*)w)[i] << 16) : ((const float*)w)[i];
        }
    }
}

// The row x = res + S partial planes (stride floats apart), its 1/rms and
// xs = bf16((x * r) * w) over [0, K), K <= kSegRow, with res and w from seg_row_pre:
// stage_norm_acc_row's arithmetic and order (gemv_core.h: planes added to 0 in split order and
// the sum to res; S = 1: res + part[0]; the fp64 sum of squares over i = tid + 256 j by the
// first 256 threads, the waves' sums as (w0 + w1) + (w2 + w3)). A thread's elements are
// tid + 512 e, e < 8; its plane loads go out together, four planes at a time (one trip to
// memory per four planes), so the registers of a primed weight pipeline stay live across it.
// x is left in xf.
__device__ __forceinline__ void seg_norm_row(const SegRowPre& pre, const float* __restrict__ part, int S,
                                             int64_t stride, int K, float eps, __bf16* xs, float* xf) {
    constexpr int E = SegRowPre::E, PB = 4;
    __shared__ double partd[4];
    const int tid = threadIdx.x;
    auto ix = [&](int e) { return min(tid + kSegThreads * e, K - 1); };   // loads stay in the row
    float v[E];
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = 0.f;
    if (S == 1) {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = pre.r0[e] + part[ix(e)];
    } else {
        for (int q = 0; q < S; q += PB) {
            float t[PB][E];
#pragma unroll
            for (int u = 0; u < PB; ++u)
#pragma unroll
                for (int e = 0; e < E; ++e) t[u][e] = part[(int64_t)min(q + u, S - 1) * stride + ix(e)];
#pragma unroll
            for (int u = 0; u < PB; ++u)
                if (q + u < S) {
#pragma unroll
                    for (int e = 0; e < E; ++e) v[e] += t[u][e];
                }
        }
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = S == 0 ? pre.r0[e] : pre.r0[e] + v[e];
    }
#pragma unroll
    for (int e = 0; e < E; ++e)
        if (tid + kSegThreads * e < K) xf[tid + kSegThreads * e] = v[e];
    __syncthreads();
    float x[kAccRowJ];
    if (tid < 256) {
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < kAccRowJ; ++j) {
            x[j] = tid + 256 * j < K ? xf[tid + 256 * j] : 0.f;
            if (tid + 256 * j < K) ss += (double)x[j] * (double)x[j];
        }
        const double wsum = wave_sum_ss(ss);
        if ((tid & 63) == 0) partd[tid >> 6] = wsum;
    }
    __syncthreads();
    if (tid < 256) {
        const float r = inv_rms(partd, K, eps);
#pragma unroll
        for (int j = 0; j < kAccRowJ; ++j) {
            const int i = tid + 256 * j;
            if (i < K) ((uint16_t*)xs)[i] = (uint16_t)f32_to_bf16_rne(x[j] * r * pre.wv[j]);
        }
    }
    __syncthreads();
}

__device__ __forceinline__ float seg_silu(float g) { return g / (1.0f + expf(-g)); }

// A workgroup with no item in a phase skips that phase's wait (its arrival still counts),
// so a phase's waiters see every workgroup's earlier outputs.
template <int QNG, int NW>
__global__ __launch_bounds__(kSegThreads) void decode_segment_kernel(SegParams P) {
    __shared__ float red[kSegWaves][4][1][64];
    __shared__ __attribute__((aligned(16))) __bf16 xs[kSegXs];
    __shared__ float xf[kSegRow];
    const int G = (int)gridDim.x, w = (int)blockIdx.x;
    const int KBh = P.H >> 5, KBf = P.F >> 5;
    const int64_t th = (int64_t)KBh * kTileBytes, tf = (int64_t)KBf * kTileBytes;   // bytes per row group
    // ---- 1. o: items (row group, split); the attention row is an input, no wait ----
    {
        const int items = (P.H >> 6) * P.So;
        for (int it = w; it < items; it += G) {
            const int g = it / P.So, sp = it % P.So;
            const uint8_t* const gb[1] = {P.o + g * th};
            SegStream<1, 4, true> st;
            st.xg = P.attn;
            st.setup(gb, sp * KBh / P.So, (sp + 1) * KBh / P.So);
            st.prime();
            float acc[1][4][1];
            zero_acc(acc);
            st.run(xs, 0, acc);
            const int64_t n0[1] = {(int64_t)sp * P.H + g * 64};
            store_rows<true>(acc, red, P.po, n0);
        }
    }
    // The previous call's hand-overs 1 and 2 (see the hand-over notes), zeroed after workgroup
    // 0's stream: a wave's stores count in its vmcnt, so stores ahead of a stream's first wait
    // would hold that wait for their acknowledgements. The arrival waits for them.
    if (w == 0) {
        zero_hop(P.sync, 1);
        zero_hop(P.sync, 2);
    }
    grid_arrive(P.sync, 0);

    // ---- 2. gate/up: items (row group of F) over all of K, x' = x + po normalised first ----
    {
        const int items = P.F >> 6;
        auto finish = [&](float (&acc)[2][4][1], int g) {
            float vg[1], vu[1];
            wave_sum<1, kSegWaves>(acc[0], red, vg);
            __syncthreads();
            wave_sum<1, kSegWaves>(acc[1], red, vu);
            // rows 16 r + i16 in lanes i16 < 16 of waves r < 4: an even lane stores its h and
            // its odd neighbour's as one 32-bit device-scope word
            const int tid = threadIdx.x, lane = tid & 63;
            const uint32_t hb = tid < 256 && lane < 16 ? f32_to_bf16_rne(seg_silu(vg[0]) * vu[0]) : 0u;
            const uint32_t odd = (uint32_t)__shfl_xor((int)hb, 1);
            if (tid < 256 && lane < 16 && (lane & 1) == 0)
                store_dev((uint32_t*)(P.h + (int64_t)g * 64 + (tid >> 6) * 16 + lane), hb | (odd << 16));
            __syncthreads();
        };
        if (w < items) {            // workgroup 0 always has an item: it writes x'
            SegStream<2, 4> st;
            const uint8_t* const gb[2] = {P.gate + w * th, P.up + w * th};
            st.setup(gb, 0, KBh);
            st.prime();                           // in flight across the hand-over
            SegRowPre pre;
            seg_row_pre<NW>(P.x, P.nw_post, P.H, pre);     // inputs of the call: no wait needed
            grid_wait(P.sync, 0);
            seg_norm_row(pre, P.po, P.So, P.H, P.H, P.eps, xs, xf);
            float acc[2][4][1];
            zero_acc(acc);
            st.run(xs, 0, acc);
            finish(acc, w);
            if (w == 0) store_row<true>(xf, P.xmid, P.H);   // after the stream (vmcnt), before arrival 1
            for (int it = w + G; it < items; it += G) {
                const uint8_t* const gb2[2] = {P.gate + it * th, P.up + it * th};
                SegStream<2, 4> s2;
                s2.setup(gb2, 0, KBh);
                s2.prime();
                zero_acc(acc);
                s2.run(xs, 0, acc);
                finish(acc, it);
            }
        } else {
            grid_wait(P.sync, 0);     // no arrival at hand-over 1 before hand-over 0 completes
        }
    }
    grid_arrive(P.sync, 1);

    // ---- 3. down: items (row group, split of F); h's K range staged per item ----
    {
        const int items = (P.H >> 6) * P.Sd;
        auto range = [&](int it, int& k0, int& k1) {
            const int sp = it % P.Sd;
            k0 = sp * KBf / P.Sd;
            k1 = (sp + 1) * KBf / P.Sd;
        };
        if (w < items) {
            int k0, k1;
            range(w, k0, k1);
            SegStream<1, 4> st;
            const uint8_t* const gb[1] = {P.down + (w / P.Sd) * tf};
            st.setup(gb, k0, k1);
            st.prime();                           // in flight across the hand-over
            grid_wait(P.sync, 1);
            stage_bf16(P.h + (int64_t)k0 * 32, (k1 - k0) * 32, xs);
            float acc[1][4][1];
            zero_acc(acc);
            st.run(xs, k0, acc);
            const int64_t n0[1] = {(int64_t)(w % P.Sd) * P.H + (w / P.Sd) * 64};
            store_rows<true>(acc, red, P.pd, n0);
            if (w == 0) zero_hop(P.sync, 0);      // every wait on hand-over 0 is over
            for (int it = w + G; it < items; it += G) {
                range(it, k0, k1);
                const uint8_t* const gb2[1] = {P.down + (it / P.Sd) * tf};
                SegStream<1, 4> s2;
                s2.setup(gb2, k0, k1);
                s2.prime();
                stage_bf16(P.h + (int64_t)k0 * 32, (k1 - k0) * 32, xs);
                zero_acc(acc);
                s2.run(xs, k0, acc);
                const int64_t n2[1] = {(int64_t)(it % P.Sd) * P.H + (it / P.Sd) * 64};
                store_rows<true>(acc, red, P.pd, n2);
            }
        } else if (P.qkv) {
            grid_wait(P.sync, 1);     // no arrival at hand-over 2 before hand-over 1 completes
        }
    }

    // ---- 4. the next layer's qkv: items (QNG row groups, split), x" = x' + pd normalised ----
    if (P.qkv) {
        grid_arrive(P.sync, 2);
        constexpr int QU = QNG >= 3 ? 2 : 4;
        const int items = (P.NQ >> 6) / QNG * P.Sq;
        auto item = [&](int it, const uint8_t* (&gb)[QNG], int64_t (&n0)[QNG], int& k0, int& k1) {
            const int grp = it / P.Sq, sp = it % P.Sq;
#pragma unroll
            for (int i = 0; i < QNG; ++i) {
                gb[i] = P.qkv + (int64_t)(grp * QNG + i) * th;
                n0[i] = (int64_t)sp * P.NQ + (int64_t)(grp * QNG + i) * 64;
            }
            k0 = sp * KBh / P.Sq;
            k1 = (sp + 1) * KBh / P.Sq;
        };
        if (w < items) {            // workgroup 0 always has an item: it writes x"
            const uint8_t* gb[QNG];
            int64_t n0[QNG];
            int k0, k1;
            item(w, gb, n0, k0, k1);
            SegStream<QNG, QU> st;
            st.setup(gb, k0, k1);
            st.prime();                           // in flight across the hand-over
            SegRowPre pre;
            seg_row_pre<NW>(P.xmid, P.nw_next, P.H, pre);  // x' is complete since hand-over 1
            grid_wait(P.sync, 2);
            seg_norm_row(pre, P.pd, P.Sd, P.H, P.H, P.eps, xs, xf);
            float acc[QNG][4][1];
            zero_acc(acc);
            st.run(xs, 0, acc);
            store_rows<false>(acc, red, P.pq, n0);
            if (w == 0) store_row<false>(xf, P.xnext, P.H);   // after the stream (vmcnt)
            for (int it = w + G; it < items; it += G) {
                item(it, gb, n0, k0, k1);
                SegStream<QNG, QU> s2;
                s2.setup(gb, k0, k1);
                s2.prime();
                zero_acc(acc);
                s2.run(xs, 0, acc);
                store_rows<false>(acc, red, P.pq, n0);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// host side

struct SegPlan {
    int G, So, Sd, Sq, QNG;
};

int seg_cus() {
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

// Workgroups: one per CU (Q4MI_SEGMENT_WGS lowers it, for tests of the item loops).
int seg_grid() {
    int g = seg_cus();
    if (const char* e = getenv("Q4MI_SEGMENT_WGS")) {
        const int v = atoi(e);
        if (v > 0 && v < g) g = v;
    }
    return g;
}

// Splits fill the grid with at most one item per workgroup where the shapes allow, each
// split keeping >= 8 K positions (one per wave); down's K range fits the LDS stage.
SegPlan seg_plan(int64_t H, int64_t F, int64_t NQ) {
    SegPlan p{seg_grid(), 1, 1, 1, 1};
    const int64_t KBh = H / 32, KBf = F / 32, Rh = H / 64;
    auto splits = [&](int64_t rows, int64_t kb) {
        return (int)std::max<int64_t>(1, std::min<int64_t>(p.G / std::max<int64_t>(rows, 1), kb / kSegWaves));
    };
    p.So = splits(Rh, KBh);
    p.Sd = std::max(splits(Rh, KBf), (int)ceil_div(KBf, kSegXs / 32));
    if (NQ > 0) {
        int64_t best = -1;
        for (int ng = 1; ng <= 4; ++ng) {
            const int64_t R = NQ / 64;
            if (R % ng) continue;
            const int s = splits(R / ng, KBh);
            const int64_t items = std::min<int64_t>((R / ng) * s, p.G);
            if (items >= best) best = items, p.QNG = ng, p.Sq = s;
        }
    }
    return p;
}

size_t seg_ws_bytes(int64_t H, int64_t F, const SegPlan& p) {
    return kSyncBytes + (size_t)p.So * H * 4 + (size_t)ceil_div(F * 2, 256) * 256;
}

bool seg_shape_ok(int64_t H, int64_t F, int64_t NQ) {
    return H > 0 && F > 0 && NQ >= 0 && H % 64 == 0 && F % 64 == 0 && NQ % 64 == 0 && H <= kSegRow &&
           H / 32 >= kSegWaves && F / 32 >= kSegWaves;
}

template <int QNG, int NW>
int seg_launch(const SegPlan& p, const SegParams& P, hipStream_t st) {
    auto kern = decode_segment_kernel<QNG, NW>;
    static const int per_cu = [&] {      // workgroups the runtime can keep resident per CU
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, kSegThreads, 0) != hipSuccess) {
            (void)hipGetLastError();
            return 0;
        }
        return n;
    }();
    if (per_cu < 1 || p.G > per_cu * seg_cus()) return Q4MI_E_LAUNCH;   // the grid must be resident
    hipLaunchKernelGGL(kern, dim3((unsigned)p.G), dim3(kSegThreads), 0, st, P);
    return launch_status();
}

}  // namespace

extern "C" int q4_decode_segment_splits(int64_t H, int64_t F, int64_t NQ, int* splits) {
    if (!splits) return Q4MI_E_ARG;
    if (!seg_shape_ok(H, F, NQ)) return Q4MI_E_SHAPE;
    const SegPlan p = seg_plan(H, F, NQ);
    splits[0] = p.So;
    splits[1] = p.Sd;
    splits[2] = NQ > 0 ? p.Sq : 0;
    return Q4MI_OK;
}

extern "C" size_t q4_decode_segment_workspace_bytes(int64_t H, int64_t F, int64_t NQ) {
    if (!seg_shape_ok(H, F, NQ)) return 0;
    return seg_ws_bytes(H, F, seg_plan(H, F, NQ));
}

extern "C" int q4_decode_segment(const uint8_t* o, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                                 const uint8_t* qkv, const void* attn, const float* x, const void* nw_post,
                                 const void* nw_next, int nw_dtype, float eps, float* x_mid, float* x_next,
                                 float* down_planes, float* qkv_planes, int64_t H, int64_t F, int64_t NQ,
                                 void* workspace, size_t workspace_bytes, void* stream) {
    if (!qkv) NQ = 0;
    if (!seg_shape_ok(H, F, NQ) || (qkv && NQ == 0)) return Q4MI_E_SHAPE;
    if (nw_dtype != Q4MI_F32 && nw_dtype != Q4MI_BF16) return Q4MI_E_ARG;
    if (!o || !gate || !up || !down || !attn || !x || !nw_post || !x_mid || !down_planes || !workspace)
        return Q4MI_E_ARG;
    if (qkv && (!nw_next || !x_next || !qkv_planes)) return Q4MI_E_ARG;
    for (const void* p : {(const void*)o, (const void*)gate, (const void*)up, (const void*)down, (const void*)qkv,
                          attn, (const void*)x, nw_post, nw_next, (const void*)x_mid, (const void*)x_next,
                          (const void*)down_planes, (const void*)qkv_planes, (const void*)workspace})
        if (misaligned16(p)) return Q4MI_E_ARG;
    const SegPlan p = seg_plan(H, F, NQ);
    const size_t ws = seg_ws_bytes(H, F, p);
    if (workspace_bytes < ws) return Q4MI_E_WORKSPACE;
    // x" is written while every workgroup reads x' and the planes: x_next must not overlap
    // them (it may be x, read only before the second barrier); no output may overlap the
    // workspace or another output
    const int64_t row = H * 4;
    const int64_t pd_b = (int64_t)p.Sd * row, pq_b = qkv ? (int64_t)p.Sq * NQ * 4 : 0;
    if (overlaps(x_mid, row, x, row) || overlaps(x_mid, row, down_planes, pd_b) ||
        overlaps(x_mid, row, qkv_planes, pq_b) || overlaps(down_planes, pd_b, qkv_planes, pq_b) ||
        overlaps(workspace, (int64_t)ws, x, row) || overlaps(workspace, (int64_t)ws, x_mid, row) ||
        overlaps(workspace, (int64_t)ws, down_planes, pd_b) || overlaps(workspace, (int64_t)ws, qkv_planes, pq_b) ||
        overlaps(workspace, (int64_t)ws, attn, H * 2))
        return Q4MI_E_ARG;
    if (qkv && (overlaps(x_next, row, x_mid, row) || overlaps(x_next, row, down_planes, pd_b) ||
                overlaps(x_next, row, qkv_planes, pq_b) || overlaps(workspace, (int64_t)ws, x_next, row)))
        return Q4MI_E_ARG;
    SegParams P{};
    P.o = o;
    P.gate = gate;
    P.up = up;
    P.down = down;
    P.qkv = qkv;
    P.attn = (const uint16_t*)attn;
    P.x = x;
    P.xmid = x_mid;
    P.xnext = qkv ? x_next : nullptr;
    P.nw_post = nw_post;
    P.nw_next = nw_next;
    P.eps = eps;
    uint8_t* wsb = (uint8_t*)workspace;
    P.sync = (uint32_t*)wsb;
    P.po = (float*)(wsb + kSyncBytes);
    P.h = (uint16_t*)(wsb + kSyncBytes + (size_t)p.So * H * 4);
    P.pd = down_planes;
    P.pq = qkv_planes;
    P.H = (int)H;
    P.F = (int)F;
    P.NQ = (int)NQ;
    P.So = p.So;
    P.Sd = p.Sd;
    P.Sq = p.Sq;
    const hipStream_t st = (hipStream_t)stream;
    const bool bw = nw_dtype == Q4MI_BF16;
    switch (p.QNG) {
        case 1: return bw ? seg_launch<1, 1>(p, P, st) : seg_launch<1, 2>(p, P, st);
        case 2: return bw ? seg_launch<2, 1>(p, P, st) : seg_launch<2, 2>(p, P, st);
        case 3: return bw ? seg_launch<3, 1>(p, P, st) : seg_launch<3, 2>(p, P, st);
        default: return bw ? seg_launch<4, 1>(p, P, st) : seg_launch<4, 2>(p, P, st);
    }
}
