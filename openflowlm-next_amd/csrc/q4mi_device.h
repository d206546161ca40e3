// q4mi_device.h -- device helpers shared by the gfx950 Q4_1 kernels.
//
// The mx weight layout (an [N, K] matrix, N % 64 == 0, K % 32 == 0):
//   tile (g, kb) = 64 rows x 32 K, 1280 B, at byte (g * K/32 + kb) * 1280.
//   codes  [0, 1024): dword (lane, r) at lane*16 + r*4 (lane 0..63, r 0..3)
//            row n = 64 g + 16 r + lane % 16, k = 32 kb + 8 (lane / 16) + e,
//            code e (0..7) at bit 16 * (e & 1) + 4 * (e >> 1).
//   scales [1024, 1280): dword at 1024 + (lane % 16)*16 + r*4 for the same
//            row: (bf16 d << 16) | bf16 m.
// One codes dword is the B operand of a v_mfma_f32_16x16x32_bf16 for the
// eight k of row lane%16 in k-group lane/16: codes_to_bf16 turns it into
// eight bf16 values 128 + q with two ALU ops per pair (mask, or a magic
// exponent) and the MFMA folds the 128 offset back out through its C input.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q4mi {

// The native Q4_K ("mxk") layout of an [N, K] matrix (N % 64 == 0, K % 256 == 0): tile
// (g, sb) = 64 rows x 256 K (one Q4_K super-block per row), 9728 B, at byte
// (g * K/256 + sb) * 9728:
//   codes [0, 8192): sub-block j (32 K) at j * 1024, laid out as the mx codes above;
//   sc/mn [8192, 9216): row 16 r + i16 at 8192 + i16 * 64 + r * 16: the 8-bit integer
//         multipliers sc[0..7] of its 8 sub-blocks, then mn[0..7];
//   d     [9216, 9472): f32 at 9216 + i16 * 16 + r * 4;  m [9472, 9728): same order.
// Weight = fl32(d sc q + m mn): d sc and m mn are exact in f32 (<= 11-bit x 8-bit
// significands), so a block reads as Q4_1 with scale d sc and offset m mn, exactly.
constexpr int kKTileBytes = 9728;
constexpr int kKScOff = 8192, kKDOff = 9216, kKMOff = 9472;

// The native q8 ("mx8") layout of an [N, K] matrix (N % 64 == 0, K % 32 == 0): tile
// (g, kb) = 64 rows x 32 K, 2176 B, at byte (g * K/32 + kb) * 2176:
//   codes [0, 2048): lane (kg * 16 + i16) holds at (r / 2) * 1024 + lane * 16 + (r % 2) * 8
//         the 8 codes of row 16 r + i16 at k = 32 kb + 8 kg + 0..7 as unsigned bytes
//         b = q + 128, each dword in the order (k0, k2, k1, k3) so that masking nibble
//         pairs out of it yields consecutive k (one 16-byte load per lane covers rows r and
//         r + 1 and a wave's load is 1 KB contiguous);
//   scale [2048, 2176): bf16 s of row 16 r + i16 at 2048 + i16 * 8 + r * 2.
// Weight = s * q, exact in f32 (8-bit x 8-bit). 1.0625 bytes per weight, as GGUF Q8_0.
constexpr int kQ8TileBytes = 2176;
constexpr int kQ8ScaleOff = 2048;

// The Q4_0-native ("mx0") layout of an [N, K] matrix (N % 64 == 0, K % 32 == 0): tile
// (g, kb) = 64 rows x 32 K, 1152 B, at byte (g * K/32 + kb) * 1152:
//   codes [0, 1024): as the mx layout;
//   d     [1024, 1152): bf16 d of row 16 r + i16 at 1024 + i16 * 8 + r * 2.
// Q4_0 stores no min: weight = fl32(q d + m) with m = -8 d, exact in bf16 and f32, so the
// values equal the mx layout's for the same blocks at 0.5625 B per weight against 0.625
// (the reference's 4608 B Q4_0-native chunk, open_kernels/q4_1_pack.py:145-152, read by
// designs/gemv_q4/gemv_q4.h:66-82 with m = -8 d).
constexpr int kQ0TileBytes = 1152;

constexpr int kRows = 64;        // rows per tile / row group
constexpr int kBlk = 32;         // K per tile (one GGUF block)
constexpr int kTileBytes = 1280;
constexpr int kCodeBytes = 1024;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// bf16 128.0 in both halves: OR-ing a code q (0..15) into the low mantissa
// bits gives exactly the bf16 value 128 + q (exponent 2^7, unit mantissa step 1).
constexpr uint32_t kMagic128 = 0x43004300u;
constexpr uint32_t kNib2 = 0x000F000Fu;

// A constant held in a VGPR the optimizer cannot see through. gfx9 VOP3
// encodings take no literal and read at most one SGPR, so v_and_or_b32 with
// the mask and the magic needs both in VGPRs; hoisted out of loops by the
// caller, this keeps the conversion at one op per pair (plus a shift).
__device__ __forceinline__ uint32_t vgpr_const(uint32_t c) {
    uint32_t v;
    asm("v_mov_b32 %0, %1" : "=v"(v) : "s"(c));
    return v;
}

struct CodeConsts {
    uint32_t nib2, magic;
};
__device__ __forceinline__ CodeConsts code_consts() { return {vgpr_const(kNib2), vgpr_const(kMagic128)}; }

__device__ __forceinline__ bf16x8 codes_to_bf16(uint32_t w, CodeConsts k) {
    u32x4 v;
    v[0] = (w & k.nib2) | k.magic;
    v[1] = ((w >> 4) & k.nib2) | k.magic;
    v[2] = ((w >> 8) & k.nib2) | k.magic;
    v[3] = ((w >> 12) & k.nib2) | k.magic;
    return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ float bf16_hi_to_f32(uint32_t s) {   // d from a scale word
    return __builtin_bit_cast(float, s & 0xFFFF0000u);
}
__device__ __forceinline__ float bf16_lo_to_f32(uint32_t s) {   // m from a scale word
    return __builtin_bit_cast(float, s << 16);
}

// f32 -> bf16 bits, round to nearest even (finite inputs).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// fp16 bits -> f32 (exact).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// The scale word's d and m as f32: bf16 halves (the mx layout's default, the reference
// pool's narrowing) or, with F16S, GGUF's own fp16 d and m kept exactly (q4_repack
// scale_mode 1). Either converts exactly.
template <bool F16S>
__device__ __forceinline__ float scale_d(uint32_t s) {
    if constexpr (F16S) return f16_bits_to_f32(s >> 16);
    else return bf16_hi_to_f32(s);
}
template <bool F16S>
__device__ __forceinline__ float scale_m(uint32_t s) {
    if constexpr (F16S) return f16_bits_to_f32(s & 0xFFFFu);
    else return bf16_lo_to_f32(s);
}

// Device buffers are global memory. Loads through these address-space-1 pointers are
// global_load instructions whatever the pointer's origin: a pointer read from memory (a
// descriptor table) is otherwise a flat pointer, and flat loads count on lgkmcnt too, so
// their waits cannot leave younger loads in flight.
template <class T>
using global_ptr = const __attribute__((address_space(1))) T*;

template <class T>
__device__ __forceinline__ T load_global(const void* p) {
    return *(global_ptr<T>)p;
}

// Streaming loads of weight bytes: read once, keep them out of the caches'
// way (the "nt" bit on the global load).
__device__ __forceinline__ u32x4 load_nt_u32x4(const void* p) {
    return __builtin_nontemporal_load((global_ptr<u32x4>)p);
}
__device__ __forceinline__ u32x2 load_nt_u32x2(const void* p) {
    return __builtin_nontemporal_load((global_ptr<u32x2>)p);
}
__device__ __forceinline__ uint32_t load_nt_u32(const void* p) {
    return __builtin_nontemporal_load((global_ptr<uint32_t>)p);
}

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

}  // namespace q4mi
