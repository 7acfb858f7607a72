// common.hpp — device helpers shared by the gfx950 kernels of the paged
// KV-cache path: 16-byte vector types, wave64 cross-lane reductions, fp16 and
// OCP e4m3fn conversions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace vkv {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
// Threads per workgroup of the fixed-size launches (append, RoPE + append,
// decode partitions, prefill row map).  Those kernels use this constant, not
// blockDim.x: HIP reads blockDim.x from the dispatch's hidden arguments with
// two dependent memory loads (block count, then group size), which every
// workgroup would await before its first load of real data.
constexpr int kBlockThreads = 256;

enum KvType : int { kF32 = 0, kF16 = 1, kFp8 = 2 };

template <int KVT>
struct KvTraits;
template <>
struct KvTraits<kF32> { static constexpr int bytes = 4; };
template <>
struct KvTraits<kF16> { static constexpr int bytes = 2; };
template <>
struct KvTraits<kFp8> { static constexpr int bytes = 1; };

// Bit casts between 32-bit lanes and float always go through these by-value
// helpers.  clang (ROCm 7.2) lowers __builtin_bit_cast applied directly to an
// element of an ext_vector_type value as a read of element 0 for every index
// (one dword load feeding all four uses), so that form is never used here.
__device__ __forceinline__ float as_f32(uint32_t w) { return __builtin_bit_cast(float, w); }
__device__ __forceinline__ uint32_t as_u32(float x) { return __builtin_bit_cast(uint32_t, x); }

__device__ __forceinline__ u32x4 load16(const void* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ void store16(void* p, u32x4 v) {
    *reinterpret_cast<u32x4*>(p) = v;
}

__device__ __forceinline__ u32x4 load16_nt(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ void store16_nt(void* p, u32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// ---------------------------------------------------------------- lanes

// DPP controls (GFX9 encoding): quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror.  Applied in this order each one pairs every
// lane with a lane of the other half of a 2-, 4-, 8- and 16-lane group, so
// adding the moved value after each step leaves the group sum in every lane.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL,
                                                                0xF, 0xF, true));
}

// x combined with the value of lane l ^ O.  O = 16 and 32 use gfx950's
// permlane swaps on the VALU (16-lane rows, or wave halves, change places;
// swapping a value with itself leaves the two partners' values, one in each
// result), other distances an LDS permute.  Both operations are commutative,
// so every lane gets the same bits whichever result holds its own value.
template <int O>
__device__ __forceinline__ float xor_add(float x) {
    if constexpr (O == 16 || O == 32) {
        const auto a = O == 16 ? __builtin_amdgcn_permlane16_swap(as_u32(x), as_u32(x), false, false)
                               : __builtin_amdgcn_permlane32_swap(as_u32(x), as_u32(x), false, false);
        return as_f32(a[0]) + as_f32(a[1]);
    } else {
        return x + __shfl_xor(x, O, 64);
    }
}
template <int O>
__device__ __forceinline__ float xor_max(float x) {
    if constexpr (O == 16 || O == 32) {
        const auto a = O == 16 ? __builtin_amdgcn_permlane16_swap(as_u32(x), as_u32(x), false, false)
                               : __builtin_amdgcn_permlane32_swap(as_u32(x), as_u32(x), false, false);
        return fmaxf(as_f32(a[0]), as_f32(a[1]));
    } else {
        return fmaxf(x, __shfl_xor(x, O, 64));
    }
}

// Sum over aligned groups of N lanes (N a power of two <= 64); every lane of a
// group receives the group sum.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (N >= 2) x += dpp_mov<0xB1>(x);
    if constexpr (N >= 4) x += dpp_mov<0x4E>(x);
    if constexpr (N >= 8) x += dpp_mov<0x141>(x);
    if constexpr (N >= 16) x += dpp_mov<0x140>(x);
    if constexpr (N >= 32) x = xor_add<16>(x);
    if constexpr (N >= 64) x = xor_add<32>(x);
    return x;
}

template <int N>
__device__ __forceinline__ float group_max(float x) {
    if constexpr (N >= 2) x = fmaxf(x, dpp_mov<0xB1>(x));
    if constexpr (N >= 4) x = fmaxf(x, dpp_mov<0x4E>(x));
    if constexpr (N >= 8) x = fmaxf(x, dpp_mov<0x141>(x));
    if constexpr (N >= 16) x = fmaxf(x, dpp_mov<0x140>(x));
    if constexpr (N >= 32) x = xor_max<16>(x);
    if constexpr (N >= 64) x = xor_max<32>(x);
    return x;
}

// Inclusive prefix sum of v over the wave's 64 lanes in lane order, in
// registers (no LDS round trip per step): a Hillis-Steele scan inside each
// 16-lane row by DPP row_shr:1, 2, 4, 8 (lanes shifted in from outside the row
// read 0), then row_bcast:15 adds lane 15 of rows 0 and 2 into rows 1 and 3,
// and row_bcast:31 adds lane 31 (the total of rows 0-1) into rows 2 and 3.
// Lane 63 ends with the wave total.
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
    return v;
}

// Sum over lanes that share (lane % STRIDE), i.e. across the 64/STRIDE groups
// of STRIDE consecutive lanes.  STRIDE is a power of two.
template <int STRIDE>
__device__ __forceinline__ float cross_group_sum(float x) {
    if constexpr (STRIDE < kWave) return cross_group_sum<2 * STRIDE>(xor_add<STRIDE>(x));
    else return x;
}

template <int STRIDE>
__device__ __forceinline__ float cross_group_max(float x) {
    if constexpr (STRIDE < kWave) return cross_group_max<2 * STRIDE>(xor_max<STRIDE>(x));
    else return x;
}

// Orders this wave's earlier LDS writes before its later LDS reads of other
// lanes' data (one wave, no workgroup barrier).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------- fp16

__device__ __forceinline__ half2_t as_half2(uint32_t w) { return __builtin_bit_cast(half2_t, w); }

__device__ __forceinline__ float dot2(half2_t a, half2_t b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// ---------------------------------------------------------------- fp8 e4m3fn

// Four e4m3fn codes (bytes b0..b3 of w) re-expressed exactly as fp16 values
// scaled by 2^-8: the e4m3 sign/exponent/mantissa fields placed in the fp16
// fields read the exponent with bias 15 instead of 7, a factor 2^-8 for
// normal and subnormal codes alike.  Returns lo = (b0, b2), hi = (b1, b3).
// The NaN code 0x7F is never produced by the encoder below and is not handled.
__device__ __forceinline__ void fp8x4_to_half2x2_scaled(uint32_t w, uint32_t& lo, uint32_t& hi) {
    const uint32_t a = w & 0x00FF00FFu;
    const uint32_t b = (w >> 8) & 0x00FF00FFu;
    lo = ((a & 0x00800080u) << 8) | ((a & 0x007F007Fu) << 7);
    hi = ((b & 0x00800080u) << 8) | ((b & 0x007F007Fu) << 7);
}

constexpr float kFp8HalfScale = 256.0f;  // undoes the 2^-8 of the re-expression above

// Two e4m3fn codes (bits 0-15 of w, or bits 16-31 with HI) as their exact fp16
// values, element 0 from the lower byte: gfx950's v_cvt_scalef32_pk_f16_fp8
// with scale 1 (every finite e4m3fn value is an fp16 value).
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_half2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
}

// fp32 -> e4m3fn, round to nearest even, saturating: |x| beyond 448 (and inf)
// encode as 448, NaN as 0x7F with the sign of x.
__device__ __forceinline__ uint32_t f32_to_fp8_sat(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7FFFFFFFu;
    uint32_t code;
    if (a > 0x7F800000u) {
        code = 0x7Fu;
    } else if (a > 0x43E00000u) {  // > 448.0f
        code = 0x7Eu;
    } else if (a < 0x3C800000u) {  // < 2^-6: subnormal grid m * 2^-9, m in 0..8
        const float m = __builtin_rintf(__builtin_bit_cast(float, a) * 512.0f);
        code = static_cast<uint32_t>(m);  // 8 becomes 0x08 = 2^-6, the smallest normal
    } else {
        const uint32_t lsb = (a >> 20) & 1u;
        const uint32_t r = a + 0x7FFFFu + lsb;  // round the 23-bit mantissa to 3 bits, ties to even
        code = (r >> 20) - (120u << 3);         // rebias exponent 127 -> 7
    }
    return sign | code;
}

// Per-(token, head) FP8 scale rule: amax / 448 in IEEE fp32, 1 for amax == 0.
__device__ __forceinline__ float fp8_scale_from_amax(float amax) {
    return amax == 0.0f ? 1.0f : amax / 448.0f;
}

// Attention logit scale in the log2 domain (scale * log2 e), as the decode
// and prefill kernels take it.  A scale of magnitude below 2^-100 (zero
// included) runs as +-2^-100: the reference then weights every key
// e^(dot * 0 - 0) = 1, i.e. returns the mean of V (src/attention/
// paged_attention.cu:47-51,75 with m0 = -1e30), and exp2((dot - max) * 2^-100)
// rounds to exactly 1 for |dot - max| < 2^75, while the kernels' -inf running-
// max start and masked keys still weigh 0 instead of -inf * 0 = NaN.
inline float logit_scale_log2(float scale) {
    constexpr float kMinLog2Scale = 0x1p-100f;
    const float s = scale * 1.4426950408889634f;
    if (s < kMinLog2Scale && s > -kMinLog2Scale) return s < 0.0f ? -kMinLog2Scale : kMinLog2Scale;
    return s;  // NaN stays NaN, as in the reference
}

}  // namespace vkv
