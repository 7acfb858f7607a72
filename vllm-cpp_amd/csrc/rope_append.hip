// rope_append.hip — rotary position embedding fused with the KV append (gfx950).
//
// The reference rotates q and k in place (rope_kernel, src/kernels/rotary_embedding.cu:8-35,
// one thread per (token, head, dim pair)) and then copies the rotated k and v
// rows into the cache with two cudaMemcpyAsync calls per token
// (src/layers/attention.cpp:79-102).  Here one launch reads q, k and v once:
// q is rotated in place, the rotated k and the plain v go straight into their
// cache slots (k's source buffer is not written back).  With no cache
// (key_cache == NULL) the kernel is the reference's rope_forward: q and k are
// both rotated in place.
//
// Rotation (the reference's pairing, dims d and d + D/2 with the interleaved
// [pos][D/2][cos, sin] table of src/model/qwen.cpp:119-128):
//   x[d]       <- fma(x[d], cos, -(x[d+D/2] * sin))
//   x[d+D/2]   <- fma(x[d], sin,   x[d+D/2] * cos)
// in fp32, then rounded to the source type, so the fused op equals the
// unfused rope followed by vkv_reshape_and_cache bit for bit.
//
// Work item = one lane per (token, head, group of 8 dim pairs): the lane loads
// 8 elements at d0 = 8c and 8 at D/2 + d0 (16-byte loads for fp16) plus its 16
// table floats (64 contiguous bytes); a head is LPH = D/16 consecutive lanes,
// so the FP8 per-(token, kv head) amax is a DPP reduction over those lanes.
// Heads of a token are ordered q (H), k (Hkv), v (Hkv).
#include "common.hpp"
#include "launch.hpp"

namespace vkv {
namespace {

constexpr int kRopeOnly = -1;

typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));

struct RopeArgs {
    char* q;
    char* k;
    const char* v;
    int64_t q_stride_bytes;
    int64_t k_stride_bytes;
    int64_t v_stride_bytes;
    const float* cos_sin;
    const int32_t* positions;
    int32_t start_pos;
    int32_t max_position;
    char* key_cache;
    char* value_cache;
    float* key_scales;
    float* value_scales;
    const int32_t* slot_mapping;
    int64_t row_bytes;   // cache bytes of one slot (all kv heads)
    int64_t num_slots;
    int64_t total;       // lanes
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t heads_per_token;  // H + Hkv (+ Hkv with a cache)
};

template <typename SRC>
__device__ __forceinline__ void load8(const char* p, float (&x)[8]) {
    if constexpr (sizeof(SRC) == 2) {
        const u32x4 w = load16_nt(p);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[2 * e] = f16_bits_to_f32(uint16_t(w[e] & 0xFFFFu));
            x[2 * e + 1] = f16_bits_to_f32(uint16_t(w[e] >> 16));
        }
    } else {
        const u32x4 a = load16_nt(p), b = load16_nt(p + 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[e] = as_f32(a[e]);
            x[4 + e] = as_f32(b[e]);
        }
    }
}

// Rounds to SRC and returns the rounded values as fp32 (for the cache path).
// The empty asm pins each fp32 result in a register first: otherwise the
// compiler folds fma + fp32->fp16 into one v_fma_mixlo_f16, which rounds the
// exact product sum once to fp16 instead of to fp32 and then to fp16 (the two
// differ on fp16 rounding ties).
template <typename SRC>
__device__ __forceinline__ void round_to(float (&x)[8]) {
    if constexpr (sizeof(SRC) == 2) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float r = x[e];
            asm volatile("" : "+v"(r));
            x[e] = static_cast<float>(static_cast<_Float16>(r));
        }
    }
}

template <int EB>
__device__ __forceinline__ void store8(char* p, const float (&x)[8]) {
    if constexpr (EB == 2) {
        u32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            w[e] = uint32_t(f32_to_f16_bits(x[2 * e])) | (uint32_t(f32_to_f16_bits(x[2 * e + 1])) << 16);
        store16_nt(p, w);
    } else {
        store16_nt(p, u32x4{as_u32(x[0]), as_u32(x[1]), as_u32(x[2]), as_u32(x[3])});
        store16_nt(p + 16, u32x4{as_u32(x[4]), as_u32(x[5]), as_u32(x[6]), as_u32(x[7])});
    }
}

template <typename SRC, int CT, int LPH>
__global__ __launch_bounds__(kBlockThreads) void rope_append_kernel(RopeArgs a) {
    constexpr int D = LPH * 16;
    constexpr int HALF = D / 2;
    constexpr int SEB = int(sizeof(SRC));
    const int64_t stride = int64_t(gridDim.x) * kBlockThreads;
    const int64_t per_token = int64_t(a.heads_per_token) * LPH;
    for (int64_t i = int64_t(blockIdx.x) * kBlockThreads + threadIdx.x; i < a.total; i += stride) {
        const int64_t t = i / per_token;
        const int u = int(i - t * per_token);
        const int head = u / LPH;
        const int d0 = 8 * (u % LPH);
        // kind 0 = query head, 1 = key head, 2 = value head (uniform over a head's lanes)
        const int kind = head < a.num_heads ? 0 : (head < a.num_heads + a.num_kv_heads ? 1 : 2);
        const int hh = kind == 0 ? head : (kind == 1 ? head - a.num_heads : head - a.num_heads - a.num_kv_heads);
        // The slot id, the source row and the position are read together
        // (the slot check waits for all three, not the loads for the check).
        int64_t slot = -1;
        if constexpr (CT != kRopeOnly)
            if (kind != 0) slot = a.slot_mapping[t];
        char* src = kind == 0 ? a.q + t * a.q_stride_bytes
                              : (kind == 1 ? a.k + t * a.k_stride_bytes
                                           : const_cast<char*>(a.v) + t * a.v_stride_bytes);
        src += int64_t(hh) * D * SEB;
        float x0[8], x1[8];
        load8<SRC>(src + d0 * SEB, x0);
        load8<SRC>(src + (HALF + d0) * SEB, x1);
        const int pos_in = a.positions ? a.positions[t] : a.start_pos + int(t);
        if constexpr (CT != kRopeOnly)
            if (kind != 0 && (slot < 0 || slot >= a.num_slots)) continue;  // padding token: nothing to store
        if (kind != 2) {
            int pos = pos_in;
            pos = pos < 0 ? 0 : (pos >= a.max_position ? a.max_position - 1 : pos);
            const float* tb = a.cos_sin + int64_t(pos) * D + 2 * d0;
            const u32x4 c0 = load16(tb), c1 = load16(tb + 4), c2 = load16(tb + 8), c3 = load16(tb + 12);
            const uint32_t cs[16] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3],
                                     c2[0], c2[1], c2[2], c2[3], c3[0], c3[1], c3[2], c3[3]};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float c = as_f32(cs[2 * e]), s = as_f32(cs[2 * e + 1]);
                const float a0 = x0[e], a1 = x1[e];
                x0[e] = __builtin_fmaf(a0, c, -(a1 * s));
                x1[e] = __builtin_fmaf(a0, s, a1 * c);
            }
            round_to<SRC>(x0);
            round_to<SRC>(x1);
        }
        if (kind == 0 || CT == kRopeOnly) {  // rotated in place
            store8<SEB>(src + d0 * SEB, x0);
            store8<SEB>(src + (HALF + d0) * SEB, x1);
            continue;
        }
        if constexpr (CT != kRopeOnly) {
            constexpr int CEB = KvTraits<CT>::bytes;
            char* row = (kind == 1 ? a.key_cache : a.value_cache) + slot * a.row_bytes + int64_t(hh) * D * CEB;
            if constexpr (CT == kFp8) {
                float amax = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fmaxf(fabsf(x0[e]), fabsf(x1[e])));
                amax = group_max<LPH>(amax);
                const float scale = fp8_scale_from_amax(amax);
                u32x2v q0, q1;
#pragma unroll
                for (int w = 0; w < 2; ++w) {
                    uint32_t p0 = 0, p1 = 0;
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        p0 |= f32_to_fp8_sat(x0[4 * w + b] / scale) << (8 * b);
                        p1 |= f32_to_fp8_sat(x1[4 * w + b] / scale) << (8 * b);
                    }
                    q0[w] = p0;
                    q1[w] = p1;
                }
                *reinterpret_cast<u32x2v*>(row + d0) = q0;
                *reinterpret_cast<u32x2v*>(row + HALF + d0) = q1;
                if (d0 == 0) (kind == 1 ? a.key_scales : a.value_scales)[slot * a.num_kv_heads + hh] = scale;
            } else {
                store8<CEB>(row + d0 * CEB, x0);
                store8<CEB>(row + (HALF + d0) * CEB, x1);
            }
        }
    }
}

int rope_grid(int64_t total) {
    int64_t blocks = (total + 255) / 256;
    const int64_t cap = int64_t(256) * 64;
    if (blocks > cap) blocks = cap;
    return int(blocks < 1 ? 1 : blocks);
}

template <typename SRC, int CT>
int launch_rope_t(const RopeArgs& a, int lph, hipStream_t st) {
    const int g = rope_grid(a.total);
    switch (lph) {
        case 4: hipLaunchKernelGGL((rope_append_kernel<SRC, CT, 4>), dim3(g), dim3(kBlockThreads), 0, st, a); break;
        case 8: hipLaunchKernelGGL((rope_append_kernel<SRC, CT, 8>), dim3(g), dim3(kBlockThreads), 0, st, a); break;
        case 16: hipLaunchKernelGGL((rope_append_kernel<SRC, CT, 16>), dim3(g), dim3(kBlockThreads), 0, st, a); break;
        default: return -1;
    }
    return 0;
}

}  // namespace

int launch_rope_append(const vkv_rope_append_params* p, hipStream_t st) {
    const bool f32 = p->src_dtype == VKV_DTYPE_F32;
    const int seb = f32 ? 4 : 2;
    const bool rope_only = p->key_cache == nullptr;
    const int ceb = p->cache_dtype == VKV_DTYPE_F32 ? 4 : (p->cache_dtype == VKV_DTYPE_F16 ? 2 : 1);
    const int64_t src_row = int64_t(p->num_kv_heads) * p->head_dim;
    RopeArgs a;
    a.q = static_cast<char*>(p->query);
    a.k = static_cast<char*>(p->key);
    a.v = static_cast<const char*>(p->value);
    a.q_stride_bytes = (p->query_stride ? p->query_stride : int64_t(p->num_heads) * p->head_dim) * seb;
    a.k_stride_bytes = (p->key_stride ? p->key_stride : src_row) * seb;
    a.v_stride_bytes = (p->value_stride ? p->value_stride : src_row) * seb;
    a.cos_sin = p->cos_sin;
    a.positions = p->positions;
    a.start_pos = p->start_pos;
    a.max_position = p->max_position;
    a.key_cache = static_cast<char*>(p->key_cache);
    a.value_cache = static_cast<char*>(p->value_cache);
    a.key_scales = p->key_scales;
    a.value_scales = p->value_scales;
    a.slot_mapping = p->slot_mapping;
    a.row_bytes = src_row * ceb;
    a.num_slots = int64_t(p->num_blocks) * p->block_size;
    a.num_heads = p->num_heads;
    a.num_kv_heads = p->num_kv_heads;
    a.heads_per_token = p->num_heads + p->num_kv_heads * (rope_only ? 1 : 2);
    const int lph = p->head_dim / 16;
    a.total = int64_t(p->num_tokens) * a.heads_per_token * lph;
    if (rope_only) return f32 ? launch_rope_t<float, kRopeOnly>(a, lph, st) : launch_rope_t<_Float16, kRopeOnly>(a, lph, st);
    switch (p->cache_dtype) {
        case VKV_DTYPE_F32: return f32 ? launch_rope_t<float, kF32>(a, lph, st) : -1;
        case VKV_DTYPE_F16: return f32 ? launch_rope_t<float, kF16>(a, lph, st) : launch_rope_t<_Float16, kF16>(a, lph, st);
        case VKV_DTYPE_FP8_E4M3:
            return f32 ? launch_rope_t<float, kFp8>(a, lph, st) : launch_rope_t<_Float16, kFp8>(a, lph, st);
        default: return -1;
    }
}

}  // namespace vkv
