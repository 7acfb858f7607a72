// append.hip — KV append (reshape_and_cache) for gfx950.
//
// Replaces the reference's two cudaMemcpyAsync calls per token per layer
// (src/layers/attention.cpp:84-102) with one launch over all tokens.  The
// cache layout [block][slot][kv_head][head_dim] makes a slot's K (or V) row one
// contiguous num_kv_heads*head_dim vector at slot * row, so the append is a row
// scatter: every lane moves 16 destination bytes with one 16-byte load and one
// 16-byte store per K and V, consecutive lanes on consecutive bytes.
#include "common.hpp"
#include "launch.hpp"

namespace vkv {
namespace {

struct AppendArgs {
    const char* key;
    const char* value;
    char* key_cache;
    char* value_cache;
    float* key_scales;
    float* value_scales;
    const int32_t* slot_mapping;
    int64_t key_stride_bytes;    // source bytes between tokens
    int64_t value_stride_bytes;
    int64_t row_bytes;           // destination bytes of one slot (all kv heads)
    int64_t num_slots;
    int64_t total;               // work items
    int32_t chunks_per_row;      // 16-byte destination chunks per row (copy kernels)
    int32_t num_kv_heads;
};

__device__ __forceinline__ u32x4 f32x8_to_f16x8(u32x4 a, u32x4 b) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float x0 = as_f32(a[2 * i]);
        const float x1 = as_f32(a[2 * i + 1]);
        r[i] = uint32_t(f32_to_f16_bits(x0)) | (uint32_t(f32_to_f16_bits(x1)) << 16);
        const float y0 = as_f32(b[2 * i]);
        const float y1 = as_f32(b[2 * i + 1]);
        r[2 + i] = uint32_t(f32_to_f16_bits(y0)) | (uint32_t(f32_to_f16_bits(y1)) << 16);
    }
    return r;
}

// Same-type append (bit copy, SRC_PER_DST = 1) or f32 -> f16 (SRC_PER_DST = 2,
// 32 source bytes per 16 destination bytes).  Each thread takes UNROLL
// grid-strided chunks per iteration so that their slot ids, loads and stores
// are in flight together; sources and cache rows are streamed (non-temporal:
// each byte is touched once).
// UNROLL chunks per thread and iteration: 2 while a thread has few chunks,
// 8 once every thread of the grid has at least 8 (measured, Hkv8/D128 fp16
// rows at random slots: T = 4 216 and 65 536 tokens 55 % and 63 % of 8 TB/s
// with 2 against 32 % and 58 % with 8; T = 262 144 60 % with 2, 61 % with 8).
constexpr int kAppendUnrollSmall = 2;
constexpr int kAppendUnrollLarge = 8;
template <int SRC_PER_DST, int UNROLL>
__global__ __launch_bounds__(kBlockThreads) void append_rows_kernel(AppendArgs a) {
    const int64_t stride = int64_t(gridDim.x) * kBlockThreads;
    for (int64_t i0 = int64_t(blockIdx.x) * kBlockThreads + threadIdx.x; i0 < a.total; i0 += stride * UNROLL) {
        int64_t slot[UNROLL], t[UNROLL], c[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int64_t i = i0 + u * stride;
            t[u] = i / a.chunks_per_row;
            c[u] = i - t[u] * a.chunks_per_row;
            slot[u] = i < a.total ? int64_t(a.slot_mapping[t[u]]) : -1;
        }
        // Latency-bound launches (a chunk or two per thread) request the
        // source rows together with the slot ids (every token has one), so
        // the loads do not wait for the slot check and only the stores depend
        // on it.  Streaming launches (UNROLL = kAppendUnrollLarge) issue a
        // chunk's loads after its slot check (measured: T = 4 216 57 -> 58 %
        // of 8 TB/s with the early loads, T = 262 144 61 -> 59 %).
        constexpr bool kEarlyLoads = UNROLL < kAppendUnrollLarge;
        u32x4 k[UNROLL][SRC_PER_DST], v[UNROLL][SRC_PER_DST];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            if (kEarlyLoads ? i0 + u * stride >= a.total : (slot[u] < 0 || slot[u] >= a.num_slots)) continue;
            const char* ks = a.key + t[u] * a.key_stride_bytes + c[u] * 16 * SRC_PER_DST;
            const char* vs = a.value + t[u] * a.value_stride_bytes + c[u] * 16 * SRC_PER_DST;
#pragma unroll
            for (int j = 0; j < SRC_PER_DST; ++j) {
                k[u][j] = load16_nt(ks + 16 * j);
                v[u][j] = load16_nt(vs + 16 * j);
            }
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            if (slot[u] < 0 || slot[u] >= a.num_slots) continue;
            const int64_t dst = slot[u] * a.row_bytes + c[u] * 16;
            if constexpr (SRC_PER_DST == 1) {
                store16_nt(a.key_cache + dst, k[u][0]);
                store16_nt(a.value_cache + dst, v[u][0]);
            } else {
                store16_nt(a.key_cache + dst, f32x8_to_f16x8(k[u][0], k[u][1]));
                store16_nt(a.value_cache + dst, f32x8_to_f16x8(v[u][0], v[u][1]));
            }
        }
    }
}

// x / s exactly as the correctly rounded fp32 quotient would encode to e4m3.
// z = x * fl(1/s) is within 2 fp32 ulps of fl(x / s), so the two can only
// encode differently when an e4m3 rounding midpoint is within that distance of
// z: normal e4m3 range midpoints are the fp32 values whose 20 mantissa bits
// below the kept 3 equal 0x80000.  Those cases, the e4m3 subnormal range
// (|z| < 2^-6, other midpoints) and non-finite values take the IEEE division.
__device__ __forceinline__ float quotient(float x, float s, float rinv) {
    const float z = x * rinv;
    const uint32_t b = as_u32(z) & 0x7FFFFFFFu;
    const int d = int(b & 0xFFFFFu) - 0x80000;
    if (b < 0x3C800000u || b >= 0x7F800000u || (d >= -4 && d <= 4)) return x / s;
    return z;
}

// Quantise-on-append to e4m3fn.  A group of LPT = head_dim/16 consecutive
// lanes holds one (token, kv head) vector, 16 elements per lane, for K and V
// at once (both loaded before either is used); each group's amax comes from a
// DPP max reduction, every lane forms its 16 quotients x / scale (exact, see
// quotient()) and encodes them with gfx950's v_cvt_pk_fp8_f32 (OCP e4m3fn,
// round to nearest even).  Quotients are finite and within 448 (1 + 2^-22)
// unless the input holds inf or NaN; a wave that meets one encodes with the
// software rule (f32_to_fp8_sat: NaN -> 0x7F, saturation) instead.
// EARLY (launches whose grid covers every item, one per thread): the slot id
// and the source rows are requested together and only the stores wait for
// the slot check; otherwise (grid-strided) an item's loads follow its slot
// check (measured: T = 4 216 36 -> 37 %, 65 536 64 -> 66 % of 8 TB/s with
// the early loads, T = 262 144 64 -> 63 %).
template <typename SRC, int LPT, bool EARLY>
__global__ __launch_bounds__(kBlockThreads) void append_fp8_kernel(AppendArgs a) {
    constexpr int SRC_BYTES = 16 * int(sizeof(SRC));
    const int64_t stride = int64_t(gridDim.x) * kBlockThreads;
    const int64_t per_token = int64_t(a.num_kv_heads) * LPT;
    for (int64_t i = int64_t(blockIdx.x) * kBlockThreads + threadIdx.x; i < a.total; i += stride) {
        const int64_t t = i / per_token;
        const int64_t r = i - t * per_token;  // head * LPT + sub
        // (the slot check is uniform within a group, which shares t)
        const int64_t slot = a.slot_mapping[t];
        if (!EARLY && (slot < 0 || slot >= a.num_slots)) continue;
        const int64_t head = r / LPT;
        const char* src[2] = {a.key + t * a.key_stride_bytes + r * SRC_BYTES,
                              a.value + t * a.value_stride_bytes + r * SRC_BYTES};
        u32x4 w[2][SRC_BYTES / 16];
#pragma unroll
        for (int kv = 0; kv < 2; ++kv)
#pragma unroll
            for (int j = 0; j < SRC_BYTES / 16; ++j) w[kv][j] = load16_nt(src[kv] + 16 * j);
        float x[2][16];
        float amax[2] = {0.0f, 0.0f};
#pragma unroll
        for (int kv = 0; kv < 2; ++kv) {
#pragma unroll
            for (int j = 0; j < SRC_BYTES / 16; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (sizeof(SRC) == 4) {
                        x[kv][4 * j + e] = as_f32(w[kv][j][e]);
                    } else {
                        x[kv][8 * j + 2 * e] = f16_bits_to_f32(uint16_t(w[kv][j][e] & 0xFFFFu));
                        x[kv][8 * j + 2 * e + 1] = f16_bits_to_f32(uint16_t(w[kv][j][e] >> 16));
                    }
                }
#pragma unroll
            for (int e = 0; e < 16; ++e) amax[kv] = fmaxf(amax[kv], fabsf(x[kv][e]));
        }
        amax[0] = group_max<LPT>(amax[0]);
        amax[1] = group_max<LPT>(amax[1]);
        bool finite = true;
        float scale[2];
#pragma unroll
        for (int kv = 0; kv < 2; ++kv) {
            scale[kv] = fp8_scale_from_amax(amax[kv]);
            const float rinv = 1.0f / scale[kv];  // correctly rounded
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                x[kv][e] = quotient(x[kv][e], scale[kv], rinv);
                finite &= (as_u32(x[kv][e]) & 0x7F800000u) != 0x7F800000u;
            }
        }
        u32x4 q[2];
        if (__builtin_amdgcn_ballot_w64(!finite) == 0) {
#pragma unroll
            for (int kv = 0; kv < 2; ++kv)
#pragma unroll
                for (int wd = 0; wd < 4; ++wd) {
                    int v = __builtin_amdgcn_cvt_pk_fp8_f32(x[kv][4 * wd], x[kv][4 * wd + 1], 0, false);
                    v = __builtin_amdgcn_cvt_pk_fp8_f32(x[kv][4 * wd + 2], x[kv][4 * wd + 3], v, true);
                    q[kv][wd] = uint32_t(v);
                }
        } else {
#pragma unroll
            for (int kv = 0; kv < 2; ++kv)
#pragma unroll
                for (int wd = 0; wd < 4; ++wd) {
                    uint32_t packed = 0;
#pragma unroll
                    for (int b = 0; b < 4; ++b) packed |= f32_to_fp8_sat(x[kv][4 * wd + b]) << (8 * b);
                    q[kv][wd] = packed;
                }
        }
        if (EARLY && (slot < 0 || slot >= a.num_slots)) continue;
        const int64_t dst = slot * a.row_bytes + r * 16;
        store16_nt(a.key_cache + dst, q[0]);
        store16_nt(a.value_cache + dst, q[1]);
        if ((r % LPT) == 0) {
            a.key_scales[slot * a.num_kv_heads + head] = scale[0];
            a.value_scales[slot * a.num_kv_heads + head] = scale[1];
        }
    }
}

// Any head_dim, any alignment (the reference's append is a per-token memcpy of
// any row, src/layers/attention.cpp:93-101): one wave per (token, kv head),
// lanes stride over head_dim one element at a time.  Same conversion (fp32 ->
// fp16 RNE) and FP8 rule (wave amax, scale = amax / 448, exact quotient,
// software e4m3fn encoder) as the vector kernels, so results are identical.
template <typename SRC, int DST>
__global__ __launch_bounds__(kBlockThreads) void append_elems_kernel(AppendArgs a, int head_dim) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t wave = (int64_t(blockIdx.x) * kBlockThreads + threadIdx.x) / kWave;
    const int64_t waves = int64_t(gridDim.x) * kBlockThreads / kWave;
    const int64_t pairs = a.total;  // (token, kv head) pairs
    for (int64_t i = wave; i < pairs; i += waves) {
        const int64_t t = i / a.num_kv_heads;
        const int head = int(i - t * a.num_kv_heads);
        const int64_t slot = a.slot_mapping[t];
        if (slot < 0 || slot >= a.num_slots) continue;
        const SRC* src[2] = {reinterpret_cast<const SRC*>(a.key + t * a.key_stride_bytes) + int64_t(head) * head_dim,
                             reinterpret_cast<const SRC*>(a.value + t * a.value_stride_bytes) +
                                 int64_t(head) * head_dim};
        char* dst[2] = {a.key_cache + slot * a.row_bytes, a.value_cache + slot * a.row_bytes};
        if constexpr (DST == kFp8) {
            float amax[2] = {0.0f, 0.0f};
            for (int d = lane; d < head_dim; d += kWave)
#pragma unroll
                for (int kv = 0; kv < 2; ++kv) amax[kv] = fmaxf(amax[kv], fabsf(static_cast<float>(src[kv][d])));
#pragma unroll
            for (int kv = 0; kv < 2; ++kv) {
                const float scale = fp8_scale_from_amax(group_max<kWave>(amax[kv]));
                const float rinv = 1.0f / scale;
                uint8_t* out = reinterpret_cast<uint8_t*>(dst[kv]) + int64_t(head) * head_dim;
                for (int d = lane; d < head_dim; d += kWave)
                    out[d] = uint8_t(f32_to_fp8_sat(quotient(static_cast<float>(src[kv][d]), scale, rinv)));
                if (lane == 0) (kv ? a.value_scales : a.key_scales)[slot * a.num_kv_heads + head] = scale;
            }
        } else {
#pragma unroll
            for (int kv = 0; kv < 2; ++kv) {
                for (int d = lane; d < head_dim; d += kWave) {
                    if constexpr (DST == kF16)
                        reinterpret_cast<uint16_t*>(dst[kv])[int64_t(head) * head_dim + d] =
                            sizeof(SRC) == 2 ? reinterpret_cast<const uint16_t*>(src[kv])[d]
                                             : f32_to_f16_bits(static_cast<float>(src[kv][d]));
                    else
                        reinterpret_cast<float*>(dst[kv])[int64_t(head) * head_dim + d] = static_cast<float>(src[kv][d]);
                }
            }
        }
    }
}

int grid_for(int64_t total) {
    int64_t blocks = (total + 255) / 256;
    const int64_t cap = int64_t(256) * 64;  // 64 workgroups per CU, then grid-stride
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    return int(blocks);
}

template <typename SRC, bool EARLY>
int launch_fp8_e(const AppendArgs& a, int lpt, int g, hipStream_t st) {
    switch (lpt) {
        case 1: hipLaunchKernelGGL((append_fp8_kernel<SRC, 1, EARLY>), dim3(g), dim3(kBlockThreads), 0, st, a); break;
        case 2: hipLaunchKernelGGL((append_fp8_kernel<SRC, 2, EARLY>), dim3(g), dim3(kBlockThreads), 0, st, a); break;
        case 4: hipLaunchKernelGGL((append_fp8_kernel<SRC, 4, EARLY>), dim3(g), dim3(kBlockThreads), 0, st, a); break;
        case 8: hipLaunchKernelGGL((append_fp8_kernel<SRC, 8, EARLY>), dim3(g), dim3(kBlockThreads), 0, st, a); break;
        case 16: hipLaunchKernelGGL((append_fp8_kernel<SRC, 16, EARLY>), dim3(g), dim3(kBlockThreads), 0, st, a); break;
        default: return -1;
    }
    return 0;
}

template <typename SRC>
int launch_fp8(const AppendArgs& a, int lpt, hipStream_t st) {
    const int g = grid_for(a.total);
    if (a.total <= int64_t(g) * kBlockThreads) return launch_fp8_e<SRC, true>(a, lpt, g, st);
    return launch_fp8_e<SRC, false>(a, lpt, g, st);
}

}  // namespace

int launch_append(const vkv_append_params* p, hipStream_t st) {
    const int src_eb = p->src_dtype == VKV_DTYPE_F32 ? 4 : 2;
    const int dst_eb = p->cache_dtype == VKV_DTYPE_F32 ? 4 : p->cache_dtype == VKV_DTYPE_F16 ? 2 : 1;
    const int64_t row = int64_t(p->num_kv_heads) * p->head_dim;
    AppendArgs a;
    a.key = static_cast<const char*>(p->key);
    a.value = static_cast<const char*>(p->value);
    a.key_cache = static_cast<char*>(p->key_cache);
    a.value_cache = static_cast<char*>(p->value_cache);
    a.key_scales = p->key_scales;
    a.value_scales = p->value_scales;
    a.slot_mapping = p->slot_mapping;
    a.key_stride_bytes = (p->key_stride ? p->key_stride : row) * src_eb;
    a.value_stride_bytes = (p->value_stride ? p->value_stride : row) * src_eb;
    a.row_bytes = row * dst_eb;
    a.num_slots = int64_t(p->num_blocks) * p->block_size;
    a.num_kv_heads = p->num_kv_heads;
    // The vector kernels move 16-byte pieces of whole rows (FP8: 16 elements
    // per lane, a power-of-two number of lanes per head); anything else takes
    // the element kernel.
    const uintptr_t bits = reinterpret_cast<uintptr_t>(p->key) | reinterpret_cast<uintptr_t>(p->value) |
                           uintptr_t(a.key_stride_bytes) | uintptr_t(a.value_stride_bytes) |
                           reinterpret_cast<uintptr_t>(p->key_cache) | reinterpret_cast<uintptr_t>(p->value_cache);
    const int lpt = p->head_dim / 16;
    const bool vector_rows = (bits & 15u) == 0 && (a.row_bytes % 16) == 0 &&
                             (p->cache_dtype != VKV_DTYPE_FP8_E4M3 ||
                              (p->head_dim % 16 == 0 && lpt <= 16 && (lpt & (lpt - 1)) == 0));
    if (!vector_rows) {
        a.total = int64_t(p->num_tokens) * p->num_kv_heads;
        const int g = grid_for(a.total * kWave);
        const int D = p->head_dim;
        if (p->src_dtype == VKV_DTYPE_F32) {
            switch (p->cache_dtype) {
                case VKV_DTYPE_F32: hipLaunchKernelGGL((append_elems_kernel<float, kF32>), dim3(g), dim3(kBlockThreads), 0, st, a, D); break;
                case VKV_DTYPE_F16: hipLaunchKernelGGL((append_elems_kernel<float, kF16>), dim3(g), dim3(kBlockThreads), 0, st, a, D); break;
                default: hipLaunchKernelGGL((append_elems_kernel<float, kFp8>), dim3(g), dim3(kBlockThreads), 0, st, a, D); break;
            }
        } else {
            switch (p->cache_dtype) {
                case VKV_DTYPE_F16: hipLaunchKernelGGL((append_elems_kernel<_Float16, kF16>), dim3(g), dim3(kBlockThreads), 0, st, a, D); break;
                case VKV_DTYPE_FP8_E4M3: hipLaunchKernelGGL((append_elems_kernel<_Float16, kFp8>), dim3(g), dim3(kBlockThreads), 0, st, a, D); break;
                default: return -1;
            }
        }
        return 0;
    }
    if (p->cache_dtype == VKV_DTYPE_FP8_E4M3) {
        a.chunks_per_row = 0;
        a.total = int64_t(p->num_tokens) * p->num_kv_heads * lpt;
        if (p->src_dtype == VKV_DTYPE_F32) return launch_fp8<float>(a, lpt, st);
        return launch_fp8<_Float16>(a, lpt, st);
    }
    a.chunks_per_row = int32_t(a.row_bytes / 16);
    a.total = int64_t(p->num_tokens) * a.chunks_per_row;
    const int g = grid_for(a.total);
    const bool deep = a.total >= int64_t(g) * 256 * kAppendUnrollLarge;
    if (src_eb == dst_eb) {
        if (deep) hipLaunchKernelGGL((append_rows_kernel<1, kAppendUnrollLarge>), dim3(g), dim3(kBlockThreads), 0, st, a);
        else hipLaunchKernelGGL((append_rows_kernel<1, kAppendUnrollSmall>), dim3(g), dim3(kBlockThreads), 0, st, a);
    } else {
        if (deep) hipLaunchKernelGGL((append_rows_kernel<2, kAppendUnrollLarge>), dim3(g), dim3(kBlockThreads), 0, st, a);
        else hipLaunchKernelGGL((append_rows_kernel<2, kAppendUnrollSmall>), dim3(g), dim3(kBlockThreads), 0, st, a);
    }
    return 0;
}

}  // namespace vkv
