// decode.hip — paged decode attention for gfx950 (wave64), split-K.
//
// Semantics follow the reference kernel (src/attention/paged_attention.cu:13-82):
// kv head = h / (H / Hkv), ctx = min(context_lens[s], max_context_len), output =
// softmax(scale * q.K^T) . V over the ctx tokens gathered through block_tables.
//
// Work decomposition.  One work item is (sequence, kv head, partition of P
// tokens) and is owned by ONE wave; the wave computes all G = H/Hkv query
// heads of the kv head, so every K/V byte is read from HBM once per call
// (the reference re-reads K twice and V once per query head).  Four
// independent waves share a workgroup only to share the launch.
//
// Lane mapping.  A token's head vector is D*eb bytes; LPT = D*eb/16 lanes each
// load 16 contiguous bytes of it, so one wave-wide load fetches TPL = 64/LPT
// whole tokens with fully coalesced 16-byte accesses (D=128 fp16: 16 lanes x
// 16 B per token, 4 tokens per instruction).  Each lane keeps the matching
// slice of the G query vectors in registers; the per-token dot is completed by
// a DPP butterfly over the LPT lanes.
//
// Phases per item: (A) logits of the partition into this wave's LDS slice,
// tracking the running max; (B) p = exp2(logit - max) in place and its sum;
// (C) o = sum p * V with fp32 accumulators, reduced across the TPL token lanes.
// The partial (o, max, sum) goes to the workspace; a second kernel merges the
// partitions of every (sequence, head) with the usual log-sum-exp rescale.
// Logits are kept in the log2 domain (scale * log2 e folded into the scale).
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace vkv {
namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kLoadsPerChunk = 4;  // independent 16-byte loads in flight per lane per chunk
constexpr float kLog2e = 1.4426950408889634f;

struct DecodeArgs {
    void* out;
    const void* q;
    const char* kc;
    const char* vc;
    const float* ks;
    const float* vs;
    const int32_t* bt;
    const int32_t* cl;
    const int32_t* row_seq;  // prefill: query row -> sequence (NULL for decode: row == sequence)
    const int32_t* row_ctx;  // prefill: keys visible to the row (causal), replaces the ctx clamp
    float* part_o;   // [S][H][max_parts][D]
    float* part_ml;  // [S][H][max_parts][2] (max in log2 domain, sum)
    int64_t q_stride;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t bs_log2;
    int32_t max_ctx;
    int32_t max_blocks_per_seq;
    int32_t num_blocks;
    int32_t P;
    int32_t max_parts;
    float scale_log2;
    int32_t accumulate;
};

template <typename IO>
__device__ __forceinline__ float io_to_f32(IO x) {
    return static_cast<float>(x);
}

// Unpack one 16-byte KV chunk into EPL floats in dimension order.  FP8 values
// come out scaled by 2^-8 (the caller folds 256 into its per-token scale).
template <int KVT>
__device__ __forceinline__ void unpack_chunk(const u32x4 w, float* v) {
    if constexpr (KVT == kF32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = as_f32(w[i]);
    } else if constexpr (KVT == kF16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const half2_t h = as_half2(w[i]);
            v[2 * i] = static_cast<float>(h[0]);
            v[2 * i + 1] = static_cast<float>(h[1]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t lo, hi;
            fp8x4_to_half2x2_scaled(w[i], lo, hi);
            const half2_t a = as_half2(lo), b = as_half2(hi);
            v[4 * i + 0] = static_cast<float>(a[0]);
            v[4 * i + 1] = static_cast<float>(b[0]);
            v[4 * i + 2] = static_cast<float>(a[1]);
            v[4 * i + 3] = static_cast<float>(b[1]);
        }
    }
}

template <typename IO, int KVT, int D, int G>
__global__ __launch_bounds__(256) void decode_partition_kernel(DecodeArgs a) {
    constexpr int EB = KvTraits<KVT>::bytes;
    constexpr int EPL = 16 / EB;      // elements per lane per load
    constexpr int LPT = D / EPL;      // lanes per token
    constexpr int TPL = kWave / LPT;  // tokens per wave-wide load
    constexpr int U = kLoadsPerChunk;
    constexpr int CH = U * TPL;       // tokens per chunk
    // fp16 query against fp16 or fp8 keys: packed fp16 dot products (v_dot2_f32_f16).
    constexpr bool HALF_DOT = std::is_same<IO, _Float16>::value && KVT != kF32;
    static_assert(LPT >= 1 && LPT <= kWave && (kWave % LPT) == 0, "head_dim / dtype mapping");

    extern __shared__ float lds[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int s = blockIdx.z;
    const int kvh = blockIdx.y;
    const int part = blockIdx.x * kWavesPerBlock + wave;
    if (part >= a.max_parts) return;
    const int seq = a.row_seq ? a.row_seq[s] : s;
    int ctx = a.row_ctx ? a.row_ctx[s] : a.cl[s];
    ctx = ctx < a.max_ctx ? ctx : a.max_ctx;
    const int t0 = part * a.P;
    if (t0 >= ctx) return;  // whole wave leaves; no workgroup barrier is used
    const int n = (ctx - t0) < a.P ? (ctx - t0) : a.P;
    float* lg = lds + wave * G * a.P;  // [G][P] logits, then probabilities

    const int sub = lane % LPT;  // which 16-byte slice of the head vector
    const int grp = lane / LPT;  // which token of a wave-wide load
    const int bs_mask = (1 << a.bs_log2) - 1;

    // Physical block ids of this partition, one per lane (P / block_size <= 64).
    const int nb = (n + bs_mask) >> a.bs_log2;
    int my_block = 0;
    if (lane < nb) {
        my_block = a.bt[int64_t(seq) * a.max_blocks_per_seq + (t0 >> a.bs_log2) + lane];
        if (a.num_blocks > 0 && unsigned(my_block) >= unsigned(a.num_blocks)) my_block = 0;
    }

    // Query slices of the G heads.
    const int h0 = kvh * G;
    const char* qbase = static_cast<const char*>(a.q) +
                        (int64_t(s) * a.q_stride + int64_t(h0) * D + sub * EPL) * int64_t(sizeof(IO));
    constexpr int QW = HALF_DOT ? EPL / 2 : 1;  // half2 words per head (half path)
    constexpr int QF = HALF_DOT ? 1 : EPL;      // floats per head (float path)
    uint32_t qh[G][QW];
    float qf[G][QF];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const IO* qp = reinterpret_cast<const IO*>(qbase + int64_t(h) * D * sizeof(IO));
        if constexpr (HALF_DOT) {
            const uint16_t* q16 = reinterpret_cast<const uint16_t*>(qp);
            if constexpr (KVT == kF16) {
#pragma unroll
                for (int i = 0; i < QW; ++i) qh[h][i] = uint32_t(q16[2 * i]) | (uint32_t(q16[2 * i + 1]) << 16);
            } else {
                // fp8 keys arrive as (b0,b2),(b1,b3) pairs per 4 bytes; pair the query the same way.
#pragma unroll
                for (int i = 0; i < QW / 2; ++i) {
                    qh[h][2 * i] = uint32_t(q16[4 * i]) | (uint32_t(q16[4 * i + 2]) << 16);
                    qh[h][2 * i + 1] = uint32_t(q16[4 * i + 1]) | (uint32_t(q16[4 * i + 3]) << 16);
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < EPL; ++e) qf[h][e] = io_to_f32(qp[e]);
        }
    }

    const int64_t head_off_bytes = (int64_t(kvh) * D + sub * EPL) * EB;
    const int64_t slot_stride_bytes = int64_t(a.num_kv_heads) * D * EB;
    float logit_scale = a.scale_log2;
    if constexpr (KVT == kFp8) logit_scale *= kFp8HalfScale;

    // ---------------- phase A: logits
    float mx[G];
#pragma unroll
    for (int h = 0; h < G; ++h) mx[h] = -INFINITY;

    for (int c = 0; c < n; c += CH) {
        u32x4 kr[U];
        float ksc[U];
        bool valid[U];
        int tok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            tok[u] = c + u * TPL + grp;
            valid[u] = tok[u] < n;
            const int blk = __shfl(my_block, tok[u] >> a.bs_log2, kWave);
            const int64_t slot = (int64_t(blk) << a.bs_log2) + (tok[u] & bs_mask);
            kr[u] = valid[u] ? load16(a.kc + slot * slot_stride_bytes + head_off_bytes) : u32x4{0, 0, 0, 0};
            if constexpr (KVT == kFp8) ksc[u] = valid[u] ? a.ks[slot * a.num_kv_heads + kvh] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float d[G];
            if constexpr (HALF_DOT) {
#pragma unroll
                for (int h = 0; h < G; ++h) d[h] = 0.0f;
                if constexpr (KVT == kF16) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const half2_t kk = as_half2(kr[u][i]);
#pragma unroll
                        for (int h = 0; h < G; ++h) d[h] = dot2(as_half2(qh[h][i]), kk, d[h]);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        uint32_t lo, hi;
                        fp8x4_to_half2x2_scaled(kr[u][i], lo, hi);
#pragma unroll
                        for (int h = 0; h < G; ++h) {
                            d[h] = dot2(as_half2(qh[h][2 * i]), as_half2(lo), d[h]);
                            d[h] = dot2(as_half2(qh[h][2 * i + 1]), as_half2(hi), d[h]);
                        }
                    }
                }
            } else {
                float kv[EPL];
                unpack_chunk<KVT>(kr[u], kv);
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    float acc = 0.0f;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) acc = fmaf(qf[h][e], kv[e], acc);
                    d[h] = acc;
                }
            }
            float sc = logit_scale;
            if constexpr (KVT == kFp8) sc *= ksc[u];
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float x = group_sum<LPT>(d[h]) * sc;
                x = valid[u] ? x : -INFINITY;
                mx[h] = fmaxf(mx[h], x);
                if (sub == 0 && valid[u]) lg[h * a.P + tok[u]] = x;
            }
        }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) mx[h] = cross_group_max<LPT>(mx[h]);
    wave_lds_sync();

    // ---------------- phase B: probabilities and their sum
    float sum[G];
#pragma unroll
    for (int h = 0; h < G; ++h) sum[h] = 0.0f;
    for (int j = lane; j < n; j += kWave) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float p = __builtin_amdgcn_exp2f(lg[h * a.P + j] - mx[h]);
            lg[h * a.P + j] = p;
            sum[h] += p;
        }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) sum[h] = group_sum<kWave>(sum[h]);
    wave_lds_sync();

    // ---------------- phase C: o = sum_t p_t * V_t
    float acc[G][EPL];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[h][e] = 0.0f;

    for (int c = 0; c < n; c += CH) {
        u32x4 vr[U];
        float vsc[U];
        bool valid[U];
        int tok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            tok[u] = c + u * TPL + grp;
            valid[u] = tok[u] < n;
            const int blk = __shfl(my_block, tok[u] >> a.bs_log2, kWave);
            const int64_t slot = (int64_t(blk) << a.bs_log2) + (tok[u] & bs_mask);
            vr[u] = valid[u] ? load16(a.vc + slot * slot_stride_bytes + head_off_bytes) : u32x4{0, 0, 0, 0};
            if constexpr (KVT == kFp8) vsc[u] = valid[u] ? a.vs[slot * a.num_kv_heads + kvh] * kFp8HalfScale : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float w[G];
#pragma unroll
            for (int h = 0; h < G; ++h) {
                w[h] = valid[u] ? lg[h * a.P + tok[u]] : 0.0f;
                if constexpr (KVT == kFp8) w[h] *= vsc[u];
            }
            float v[EPL];
            unpack_chunk<KVT>(vr[u], v);
#pragma unroll
            for (int e = 0; e < EPL; ++e)
#pragma unroll
                for (int h = 0; h < G; ++h) acc[h][e] = fmaf(w[h], v[e], acc[h][e]);
        }
    }
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[h][e] = cross_group_sum<LPT>(acc[h][e]);

    // ---------------- partial result
    if (grp == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const int64_t item = (int64_t(s) * a.num_heads + h0 + h) * a.max_parts + part;
            float* o = a.part_o + item * D + sub * EPL;
#pragma unroll
            for (int e = 0; e < EPL; e += 4) {
                u32x4 w4;
#pragma unroll
                for (int k = 0; k < 4 && e + k < EPL; ++k) w4[k] = as_u32(acc[h][e + k]);
                store16(o + e, w4);
            }
            if (sub == 0) {
                a.part_ml[item * 2] = mx[h];
                a.part_ml[item * 2 + 1] = sum[h];
            }
        }
    }
}

// Merge the partitions of one (sequence, head): one thread per output element.
template <typename IO, int D>
__global__ __launch_bounds__(D) void decode_reduce_kernel(DecodeArgs a) {
    const int s = blockIdx.y;
    const int h = blockIdx.x;
    const int d = threadIdx.x;
    int ctx = a.row_ctx ? a.row_ctx[s] : a.cl[s];
    ctx = ctx < a.max_ctx ? ctx : a.max_ctx;
    const int np = ctx > 0 ? (ctx + a.P - 1) / a.P : 0;
    const int64_t row = int64_t(s) * a.num_heads + h;
    float r = 0.0f;
    if (np > 0) {
        const float* ml = a.part_ml + row * a.max_parts * 2;
        const float* o = a.part_o + row * a.max_parts * D + d;
        float m = -INFINITY;
        for (int i = 0; i < np; ++i) m = fmaxf(m, ml[2 * i]);
        float l = 0.0f, acc = 0.0f;
        for (int i = 0; i < np; ++i) {
            const float w = __builtin_amdgcn_exp2f(ml[2 * i] - m);
            l = fmaf(w, ml[2 * i + 1], l);
            acc = fmaf(w, o[int64_t(i) * D], acc);
        }
        r = acc / l;
    }
    IO* out = static_cast<IO*>(a.out) + row * D + d;
    if (a.accumulate) r += static_cast<float>(*out);
    *out = static_cast<IO>(r);
}

template <typename IO, int KVT, int D, int G>
void launch_g(const DecodeArgs& args, int grid_x, int Hkv, int S, size_t lds, hipStream_t st) {
    hipLaunchKernelGGL((decode_partition_kernel<IO, KVT, D, G>), dim3(grid_x, Hkv, S),
                       dim3(kWave * kWavesPerBlock), lds, st, args);
}

template <typename IO, int KVT, int D>
int dispatch_g(int G, const DecodeArgs& args, int grid_x, int Hkv, int S, size_t lds, hipStream_t st) {
    switch (G) {
        case 1: launch_g<IO, KVT, D, 1>(args, grid_x, Hkv, S, lds, st); return 0;
        case 2: launch_g<IO, KVT, D, 2>(args, grid_x, Hkv, S, lds, st); return 0;
        case 3: launch_g<IO, KVT, D, 3>(args, grid_x, Hkv, S, lds, st); return 0;
        case 4: launch_g<IO, KVT, D, 4>(args, grid_x, Hkv, S, lds, st); return 0;
        case 5: launch_g<IO, KVT, D, 5>(args, grid_x, Hkv, S, lds, st); return 0;
        case 6: launch_g<IO, KVT, D, 6>(args, grid_x, Hkv, S, lds, st); return 0;
        case 7: launch_g<IO, KVT, D, 7>(args, grid_x, Hkv, S, lds, st); return 0;
        case 8: launch_g<IO, KVT, D, 8>(args, grid_x, Hkv, S, lds, st); return 0;
        default: return VKV_ERR_UNSUPPORTED;
    }
}

template <typename IO, int KVT>
int dispatch_d(int D, int G, const DecodeArgs& args, int grid_x, int Hkv, int S, size_t lds,
               hipStream_t st) {
    switch (D) {
        case 64: return dispatch_g<IO, KVT, 64>(G, args, grid_x, Hkv, S, lds, st);
        case 128: return dispatch_g<IO, KVT, 128>(G, args, grid_x, Hkv, S, lds, st);
        case 256: return dispatch_g<IO, KVT, 256>(G, args, grid_x, Hkv, S, lds, st);
        default: return VKV_ERR_UNSUPPORTED;
    }
}

template <typename IO>
int launch_reduce(int D, const DecodeArgs& args, int H, int S, hipStream_t st) {
    switch (D) {
        case 64: hipLaunchKernelGGL((decode_reduce_kernel<IO, 64>), dim3(H, S), dim3(64), 0, st, args); return 0;
        case 128: hipLaunchKernelGGL((decode_reduce_kernel<IO, 128>), dim3(H, S), dim3(128), 0, st, args); return 0;
        case 256: hipLaunchKernelGGL((decode_reduce_kernel<IO, 256>), dim3(H, S), dim3(256), 0, st, args); return 0;
        default: return VKV_ERR_UNSUPPORTED;
    }
}

int ilog2(int x) {
    int r = 0;
    while ((1 << r) < x) ++r;
    return r;
}

}  // namespace

DecodePlan plan_decode(const vkv_decode_params* p) {
    DecodePlan plan;
    const int bs = p->block_size;
    int P = p->partition_size > 0 ? p->partition_size : 256;
    // A partition starts on a block boundary and holds at most 64 blocks
    // (one block id per lane); logits of 4 waves x G heads x P fit 64 KiB of LDS.
    if (P < bs) P = bs;
    P = (P / bs) * bs;
    if (P > 64 * bs) P = 64 * bs;
    const int G = p->num_kv_heads > 0 ? p->num_heads / p->num_kv_heads : 1;
    while (P > bs && int64_t(kWavesPerBlock) * G * P * 4 > 65536) P -= bs;
    int64_t max_ctx = p->max_context_len;
    const int64_t table_tokens = int64_t(p->max_blocks_per_seq) * bs;
    if (max_ctx > table_tokens) max_ctx = table_tokens;
    if (max_ctx < 0) max_ctx = 0;
    plan.partition_size = P;
    plan.max_parts = int((max_ctx + P - 1) / P);
    if (plan.max_parts < 1) plan.max_parts = 1;
    plan.workspace_bytes = size_t(p->num_seqs) * p->num_heads * plan.max_parts * (p->head_dim + 2) * sizeof(float);
    return plan;
}

// Query row r of a prefill step: its sequence and the number of keys it sees
// (the reference's prefill is one decode per position, src/core/engine.cpp:157-164).
__global__ __launch_bounds__(256) void prefill_rows_kernel(const int32_t* qsl, const int32_t* cl, int32_t num_seqs,
                                                           int32_t rows, int32_t max_ctx, int32_t* row_seq,
                                                           int32_t* row_ctx) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    int lo = 0, hi = num_seqs - 1;  // last s with qsl[s] <= r
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (qsl[mid] <= r) lo = mid;
        else hi = mid - 1;
    }
    const int q0 = qsl[lo], q1 = qsl[lo + 1];
    int ctx = cl[lo] - (q1 - q0) + (r - q0) + 1;
    ctx = ctx < 0 ? 0 : (ctx > max_ctx ? max_ctx : ctx);
    row_seq[r] = lo;
    row_ctx[r] = ctx;
}

int launch_rows(const vkv_decode_params* p, const DecodePlan& plan, void* workspace, const int32_t* row_seq,
                const int32_t* row_ctx, hipStream_t st) {
    DecodeArgs a;
    a.out = p->output;
    a.q = p->query;
    a.kc = static_cast<const char*>(p->key_cache);
    a.vc = static_cast<const char*>(p->value_cache);
    a.ks = p->key_scales;
    a.vs = p->value_scales;
    a.bt = p->block_tables;
    a.cl = p->context_lens;
    a.row_seq = row_seq;
    a.row_ctx = row_ctx;
    const size_t o_elems = size_t(p->num_seqs) * p->num_heads * plan.max_parts * p->head_dim;
    a.part_o = static_cast<float*>(workspace);
    a.part_ml = a.part_o + o_elems;
    a.q_stride = p->query_stride ? p->query_stride : int64_t(p->num_heads) * p->head_dim;
    a.num_heads = p->num_heads;
    a.num_kv_heads = p->num_kv_heads;
    a.bs_log2 = ilog2(p->block_size);
    const int64_t table_tokens = int64_t(p->max_blocks_per_seq) * p->block_size;
    int64_t max_ctx = p->max_context_len < table_tokens ? p->max_context_len : table_tokens;
    a.max_ctx = int32_t(max_ctx < 0 ? 0 : max_ctx);
    a.max_blocks_per_seq = p->max_blocks_per_seq;
    a.num_blocks = p->num_blocks;
    a.P = plan.partition_size;
    a.max_parts = plan.max_parts;
    a.scale_log2 = p->scale * kLog2e;
    a.accumulate = p->accumulate;

    const int G = p->num_heads / p->num_kv_heads;
    const int grid_x = (plan.max_parts + kWavesPerBlock - 1) / kWavesPerBlock;
    const size_t lds = size_t(kWavesPerBlock) * G * plan.partition_size * sizeof(float);
    const int D = p->head_dim;
    int rc;
    if (p->io_dtype == VKV_DTYPE_F32) {
        switch (p->kv_dtype) {
            case VKV_DTYPE_F32: rc = dispatch_d<float, kF32>(D, G, a, grid_x, p->num_kv_heads, p->num_seqs, lds, st); break;
            case VKV_DTYPE_F16: rc = dispatch_d<float, kF16>(D, G, a, grid_x, p->num_kv_heads, p->num_seqs, lds, st); break;
            case VKV_DTYPE_FP8_E4M3: rc = dispatch_d<float, kFp8>(D, G, a, grid_x, p->num_kv_heads, p->num_seqs, lds, st); break;
            default: return VKV_ERR_UNSUPPORTED;
        }
        if (rc) return rc;
        return launch_reduce<float>(D, a, p->num_heads, p->num_seqs, st);
    }
    switch (p->kv_dtype) {
        case VKV_DTYPE_F16: rc = dispatch_d<_Float16, kF16>(D, G, a, grid_x, p->num_kv_heads, p->num_seqs, lds, st); break;
        case VKV_DTYPE_FP8_E4M3: rc = dispatch_d<_Float16, kFp8>(D, G, a, grid_x, p->num_kv_heads, p->num_seqs, lds, st); break;
        default: return VKV_ERR_UNSUPPORTED;
    }
    if (rc) return rc;
    return launch_reduce<_Float16>(D, a, p->num_heads, p->num_seqs, st);
}

int launch_decode(const vkv_decode_params* p, const DecodePlan& plan, void* workspace, hipStream_t st) {
    return launch_rows(p, plan, workspace, nullptr, nullptr, st);
}

DecodePlan plan_prefill(const vkv_prefill_params* p) {
    vkv_decode_params d{};
    d.num_seqs = p->num_query_tokens;
    d.num_heads = p->num_heads;
    d.num_kv_heads = p->num_kv_heads;
    d.head_dim = p->head_dim;
    d.block_size = p->block_size;
    d.max_blocks_per_seq = p->max_blocks_per_seq;
    d.max_context_len = 0x7FFFFFFF;
    DecodePlan plan = plan_decode(&d);
    // row_seq and row_ctx follow the partials
    plan.workspace_bytes += size_t(p->num_query_tokens) * 2 * sizeof(int32_t);
    return plan;
}

int launch_prefill_rows(const vkv_prefill_params* p, const DecodePlan& plan, void* workspace, hipStream_t st) {
    // Rows are decoded like sequences of a decode call, each with its causal context.
    vkv_decode_params d{};
    d.output = p->output;
    d.query = p->query;
    d.key_cache = p->key_cache;
    d.value_cache = p->value_cache;
    d.key_scales = p->key_scales;
    d.value_scales = p->value_scales;
    d.block_tables = p->block_tables;
    d.context_lens = p->context_lens;
    d.query_stride = p->query_stride;
    d.num_seqs = p->num_query_tokens;
    d.num_heads = p->num_heads;
    d.num_kv_heads = p->num_kv_heads;
    d.head_dim = p->head_dim;
    d.block_size = p->block_size;
    d.max_context_len = 0x7FFFFFFF;
    d.max_blocks_per_seq = p->max_blocks_per_seq;
    d.num_blocks = p->num_blocks;
    d.scale = p->scale;
    d.io_dtype = p->io_dtype;
    d.kv_dtype = p->kv_dtype;
    d.accumulate = 0;
    const size_t partial_bytes = plan.workspace_bytes - size_t(p->num_query_tokens) * 2 * sizeof(int32_t);
    int32_t* row_seq = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + partial_bytes);
    int32_t* row_ctx = row_seq + p->num_query_tokens;
    const int32_t table_tokens = int32_t(int64_t(p->max_blocks_per_seq) * p->block_size > 0x7FFFFFFF
                                             ? 0x7FFFFFFF
                                             : int64_t(p->max_blocks_per_seq) * p->block_size);
    hipLaunchKernelGGL(prefill_rows_kernel, dim3((p->num_query_tokens + 255) / 256), dim3(256), 0, st,
                       p->query_start_loc, p->context_lens, p->num_seqs, p->num_query_tokens, table_tokens, row_seq,
                       row_ctx);
    return launch_rows(&d, plan, workspace, row_seq, row_ctx, st);
}

}  // namespace vkv
