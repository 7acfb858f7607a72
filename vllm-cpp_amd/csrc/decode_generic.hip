// decode_generic.hip — split-K paged decode for the shapes the fixed-shape
// kernels of decode.hip do not cover: any head_dim up to 1024, any group size
// H / Hkv and any block size (the reference kernel runs for all of them: its
// lane-strided head_dim loop, src/attention/paged_attention.cu:38, its
// h / (H / Hkv) mapping, :19, and its t / block_size gather, :34).  Same
// semantics, workspace layout and merge kernel as decode.hip.
//
// Work item = (row, partition of P tokens, kv head, chunk of GC query heads
// of the group), owned by one wave; the chunks of a kv head are adjacent
// items, so the waves of a workgroup read the same K/V lines.  A token's head
// vector is split into vectors of EPV elements (16 bytes; FP8 8 bytes); LPT =
// min(64, DP / EPV) lanes hold NV vectors each, v = sub + LPT j, so one
// wave-wide load covers TPL = 64 / LPT tokens with consecutive lanes on
// consecutive vectors.  DP is head_dim rounded up to a power of two (>= 64):
// lanes past head_dim load nothing and hold zero query elements.  When
// head_dim is not a whole number of vectors (or the caches are not 16-byte
// aligned) every element is loaded on its own.  Block ids come from a
// per-lane table of the partition's blocks (a partition holds at most 64
// blocks) by division (a precomputed multiplier, block_div), so any block size
// works.  Dots and the online softmax are fp32, as in decode.hip's VALU
// variant; fp16 queries over an fp16 cache take packed fp16 dot products
// (fp32 accumulation) for the logits and, over token pairs, for p * V, with
// the weights rounded to fp16 as the fixed-shape kernels round them.  Chunks
// of up to 2 query heads load 8 tokens per lane (more bytes in flight, for
// the byte-bound shapes), larger ones 4 (2 above 4 heads).
#include "common.hpp"
#include "decode_common.hpp"
#include "launch.hpp"

namespace vkv {
namespace dec {
namespace {

// Largest padded head_dim and the group chunk the register budget allows.
constexpr int kMaxGenericDim = 1024;

// n (0..EPV) leading elements of one lane vector loaded one by one, the rest
// zero, packed as load_lane packs them (element e in word e / (4 / EB)).
template <int KVT>
__device__ __forceinline__ void load_elems(const char* p, int n, uint32_t* w) {
    constexpr int EB = KvTraits<KVT>::bytes;
    constexpr int EPW = 4 / EB;  // elements per 32-bit word
#pragma unroll
    for (int i = 0; i < LaneLoad<KVT>::words; ++i) {
        uint32_t x = 0;
#pragma unroll
        for (int k = 0; k < EPW; ++k) {
            const int e = i * EPW + k;
            if (e < n) {
                uint32_t b;
                if constexpr (EB == 4) b = *reinterpret_cast<const uint32_t*>(p + e * 4);
                else if constexpr (EB == 2) b = *reinterpret_cast<const uint16_t*>(p + e * 2);
                else b = *reinterpret_cast<const uint8_t*>(p + e);
                x |= b << (8 * EB * k);
            }
        }
        w[i] = x;
    }
}

template <int KVT, int DP, int GC>
struct GenericShape {
    static constexpr int EPV = LaneLoad<KVT>::elems;          // elements per lane vector
    static constexpr int LW = LaneLoad<KVT>::words;
    static constexpr int LPT = DP / EPV < kWave ? DP / EPV : kWave;  // lanes per token
    static constexpr int NV = DP / (LPT * EPV);               // vectors per lane
    static constexpr int TPL = kWave / LPT;                   // tokens per wave-wide load
    static constexpr int U0 = (GC <= 2 ? 8 : GC <= 4 ? 4 : 2) / NV;
    static constexpr int U = U0 > 0 ? U0 : 1;                 // token loads per lane per chunk
    static constexpr int CH = U * TPL;                        // tokens per chunk
    static_assert(LPT >= 1 && (kWave % LPT) == 0, "lane mapping");
};

// HQ: fp16 queries over an fp16 cache; the logits are packed fp16 dot
// products (v_dot2_f32_f16, fp32 accumulation) of the query and key halves
// instead of fp32 products of unpacked keys.
template <int KVT, int DP, int GC, bool HQ>
__device__ __forceinline__ void decode_item_generic(const DecodeArgs& a, const int P, const int s, const int kvh,
                                                    const int g0, const int part, const int lane) {
    static_assert(!HQ || KVT == kF16, "packed query dots need an fp16 cache");
    using Sh = GenericShape<KVT, DP, GC>;
    constexpr int EB = KvTraits<KVT>::bytes;
    constexpr int EPV = Sh::EPV, LW = Sh::LW, LPT = Sh::LPT, NV = Sh::NV, TPL = Sh::TPL, U = Sh::U, CH = Sh::CH;
    const int D = a.head_dim;
    const int Hkv = a.num_kv_heads;
    const int G = a.num_heads / Hkv;
    const int gn = G - g0 < GC ? G - g0 : GC;  // query heads of this chunk
    const int bs = a.block_size;
    const bool vec = a.vec_loads != 0;

    const int seq = a.row_seq ? a.row_seq[s] : s;
    const int ctx = row_context(a, s);
    const int t0 = part * P;
    if (t0 >= ctx) return;
    const int n = (ctx - t0) < P ? (ctx - t0) : P;
    const int sub = lane % LPT;
    const int grp = lane / LPT;

    // Physical block ids of the partition, one per lane (P <= 64 blocks).
    const int nb = (n + bs - 1) / bs;
    int my_block = 0;
    if (lane < nb) {
        my_block = a.bt[int64_t(seq) * a.max_blocks_per_seq + t0 / bs + lane];
        if (a.num_blocks > 0 && unsigned(my_block) >= unsigned(a.num_blocks)) my_block = 0;
    }

    // Query elements of the chunk's heads (zero past head_dim and past gn);
    // a negative scale is moved into the query (exact sign flip).
    const bool neg_scale = a.scale_log2 < 0.0f;
    const int64_t qrow = query_row(a, s) * a.q_stride + int64_t(kvh * G + g0) * D;
    float qf[GC][NV][EPV];
#pragma unroll
    for (int h = 0; h < GC; ++h)
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int e = 0; e < EPV; ++e) {
                const int d = (sub + LPT * j) * EPV + e;
                float x = 0.0f;
                if (h < gn && d < D) {
                    const int64_t i = qrow + int64_t(h) * D + d;
                    x = a.io_f32 ? static_cast<const float*>(a.q)[i]
                                 : static_cast<float>(static_cast<const _Float16*>(a.q)[i]);
                }
                qf[h][j][e] = neg_scale ? -x : x;
            }
    // HQ: the same query elements as fp16 pairs (exact: the query is fp16)
    uint32_t qh[HQ ? GC : 1][HQ ? NV : 1][HQ ? LW : 1];
    if constexpr (HQ) {
#pragma unroll
        for (int h = 0; h < GC; ++h)
#pragma unroll
            for (int j = 0; j < NV; ++j)
#pragma unroll
                for (int w = 0; w < LW; ++w) {
                    const half2_t p2 = {static_cast<_Float16>(qf[h][j][2 * w]), static_cast<_Float16>(qf[h][j][2 * w + 1])};
                    qh[h][j][w] = __builtin_bit_cast(uint32_t, p2);
                }
    }
    float sc = neg_scale ? -a.scale_log2 : a.scale_log2;
    if constexpr (KVT == kFp8) sc *= kFp8HalfScale;  // unpack_lane yields codes x 2^-8

    const int64_t slot_stride = int64_t(Hkv) * D * EB;
    const int64_t head_off = int64_t(kvh) * D * EB;

    float m[GC], l[GC], acc[GC][NV][EPV];
#pragma unroll
    for (int h = 0; h < GC; ++h) {
        m[h] = -INFINITY;
        l[h] = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int e = 0; e < EPV; ++e) acc[h][j][e] = 0.0f;
    }

    for (int c = 0; c < n; c += CH) {
        uint32_t kw[U][NV][LW], vw[U][NV][LW];
        float ks[U], vs[U];
        bool valid[U];
        // loads of the chunk (tokens past n read token 0 of the partition)
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int tok = c + u * TPL + grp;
            valid[u] = tok < n;
            const int tk = valid[u] ? tok : 0;
            const int bi = block_div(a, tk);
            const int blk = __shfl(my_block, bi, kWave);
            const int64_t slot = int64_t(blk) * bs + (tk - bi * bs);
            const char* kr = a.kc + slot * slot_stride + head_off;
            const char* vr = a.vc + slot * slot_stride + head_off;
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int e0 = (sub + LPT * j) * EPV;
                if (vec) {
                    if (e0 < D) {
                        load_lane<KVT>(kr + e0 * EB, kw[u][j]);
                        load_lane<KVT>(vr + e0 * EB, vw[u][j]);
                    } else {
#pragma unroll
                        for (int w = 0; w < LW; ++w) kw[u][j][w] = vw[u][j][w] = 0u;
                    }
                } else {
                    const int cnt = D - e0 < 0 ? 0 : (D - e0 < EPV ? D - e0 : EPV);
                    load_elems<KVT>(kr + e0 * EB, cnt, kw[u][j]);
                    load_elems<KVT>(vr + e0 * EB, cnt, vw[u][j]);
                }
            }
            if constexpr (KVT == kFp8) {
                ks[u] = a.ks[slot * Hkv + kvh];
                vs[u] = valid[u] ? a.vs[slot * Hkv + kvh] * kFp8HalfScale : 0.0f;
            }
        }
        // raw dot products, complete in every lane of a token group
        float r[U][GC];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float kf[HQ ? 1 : NV][HQ ? 1 : EPV];
            if constexpr (!HQ) {
#pragma unroll
                for (int j = 0; j < NV; ++j) unpack_lane<KVT>(kw[u][j], kf[j]);
            }
#pragma unroll
            for (int h = 0; h < GC; ++h) {
                float t = 0.0f;
                if constexpr (HQ) {
#pragma unroll
                    for (int j = 0; j < NV; ++j)
#pragma unroll
                        for (int w = 0; w < LW; ++w) t = dot2(as_half2(qh[h][j][w]), as_half2(kw[u][j][w]), t);
                } else {
#pragma unroll
                    for (int j = 0; j < NV; ++j)
#pragma unroll
                        for (int e = 0; e < EPV; ++e) t = fmaf(qf[h][j][e], kf[j][e], t);
                }
                float y = group_sum<LPT>(t);
                if constexpr (KVT == kFp8) y *= ks[u];
                r[u][h] = valid[u] ? y : -INFINITY;
            }
        }
        // running max (wave-uniform per head): rescale only when it grows
        float msc[GC];
#pragma unroll
        for (int h = 0; h < GC; ++h) {
            float cm = r[0][h];
#pragma unroll
            for (int u = 1; u < U; ++u) cm = fmaxf(cm, r[u][h]);
            cm = cross_group_max<LPT>(cm);
            if (cm > m[h]) {
                const float alpha = __builtin_amdgcn_exp2f((m[h] - cm) * sc);
                m[h] = cm;
                l[h] *= alpha;
#pragma unroll
                for (int j = 0; j < NV; ++j)
#pragma unroll
                    for (int e = 0; e < EPV; ++e) acc[h][j][e] *= alpha;
            }
            msc[h] = m[h] * sc;
        }
        // weights (masked tokens weigh exactly 0) and p * V.  HQ with an even
        // number of token loads: packed fp16 dot products over token pairs
        // (weights rounded to fp16, and the row sum over the same rounded
        // weights), as the fixed-shape kernels do.
        constexpr bool PAIR = HQ && (U % 2) == 0;
        if constexpr (PAIR) {
            const half2_t ones = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
#pragma unroll
            for (int u = 0; u < U; u += 2) {
                half2_t pp[GC];
#pragma unroll
                for (int h = 0; h < GC; ++h) {
                    const float p0 = valid[u] ? __builtin_amdgcn_exp2f(fmaf(r[u][h], sc, -msc[h])) : 0.0f;
                    const float p1 = valid[u + 1] ? __builtin_amdgcn_exp2f(fmaf(r[u + 1][h], sc, -msc[h])) : 0.0f;
                    pp[h] = half2_t{static_cast<_Float16>(p0), static_cast<_Float16>(p1)};
                    l[h] = dot2(pp[h], ones, l[h]);
                }
#pragma unroll
                for (int j = 0; j < NV; ++j)
#pragma unroll
                    for (int w = 0; w < LW; ++w) {
                        // (element 2w of token u, of token u + 1) and (element 2w + 1 of both)
                        const uint32_t lo = __builtin_amdgcn_perm(vw[u + 1][j][w], vw[u][j][w], 0x05040100u);
                        const uint32_t hi = __builtin_amdgcn_perm(vw[u + 1][j][w], vw[u][j][w], 0x07060302u);
#pragma unroll
                        for (int h = 0; h < GC; ++h) {
                            acc[h][j][2 * w] = dot2(pp[h], as_half2(lo), acc[h][j][2 * w]);
                            acc[h][j][2 * w + 1] = dot2(pp[h], as_half2(hi), acc[h][j][2 * w + 1]);
                        }
                    }
            }
        } else {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float vf[NV][EPV];
#pragma unroll
            for (int j = 0; j < NV; ++j) unpack_lane<KVT>(vw[u][j], vf[j]);
#pragma unroll
            for (int h = 0; h < GC; ++h) {
                const float p = valid[u] ? __builtin_amdgcn_exp2f(fmaf(r[u][h], sc, -msc[h])) : 0.0f;
                l[h] += p;
                float w = p;
                if constexpr (KVT == kFp8) w *= vs[u];
#pragma unroll
                for (int j = 0; j < NV; ++j)
#pragma unroll
                    for (int e = 0; e < EPV; ++e) acc[h][j][e] = fmaf(w, vf[j][e], acc[h][j][e]);
            }
        }
        }
    }

#pragma unroll
    for (int h = 0; h < GC; ++h) {
        l[h] = cross_group_sum<LPT>(l[h]);
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int e = 0; e < EPV; ++e) acc[h][j][e] = cross_group_sum<LPT>(acc[h][j][e]);
    }
    // partial (o, max, sum) of each head of the chunk
    if (grp == 0) {
#pragma unroll
        for (int h = 0; h < GC; ++h) {
            if (h >= gn) break;
            const int64_t item = ((int64_t(s) * Hkv + kvh) * a.max_parts + part) * G + g0 + h;
            float* o = a.part_o + item * D;
#pragma unroll
            for (int j = 0; j < NV; ++j)
#pragma unroll
                for (int e = 0; e < EPV; ++e) {
                    const int d = (sub + LPT * j) * EPV + e;
                    if (d < D) o[d] = acc[h][j][e];
                }
            if (sub == 0) {
                a.part_ml[item * 2] = m[h] * sc;  // log2-domain max, as the merge expects
                a.part_ml[item * 2 + 1] = l[h];
            }
        }
    }
}

template <int KVT, int DP, int GC, bool HQ>
__global__ __launch_bounds__(256) void decode_generic_kernel(const DecodeArgs a) {
    const int lane = threadIdx.x & (kWave - 1);
    const int G = a.num_heads / a.num_kv_heads;
    const int chunks = (G + GC - 1) / GC;
    run_partitions(a, a.num_kv_heads * chunks, [&](const int P, const int row, const int part, const int sub)
                                                   __attribute__((always_inline)) {
        const int kvh = sub / chunks;
        decode_item_generic<KVT, DP, GC, HQ>(a, P, row, kvh, (sub - kvh * chunks) * GC, part, lane);
    });
}

// One workgroup per resident slot (occupancy queried once per variant), never
// more than there are item groups.
template <int KVT, int DP, int GC, bool HQ>
void launch_variant_q(DecodeArgs& a, int64_t max_pairs, size_t lds, hipStream_t st) {
    static int per_cu_cached = 0;  // benign race: every thread computes the same value
    int per_cu = per_cu_cached;
    if (per_cu <= 0) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_generic_kernel<KVT, DP, GC, HQ>,
                                                         kWave * kWavesPerBlock, 0) != hipSuccess || per_cu <= 0)
            per_cu = 1;
        per_cu_cached = per_cu;
    }
    const int by_lds = kLdsPerCu / int(lds + 4096);
    if (by_lds < per_cu) per_cu = by_lds > 0 ? by_lds : 1;
    per_cu = blocks_per_cu(per_cu);
    const int G = a.num_heads / a.num_kv_heads;
    const int64_t items = max_pairs * a.num_kv_heads * ((G + GC - 1) / GC);
    const int64_t groups = (items + kWavesPerBlock - 1) / kWavesPerBlock;
    const int64_t wgs = int64_t(device_cu_count()) * per_cu;
    const int64_t gx = groups < wgs ? groups : wgs;
    a.wave_slots = int(gx > 0 ? gx : 1) * kWavesPerBlock;
    const int64_t cus = device_cu_count();
    a.level_waves = int(gx > 0 ? (gx < cus ? gx : cus) : 1) * kWavesPerBlock;
    hipLaunchKernelGGL((decode_generic_kernel<KVT, DP, GC, HQ>), dim3(unsigned(gx > 0 ? gx : 1)),
                       dim3(kBlockThreads), lds, st, a);
}

// fp16 queries over an fp16 cache take the packed-dot variant.
template <int KVT, int DP, int GC>
void launch_variant(DecodeArgs& a, int64_t max_pairs, size_t lds, hipStream_t st) {
    if constexpr (KVT == kF16) {
        if (!a.io_f32) {
            launch_variant_q<KVT, DP, GC, true>(a, max_pairs, lds, st);
            return;
        }
    }
    launch_variant_q<KVT, DP, GC, false>(a, max_pairs, lds, st);
}

template <int KVT, int DP>
void launch_dp(DecodeArgs& a, int G, int64_t max_pairs, size_t lds, hipStream_t st) {
    // Query-head chunk: the group rounded up to a power of two, at most 8
    // (4 when a lane holds 16 elements per head).
    constexpr int kMaxGc = GenericShape<KVT, DP, 8>::NV * GenericShape<KVT, DP, 8>::EPV > 8 ? 4 : 8;
    if (G <= 1) launch_variant<KVT, DP, 1>(a, max_pairs, lds, st);
    else if (G <= 2) launch_variant<KVT, DP, 2>(a, max_pairs, lds, st);
    else if (G <= 4 || kMaxGc == 4) launch_variant<KVT, DP, 4>(a, max_pairs, lds, st);
    else launch_variant<KVT, DP, kMaxGc>(a, max_pairs, lds, st);
}

template <int KVT>
int launch_kvt(DecodeArgs& a, int D, int G, int64_t max_pairs, size_t lds, hipStream_t st) {
    if (D <= 64) launch_dp<KVT, 64>(a, G, max_pairs, lds, st);
    else if (D <= 128) launch_dp<KVT, 128>(a, G, max_pairs, lds, st);
    else if (D <= 256) launch_dp<KVT, 256>(a, G, max_pairs, lds, st);
    else if (D <= 512) launch_dp<KVT, 512>(a, G, max_pairs, lds, st);
    else if (D <= kMaxGenericDim) launch_dp<KVT, kMaxGenericDim>(a, G, max_pairs, lds, st);
    else return VKV_ERR_UNSUPPORTED;
    return 0;
}

}  // namespace

int launch_decode_generic(DecodeArgs& a, int kv_dtype, int64_t max_pairs, size_t lds, hipStream_t st) {
    const int G = a.num_heads / a.num_kv_heads;
    switch (kv_dtype) {
        case VKV_DTYPE_F32: return launch_kvt<kF32>(a, a.head_dim, G, max_pairs, lds, st);
        case VKV_DTYPE_F16: return launch_kvt<kF16>(a, a.head_dim, G, max_pairs, lds, st);
        case VKV_DTYPE_FP8_E4M3: return launch_kvt<kFp8>(a, a.head_dim, G, max_pairs, lds, st);
        default: return VKV_ERR_UNSUPPORTED;
    }
}

}  // namespace dec
}  // namespace vkv
