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
// Single pass per item (online softmax): each chunk of CH = U*TPL tokens
// issues its K and V loads together (2U independent loads per lane, 8 KiB per
// wave for D=128 fp16), computes the chunk's logits, raises the running max
// (rescaling the accumulators only when it grows, a wave-uniform branch), then
// accumulates p * V in fp32.  No LDS is used, so occupancy is bounded by VGPRs
// alone and any partition size works.  The partial (o, max, sum) of the item
// goes to the workspace; a second kernel merges the partitions of every
// (sequence, head) with the usual log-sum-exp rescale.  Logits live in the
// log2 domain (scale * log2 e folded into the scale).
//
// FP8 lanes load 8 bytes (8 codes) so that fp8 and fp16 share one lane layout
// (D=128: 16 lanes per token) and one register footprint.
#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <type_traits>

#include "common.hpp"
#include "decode_common.hpp"
#include "launch.hpp"

namespace vkv {
namespace {

using namespace dec;

// Loads per lane per chunk for group sizes <= 4 (half that above): 8 keeps
// 16 KiB of K/V in flight per wave at D=128 fp16.  Build-time tuning knob.
#ifndef VKV_DECODE_UNROLL
#define VKV_DECODE_UNROLL 4
#endif
constexpr int kUnroll = VKV_DECODE_UNROLL;
// Register budget: at least this many waves per SIMD (3 -> at most 168 VGPRs).
#ifndef VKV_DECODE_MIN_WAVES
#define VKV_DECODE_MIN_WAVES 3
#endif
constexpr int kMinWavesPerSimd = VKV_DECODE_MIN_WAVES;
// MFMA variant: FP8 groups above kOneChunkAboveGFp8 heads load one 16-token
// chunk per step instead of two (their chunks carry scales); fp16 groups above
// kOneChunkAboveG heads keep two chunks at a lower occupancy target.
// Build-time tuning knobs.
#ifndef VKV_DECODE_ONE_CHUNK_ABOVE_G
#define VKV_DECODE_ONE_CHUNK_ABOVE_G 6
#endif
#ifndef VKV_DECODE_ONE_CHUNK_ABOVE_G_FP8
#define VKV_DECODE_ONE_CHUNK_ABOVE_G_FP8 3
#endif
constexpr int kOneChunkAboveG = VKV_DECODE_ONE_CHUNK_ABOVE_G;
constexpr int kOneChunkAboveGFp8 = VKV_DECODE_ONE_CHUNK_ABOVE_G_FP8;
// Default partition sizing aims at this many (row, partition, kv head) items.
constexpr int64_t kMinItems = 2048;
// Small batches stop splitting before a row could have more partitions than this.
constexpr int64_t kMaxSplitParts = 64;
// Per-call partition choice (library default only).  Candidates relative to
// the default size P0 (block multiples, at most 64 blocks): 3/4, 7/8, 1, 5/4,
// 5/3, 2 x P0 (at P0 = 768: 576, 672, 768, 960, 1 280 and 1 536 tokens with
// 32-token blocks; with 16-token blocks the last two are both 1 024).  The
// sizes below P0 let a batch whose items almost fill a whole
// number of waves per SIMD take shorter partitions that keep that number.
// Six, because the counts per candidate take registers in the kernels'
// prologue: with ten, the compiler reloaded a kernel argument and added a
// load wait inside the partition kernels' token loop (C5's batch: 354 us
// against 343 us at the same partition size).  Calls over more rows than
// kAdaptMaxRows keep P0.
constexpr int kCandNum[kMaxPartitionCandidates] = {3, 7, 1, 5, 5, 2};
constexpr int kCandDen[kMaxPartitionCandidates] = {4, 8, 1, 4, 3, 1};
// When the 64-block cap merges candidates (at 16-token blocks and P0 = 768,
// 5/3 and 2 x P0 are both 1 024), the freed slots take these, in order: 55/64,
// 15/16, 13/16 x P0 (656, 720, 624 tokens there).  C2's batch then takes 656
// (2 016 items, still two waves per SIMD): 97.1 us explicit against 98.0 at
// 672.
constexpr int kFillCandidates = 3;
constexpr int kFillNum[kFillCandidates] = {55, 15, 13};
constexpr int kFillDen[kFillCandidates] = {64, 16, 16};
constexpr int kAdaptMaxRows = 4096;

// One work item: partition `part` of row s (a sequence, or a prefill query
// row) for kv head kvh, computed by the calling wave alone.  Writes the
// item's partial (o, max, sum) to the workspace.
template <typename IO, int KVT, int D, int G, bool STATIC = false>
__device__ __forceinline__ void decode_item(const DecodeArgs& a, const int P, const int s, const int kvh,
                                            const int part, const int lane) {
    constexpr int EB = KvTraits<KVT>::bytes;
    constexpr int LW = LaneLoad<KVT>::words;
    constexpr int EPL = LaneLoad<KVT>::elems;  // elements per lane per load
    constexpr int LPT = D / EPL;               // lanes per token
    constexpr int TPL = kWave / LPT;           // tokens per wave-wide load
    constexpr int U = G <= 4 ? kUnroll : kUnroll / 2;  // loads per lane per chunk, for K and for V
    constexpr int CH = U * TPL;                // tokens per chunk
    // fp16 query against fp16 or fp8 keys: packed fp16 dot products (v_dot2_f32_f16).
    constexpr bool HALF_DOT = std::is_same<IO, _Float16>::value && KVT != kF32;
    static_assert(LPT >= 1 && LPT <= kWave && (kWave % LPT) == 0, "head_dim / dtype mapping");

    const int seq = a.row_seq ? a.row_seq[s] : s;
    const int t0 = part * P;
    // Static (small) calls are bound by their chain of dependent loads: the
    // table entries the partition could use are requested before the context
    // length is known (P / block_size <= 64; entries past the row's table are
    // not read), and those past the context are then dropped.
    constexpr bool early_table = STATIC;
    int my_block = 0;
    if constexpr (early_table) {
        const int tb = t0 >> a.bs_log2;
        const int nb_max = a.max_blocks_per_seq - tb < (P >> a.bs_log2) ? a.max_blocks_per_seq - tb : (P >> a.bs_log2);
        if (lane < nb_max) my_block = a.bt[int64_t(seq) * a.max_blocks_per_seq + tb + lane];
    }
    const int ctx = row_context(a, s);
    if (t0 >= ctx) return;
    const int n = (ctx - t0) < P ? (ctx - t0) : P;

    const int sub = lane % LPT;  // which slice of the head vector
    const int grp = lane / LPT;  // which token of a wave-wide load
    const int bs_mask = (1 << a.bs_log2) - 1;
    // A wave-wide load never straddles a block when block_size >= TPL: then
    // its block id is wave-uniform and comes from one readlane.
    const bool load_in_block = (1 << a.bs_log2) >= TPL;

    // Physical block ids of this partition, one per lane (P / block_size <= 64).
    const int nb = (n + bs_mask) >> a.bs_log2;
    if constexpr (early_table) {
        if (lane >= nb || (a.num_blocks > 0 && unsigned(my_block) >= unsigned(a.num_blocks))) my_block = 0;
    } else if (lane < nb) {
        my_block = a.bt[int64_t(seq) * a.max_blocks_per_seq + (t0 >> a.bs_log2) + lane];
        if (a.num_blocks > 0 && unsigned(my_block) >= unsigned(a.num_blocks)) my_block = 0;
    }

    // Query slices of the G heads.
    const int h0 = kvh * G;
    const char* qbase = static_cast<const char*>(a.q) +
                        (query_row(a, s) * a.q_stride + int64_t(h0) * D + sub * EPL) * int64_t(sizeof(IO));
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
            for (int e = 0; e < EPL; ++e) qf[h][e] = static_cast<float>(qp[e]);
        }
    }

    // The max is tracked on raw dots, which needs a positive scale: a negative
    // one is moved into the query (exact sign flip).
    const bool neg_scale = a.scale_log2 < 0.0f;
    if (neg_scale) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
#pragma unroll
            for (int i = 0; i < QW; ++i) qh[h][i] ^= 0x80008000u;
#pragma unroll
            for (int e = 0; e < QF; ++e) qf[h][e] = -qf[h][e];
        }
    }

    // Byte offsets: slots are slot_stride apart, blocks block_stride apart.  A
    // lane's offset inside a chunk is fixed (its token row and head slice), so
    // full chunks address K/V as (wave-uniform block base) + (32-bit lane offset).
    const uint32_t slot_stride = uint32_t(a.num_kv_heads) * D * EB;
    const int64_t block_stride = int64_t(slot_stride) << a.bs_log2;
    const uint32_t lane_off = uint32_t(grp) * slot_stride + uint32_t(kvh * D + sub * EPL) * EB;
    // Running max m is kept on raw dot products (fp8: times the key scale);
    // sc turns raw values into log2-domain logits inside the exp2 argument.
    float sc = neg_scale ? -a.scale_log2 : a.scale_log2;
    if constexpr (KVT == kFp8) sc *= kFp8HalfScale;
    // fp16 V: p * V as packed dot products over token pairs, weights rounded to fp16.
    constexpr bool PAIR_PV = HALF_DOT && KVT == kF16 && (U % 2) == 0;

    float m[G], l[G], acc[G][EPL];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        m[h] = -INFINITY;
        l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[h][e] = 0.0f;
    }

    // Registers of one chunk of CH tokens: K and V lane loads (plus FP8 scales).
    struct ChunkRegs {
        uint32_t k[U][LW];
        uint32_t v[U][LW];
        float ks[U];
        float vs[U];
    };

    // Issue the loads of the chunk starting at token c.  TAIL: the last,
    // partly valid chunk (masked); other chunks carry no validity checks.
    auto load_chunk = [&](ChunkRegs& b, const int c, auto) __attribute__((always_inline)) {
        if (load_in_block) {
            // Each wave-wide load covers TPL consecutive tokens of one block, so
            // its base address is wave-uniform (scalar) and every lane adds the
            // same 32-bit offset: no per-load vector address arithmetic.
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int tu = c + u * TPL;
                const int blk = __builtin_amdgcn_readlane(my_block, (tu >> a.bs_log2) & 63);
                const int64_t boff = int64_t(blk) * block_stride + int64_t(tu & bs_mask) * slot_stride;
                load_lane<KVT>(a.kc + boff + lane_off, b.k[u]);
                load_lane<KVT>(a.vc + boff + lane_off, b.v[u]);
                if constexpr (KVT == kFp8) {
                    const int64_t si = ((int64_t(blk) << a.bs_log2) + (tu & bs_mask) + grp) * a.num_kv_heads + kvh;
                    b.ks[u] = a.ks[si];
                    b.vs[u] = a.vs[si] * kFp8HalfScale;
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int tok = c + u * TPL + grp;
                const int blk = __shfl(my_block, (tok >> a.bs_log2) & 63, kWave);
                const int64_t slot = (int64_t(blk) << a.bs_log2) + (tok & bs_mask);
                const int64_t off = slot * slot_stride + (lane_off - uint32_t(grp) * slot_stride);
                load_lane<KVT>(a.kc + off, b.k[u]);
                load_lane<KVT>(a.vc + off, b.v[u]);
                if constexpr (KVT == kFp8) {
                    b.ks[u] = a.ks[slot * a.num_kv_heads + kvh];
                    b.vs[u] = a.vs[slot * a.num_kv_heads + kvh] * kFp8HalfScale;
                }
            }
        }
    };

    // Consume a loaded chunk: logits, running max, weights, p * V.
    auto compute_chunk = [&](const ChunkRegs& b_in, auto tail_tag, const int c = 0) __attribute__((always_inline)) {
        constexpr bool TAIL = decltype(tail_tag)::value;
        // In the last chunk, tokens at or past n are masked: their logit is
        // -inf, their weight 0 and their V zero (whatever the memory held).
        bool valid[U];
        ChunkRegs b = b_in;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            valid[u] = !TAIL || (c + u * TPL + grp < n);
            if constexpr (TAIL) {
#pragma unroll
                for (int w = 0; w < LW; ++w) b.v[u][w] = valid[u] ? b.v[u][w] : 0u;
                if constexpr (KVT == kFp8) b.vs[u] = valid[u] ? b.vs[u] : 0.0f;
            }
        }
        // raw dot products of the chunk, complete in every lane of a token group
        float r[U][G];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float x[G];
            if constexpr (HALF_DOT) {
#pragma unroll
                for (int h = 0; h < G; ++h) x[h] = 0.0f;
                if constexpr (KVT == kF16) {
#pragma unroll
                    for (int i = 0; i < LW; ++i) {
                        const half2_t kk = as_half2(b.k[u][i]);
#pragma unroll
                        for (int h = 0; h < G; ++h) x[h] = dot2(as_half2(qh[h][i]), kk, x[h]);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < LW; ++i) {
                        uint32_t lo, hi;
                        fp8x4_to_half2x2_scaled(b.k[u][i], lo, hi);
#pragma unroll
                        for (int h = 0; h < G; ++h) {
                            x[h] = dot2(as_half2(qh[h][2 * i]), as_half2(lo), x[h]);
                            x[h] = dot2(as_half2(qh[h][2 * i + 1]), as_half2(hi), x[h]);
                        }
                    }
                }
            } else {
                float kv[EPL];
                unpack_lane<KVT>(b.k[u], kv);
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    float t = 0.0f;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) t = fmaf(qf[h][e], kv[e], t);
                    x[h] = t;
                }
            }
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float y = group_sum<LPT>(x[h]);
                if constexpr (KVT == kFp8) y *= b.ks[u];
                r[u][h] = (TAIL && !valid[u]) ? -INFINITY : y;
            }
        }

        // running max: rescale only when it grows (the value is wave-uniform)
        float msc[G];
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float cm = r[0][h];
#pragma unroll
            for (int u = 1; u < U; ++u) cm = fmaxf(cm, r[u][h]);
            cm = cross_group_max<LPT>(cm);
            if (cm > m[h]) {
                const float alpha = __builtin_amdgcn_exp2f((m[h] - cm) * sc);
                m[h] = cm;
                l[h] *= alpha;
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[h][e] *= alpha;
            }
            msc[h] = m[h] * sc;
        }

        // weights p = exp2(r * sc - m * sc); masked tokens weigh exactly 0
        float p[U][G];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float e2 = __builtin_amdgcn_exp2f(fmaf(r[u][h], sc, -msc[h]));
                p[u][h] = (TAIL && !valid[u]) ? 0.0f : e2;
            }

        if constexpr (PAIR_PV) {
            const half2_t ones = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
#pragma unroll
            for (int u = 0; u < U; u += 2) {
                half2_t pp[G];
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    pp[h] = half2_t{static_cast<_Float16>(p[u][h]), static_cast<_Float16>(p[u + 1][h])};
                    l[h] = dot2(pp[h], ones, l[h]);
                }
#pragma unroll
                for (int i = 0; i < LW; ++i) {
                    // (dim 2i of token u, of token u+1) and (dim 2i+1 of both)
                    const uint32_t lo = __builtin_amdgcn_perm(b.v[u + 1][i], b.v[u][i], 0x05040100u);
                    const uint32_t hi = __builtin_amdgcn_perm(b.v[u + 1][i], b.v[u][i], 0x07060302u);
#pragma unroll
                    for (int h = 0; h < G; ++h) {
                        acc[h][2 * i] = dot2(pp[h], as_half2(lo), acc[h][2 * i]);
                        acc[h][2 * i + 1] = dot2(pp[h], as_half2(hi), acc[h][2 * i + 1]);
                    }
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                float v[EPL];
                unpack_lane<KVT>(b.v[u], v);
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    l[h] += p[u][h];
                    float w = p[u][h];
                    if constexpr (KVT == kFp8) w *= b.vs[u];
#pragma unroll
                    for (int e = 0; e < EPL; ++e) acc[h][e] = fmaf(w, v[e], acc[h][e]);
                }
            }
        }
    };

    // Chunks in order; each chunk's loads are issued together and consumed
    // before the next chunk's.  Loads are never masked: every address is
    // valid (block ids past the partition are 0), so the steady-state loop
    // has no branches; only the last chunk masks tokens past n (and zeroes
    // their V).
    const int nc = (n + CH - 1) / CH;
    for (int i = 0; i + 1 < nc; ++i) {
        ChunkRegs b;
        load_chunk(b, i * CH, std::false_type{});
        compute_chunk(b, std::false_type{});
    }
    {
        ChunkRegs b;
        load_chunk(b, (nc - 1) * CH, std::false_type{});
        if constexpr (KVT == kF16 || KVT == kF32) {
            // Fused append: the row's last position reads the new token's
            // rows when the append targets that position's slot.
            if (a.fkey && t0 + n == ctx) {
                const int c = (nc - 1) * CH, pn = n - 1;
                const int pblk = __builtin_amdgcn_readlane(my_block, (pn >> a.bs_log2) & 63);
                const int64_t pslot = (int64_t(pblk) << a.bs_log2) + (pn & bs_mask);
                if (int64_t(a.fslots[s]) == pslot) {
                    uint32_t kw[LW], vw[LW];
                    load_lane<KVT>(a.fkey + s * a.fkey_stride + (kvh * D + sub * EPL) * EB, kw);
                    load_lane<KVT>(a.fval + s * a.fval_stride + (kvh * D + sub * EPL) * EB, vw);
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        if (c + u * TPL + grp == pn) {
#pragma unroll
                            for (int w = 0; w < LW; ++w) {
                                b.k[u][w] = kw[w];
                                b.v[u][w] = vw[w];
                            }
                        }
                    }
                }
            }
        }
        if ((n % CH) != 0) compute_chunk(b, std::true_type{}, (nc - 1) * CH);
        else compute_chunk(b, std::false_type{});
    }

#pragma unroll
    for (int h = 0; h < G; ++h) {
        l[h] = cross_group_sum<LPT>(l[h]);
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[h][e] = cross_group_sum<LPT>(acc[h][e]);
    }

    // ---------------- partial result
    if (grp == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const int64_t item = ((int64_t(s) * a.num_kv_heads + kvh) * a.max_parts + part) * G + h;
            float* o = a.part_o + item * D + sub * EPL;
#pragma unroll
            for (int e = 0; e < EPL; e += 4) {
                u32x4 w4;
#pragma unroll
                for (int k = 0; k < 4; ++k) w4[k] = as_u32(acc[h][e + k]);
                store16(o + e, w4);
            }
            if (sub == 0) {
                a.part_ml[item * 2] = m[h] * sc;  // log2-domain max, as the merge expects
                a.part_ml[item * 2 + 1] = l[h];
            }
        }
    }
}

// MFMA variant of one work item, for fp16 queries over fp16 or FP8 caches with
// D = 128 and block_size a multiple of 16.  A chunk is 16 tokens of one block.
//   QK^T on the matrix cores (v_mfma_f32_16x16x32_f16, 4 per chunk): rows =
//   the chunk's 16 tokens (A operand = K, lane l holds token l%16 and 8 dims
//   chosen by l/16 and the MFMA index), columns = query heads (B operand = Q,
//   head l%16 of the group, zero for l%16 >= G, its dims in the same order).
//   The accumulator gives lane l the logits of head l%16 for tokens
//   4(l/16)..+3.  fp16 K: lane l loads dims 32i + 8(l/16) for MFMA i.  FP8 K:
//   lane l loads 16 codes, dims 32(l/16) + 16j (two loads), feeding MFMAs 2j
//   and 2j+1; codes are converted exactly to fp16 (v_cvt_scalef32_pk_f16_fp8,
//   scale 1) and the token's scale multiplies the logit.
//   Softmax on that layout (running max per head, lanes sharing l%16 agree),
//   probabilities through a 16 x G slice of LDS to the V layout, and p * V as
//   packed fp16 dot products over token pairs (lane l: token 4u + l/16, dims
//   8(l%16)..+7), as in the VALU variant; FP8 V scales are folded into p.
// This moves the 128 VALU instructions of the per-token dot products and their
// cross-lane sums per chunk onto the matrix pipe.
template <int G, int KVT>
__device__ __forceinline__ void decode_item_mfma(const DecodeArgs& a, const int P, const int s, const int kvh,
                                                 const int part, const int lane, float* plds) {
    constexpr int D = 128;
    constexpr int CH = 16;
    constexpr bool FP8 = KVT == kFp8;
    constexpr int EB = FP8 ? 1 : 2;
    typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
    typedef float float4_t __attribute__((ext_vector_type(4)));
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    static_assert(G <= 16, "group size must fit the 16 MFMA columns");

    const int seq = a.row_seq ? a.row_seq[s] : s;
    const int ctx = row_context(a, s);
    const int t0 = part * P;
    if (t0 >= ctx) return;
    const int n = (ctx - t0) < P ? (ctx - t0) : P;
    const int bs_mask = (1 << a.bs_log2) - 1;
    const int col = lane & 15;  // MFMA column (query head) / V dim slice
    const int quad = lane >> 4; // MFMA k-slice / accumulator row group / V token in a load

    const int nb = (n + bs_mask) >> a.bs_log2;
    int my_block = 0;
    if (lane < nb) {
        my_block = a.bt[int64_t(seq) * a.max_blocks_per_seq + (t0 >> a.bs_log2) + lane];
        if (a.num_blocks > 0 && unsigned(my_block) >= unsigned(a.num_blocks)) my_block = 0;
    }

    // Q as the B operand; a negative scale is moved into Q (exact sign flip).
    // Loads are unconditional (head h0 stands in for the unused columns, which
    // are then zeroed) so that they overlap instead of each being awaited.
    const int h0 = kvh * G;
    const bool neg_scale = a.scale_log2 < 0.0f;
    const uint32_t qkeep = col < G ? 0xFFFFFFFFu : 0u;
    const uint32_t qflip = neg_scale ? 0x80008000u : 0u;
    const char* qrow = static_cast<const char*>(a.q) +
                       (query_row(a, s) * a.q_stride + int64_t(h0 + (col < G ? col : 0)) * D) * 2;
    half8_t qb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // dims of MFMA i: fp16 32i + 8 quad; FP8 32 quad + 16 (i / 2) + 8 (i % 2)
        const int d0 = FP8 ? 32 * quad + 16 * (i >> 1) + 8 * (i & 1) : 32 * i + 8 * quad;
        u32x4 w = load16(qrow + d0 * 2);
        w = (w ^ u32x4{qflip, qflip, qflip, qflip}) & u32x4{qkeep, qkeep, qkeep, qkeep};
        qb[i] = __builtin_bit_cast(half8_t, w);
    }
    const float sc = neg_scale ? -a.scale_log2 : a.scale_log2;

    const uint32_t slot_stride = uint32_t(a.num_kv_heads) * D * EB;
    const int64_t block_stride = int64_t(slot_stride) << a.bs_log2;
    const uint32_t koff = FP8 ? uint32_t(col) * slot_stride + uint32_t(kvh * D + 32 * quad)
                              : uint32_t(col) * slot_stride + uint32_t(kvh * D + 8 * quad) * 2;
    const uint32_t voff = uint32_t(quad) * slot_stride + uint32_t(kvh * D + 8 * col) * EB;

    float m = -INFINITY;  // running max of this lane's head (col), raw units
    float l = 0.0f;       // this lane's share of the head's weight sum
    float acc[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;

    struct Chunk {
        u32x4 k[FP8 ? 2 : 4];
        u32x4 v[FP8 ? 1 : 4];
        u32x2 v8[FP8 ? 4 : 1];
        // FP8: one scale per lane (lanes 0-15: K scale of token l, lanes
        // 16-31: V scale of token l - 16), shuffled to the lanes that use it;
        // after compute starts, ks/vs hold the per-lane values.
        float sc1;
        float ks[FP8 ? 4 : 1];  // scales of tokens 4 quad + k
        float vs[FP8 ? 4 : 1];  // scales of tokens 4 u + quad
    };
    // Issue the K (A-operand layout) and V (row layout) loads of the 16 tokens
    // at c.  Addresses are always valid (block ids past the partition are 0).
    auto load_chunk = [&](Chunk& ch, const int c) __attribute__((always_inline)) {
        const int blk = __builtin_amdgcn_readlane(my_block, (c >> a.bs_log2) & 63);
        const int64_t boff = int64_t(blk) * block_stride + int64_t(c & bs_mask) * slot_stride;
        const char* kb = a.kc + boff;
        const char* vb = a.vc + boff;
        // K lines are read in two halves by different instructions: ordinary
        // loads keep the line for the second half; V rows stream (non-temporal).
        if constexpr (FP8) {
#pragma unroll
            for (int j = 0; j < 2; ++j) ch.k[j] = load16(kb + koff + 16 * j);
#pragma unroll
            for (int u = 0; u < 4; ++u)
                ch.v8[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(vb + voff + u * 4 * slot_stride));
            const int64_t sbase = ((int64_t(blk) << a.bs_log2) + (c & bs_mask)) * a.num_kv_heads + kvh;
            ch.sc1 = ((lane & 16) ? a.vs : a.ks)[sbase + int64_t(col) * a.num_kv_heads];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) ch.k[i] = load16(kb + koff + 64 * i);
#pragma unroll
            for (int u = 0; u < 4; ++u) ch.v[u] = load16_nt(vb + voff + u * 4 * slot_stride);
        }
    };

    auto compute_chunk = [&](Chunk& ch, const int c, auto tail_tag) __attribute__((always_inline)) {
        constexpr bool TAIL = decltype(tail_tag)::value;
        u32x4* vr = ch.v;  // (fp16 only)
        float4_t cc = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (FP8) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t c0 = ch.k[i >> 1][2 * (i & 1)], c1 = ch.k[i >> 1][2 * (i & 1) + 1];
                const u32x4 w = {fp8x2_to_half2<false>(c0), fp8x2_to_half2<true>(c0), fp8x2_to_half2<false>(c1),
                                 fp8x2_to_half2<true>(c1)};
                cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, w), qb[i], cc, 0, 0, 0);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                ch.ks[k] = __shfl(ch.sc1, 4 * quad + k, kWave);
                ch.vs[k] = __shfl(ch.sc1, 16 + 4 * k + quad, kWave);
                cc[k] *= ch.ks[k];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, ch.k[i]), qb[i], cc, 0, 0, 0);
        }
        float r[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) r[k] = (TAIL && c + 4 * quad + k >= n) ? -INFINITY : cc[k];
        if constexpr (TAIL) {
            // past n: V zero and (FP8) scale zero, whatever the slots hold
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (c + 4 * u + quad >= n) {
                    if constexpr (FP8) {
                        ch.v8[u] = u32x2{0u, 0u};  // code 0 widens to +0
                        ch.vs[u] = 0.0f;
                    } else {
                        vr[u] = u32x4{0u, 0u, 0u, 0u};
                    }
                }
            }
        }

        // running max per head: lanes sharing col hold the same value after the exchange
        float cm = fmaxf(fmaxf(r[0], r[1]), fmaxf(r[2], r[3]));
        // (FP8 chunks keep the exchange on the LDS permute: their VALU is the
        // busier pipe, and the VALU swaps measured C5 1 % slower)
        if constexpr (FP8) cm = fmaxf(cm, __shfl_xor(cm, 16, kWave)), cm = fmaxf(cm, __shfl_xor(cm, 32, kWave));
        else cm = xor_max<32>(xor_max<16>(cm));
        const bool grow = cm > m;
        if (__builtin_amdgcn_ballot_w64(grow && col < G)) {
            const float alpha = grow ? __builtin_amdgcn_exp2f((m - cm) * sc) : 1.0f;
            if (grow) m = cm;
            l *= alpha;
#pragma unroll
            for (int h = 0; h < G; ++h) {
                // lane h holds column (head) h
                const float ah = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), h));
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h][e] *= ah;
            }
        }
        const float msc = m * sc;
        float pr[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            pr[k] = __builtin_amdgcn_exp2f(fmaf(r[k], sc, -msc));
            if (TAIL && c + 4 * quad + k >= n) pr[k] = 0.0f;
        }
        // weights to LDS as [token][head]; the sum uses the fp16-rounded values
        // that the p * V products use
        if (col < G) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float pk = static_cast<float>(static_cast<_Float16>(pr[k]));
                l += pk;
                plds[(4 * quad + k) * G + col] = pk;
            }
        }
        wave_lds_sync();
#pragma unroll
        for (int u = 0; u < 4; u += 2) {
            half2_t pp[G];
            const float v0 = FP8 ? ch.vs[u] : 1.0f;
            const float v1 = FP8 ? ch.vs[u + 1] : 1.0f;
#pragma unroll
            for (int h = 0; h < G; ++h)
                pp[h] = half2_t{static_cast<_Float16>(plds[(4 * u + quad) * G + h] * v0),
                                static_cast<_Float16>(plds[(4 * (u + 1) + quad) * G + h] * v1)};
            u32x4 va, vb;
            if constexpr (!FP8) {
                va = vr[u];
                vb = vr[u + 1];
            } else {
                // the two tokens' codes as fp16 in dim order: (b0, b1), (b2, b3)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    va[2 * h] = fp8x2_to_half2<false>(ch.v8[u][h]);
                    va[2 * h + 1] = fp8x2_to_half2<true>(ch.v8[u][h]);
                    vb[2 * h] = fp8x2_to_half2<false>(ch.v8[u + 1][h]);
                    vb[2 * h + 1] = fp8x2_to_half2<true>(ch.v8[u + 1][h]);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo = __builtin_amdgcn_perm(vb[i], va[i], 0x05040100u);
                const uint32_t hi = __builtin_amdgcn_perm(vb[i], va[i], 0x07060302u);
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    acc[h][2 * i] = dot2(pp[h], as_half2(lo), acc[h][2 * i]);
                    acc[h][2 * i + 1] = dot2(pp[h], as_half2(hi), acc[h][2 * i + 1]);
                }
            }
        }
        wave_lds_sync();
    };

    // Two chunks (32 tokens, 16 KiB of K/V per wave at D=128 fp16) are loaded
    // before either is computed, doubling the bytes in flight per wave.  FP8
    // groups above 3 heads (their chunks carry scales) load one chunk at a
    // time so that the 8 G accumulators per lane fit without spilling.
    const int nc = (n + CH - 1) / CH;
    const bool ragged = (n % CH) != 0;
    // Fused append (fp16): the row's last position reads the new token's rows
    // when the append targets that position's slot.  Applied to the last
    // chunk right after its loads are issued.
    auto fuse_last = [&](Chunk& ch, const int c) __attribute__((always_inline)) {
        if constexpr (!FP8) {
            if (a.fkey && t0 + n == ctx) {
                const int pn = n - 1;
                const int pblk = __builtin_amdgcn_readlane(my_block, (pn >> a.bs_log2) & 63);
                const int64_t pslot = (int64_t(pblk) << a.bs_log2) + (pn & bs_mask);
                if (int64_t(a.fslots[s]) == pslot) {
                    const char* kr = a.fkey + s * a.fkey_stride + kvh * D * 2;
                    const char* vr = a.fval + s * a.fval_stride + kvh * D * 2;
                    // K: lane (col, quad) holds token c + col, dims 32 i + 8 quad
                    if (c + col == pn) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) ch.k[i] = load16(kr + (32 * i + 8 * quad) * 2);
                    }
                    // V: load u holds token c + 4 u + quad, dims 8 col..+7
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (c + 4 * u + quad == pn) ch.v[u] = load16(vr + 8 * col * 2);
                }
            }
        }
    };
    int ci = 0;
    if constexpr (FP8 && G > kOneChunkAboveGFp8) {
        for (; ci + 1 < nc; ++ci) {
            Chunk x;
            load_chunk(x, ci * CH);
            compute_chunk(x, ci * CH, std::false_type{});
        }
        Chunk x;
        load_chunk(x, ci * CH);
        if (ragged) compute_chunk(x, ci * CH, std::true_type{});
        else compute_chunk(x, ci * CH, std::false_type{});
    } else {
    for (; ci + 2 < nc; ci += 2) {
        Chunk x, y;
        load_chunk(x, ci * CH);
        load_chunk(y, (ci + 1) * CH);
        compute_chunk(x, ci * CH, std::false_type{});
        compute_chunk(y, (ci + 1) * CH, std::false_type{});
    }
    if (ci + 1 < nc) {
        Chunk x, y;
        load_chunk(x, ci * CH);
        load_chunk(y, (ci + 1) * CH);
        fuse_last(y, (ci + 1) * CH);
        compute_chunk(x, ci * CH, std::false_type{});
        if (ragged) compute_chunk(y, (ci + 1) * CH, std::true_type{});
        else compute_chunk(y, (ci + 1) * CH, std::false_type{});
    } else {
        Chunk x;
        load_chunk(x, ci * CH);
        fuse_last(x, ci * CH);
        if (ragged) compute_chunk(x, ci * CH, std::true_type{});
        else compute_chunk(x, ci * CH, std::false_type{});
    }
    }

    // head sums: lanes sharing col; accumulators: lanes sharing col (token groups)
    l = xor_add<32>(xor_add<16>(l));
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = cross_group_sum<16>(acc[h][e]);

    if (quad == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const int64_t item = ((int64_t(s) * a.num_kv_heads + kvh) * a.max_parts + part) * G + h;
            float* o = a.part_o + item * D + col * 8;
            store16(o, u32x4{as_u32(acc[h][0]), as_u32(acc[h][1]), as_u32(acc[h][2]), as_u32(acc[h][3])});
            store16(o + 4, u32x4{as_u32(acc[h][4]), as_u32(acc[h][5]), as_u32(acc[h][6]), as_u32(acc[h][7])});
        }
        if (col < G) {
            const int64_t item = ((int64_t(s) * a.num_kv_heads + kvh) * a.max_parts + part) * G + col;
            a.part_ml[item * 2] = m * sc;
            a.part_ml[item * 2 + 1] = l;
        }
    }
}

// Persistent partition kernel (the item loop of decode_common.hpp) whose
// items are (row, partition, kv head), kv head fastest.
// Register budget per instantiation: the fp16 matrix-core variant with 7-8
// heads per group keeps two chunks in flight at 2 waves per SIMD (measured
// faster than one chunk at 3), and FP8 groups of 7-8 fit their one chunk
// without spilling at 2; everything else targets kMinWavesPerSimd.
template <int KVT, int G, bool MFMA>
constexpr int min_waves_per_simd() {
    return (MFMA && ((KVT == kF16 && G > kOneChunkAboveG) || (KVT == kFp8 && G > 6))) ? 2 : kMinWavesPerSimd;
}

// STATIC: the small-call variant (a static grid, static_parts > 0).
template <typename IO, int KVT, int D, int G, bool MFMA, bool STATIC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(min_waves_per_simd<KVT, G, MFMA>())))
void decode_partition_kernel(const DecodeArgs a) {
    __shared__ float plds[MFMA ? kWavesPerBlock : 1][MFMA ? 16 * G : 1];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    // (matrix-core items are dealt, VALU ones claimed: run_partitions)
    run_partitions<STATIC, MFMA>(a, a.num_kv_heads, [&](const int P, const int row, const int part, const int kvh)
                                                  __attribute__((always_inline)) {
        if constexpr (MFMA) decode_item_mfma<G, KVT>(a, P, row, kvh, part, lane, plds[wave]);
        else decode_item<IO, KVT, D, G, STATIC>(a, P, row, kvh, part, lane);
    });
}

// Fused append: the merge kernel (after every read of the call) stores
// elements [d, d + E) of row s's new K and V rows for kv head kvh (elements of
// a.fbytes bytes), unless the slot lies outside the pool (the plain append
// skips those slots too).
template <int E>
__device__ __forceinline__ void store_new_token(const DecodeArgs& a, const int s, const int kvh, const int d,
                                                const int D) {
    const int64_t slot = a.fslots[s];
    if (slot < 0 || slot >= a.fnum_slots) return;
    const int64_t eb = a.fbytes;
    const int64_t dst = ((slot * a.num_kv_heads + kvh) * D + d) * eb;
    const char* kr = a.fkey + s * a.fkey_stride + (int64_t(kvh) * D + d) * eb;
    const char* vr = a.fval + s * a.fval_stride + (int64_t(kvh) * D + d) * eb;
    char* kc = const_cast<char*>(a.kc) + dst;
    char* vc = const_cast<char*>(a.vc) + dst;
    if (E * eb % 4 == 0) {
        // E fp16 (E even) or E fp32 elements as 32-bit words
        const int words = int(E * eb / 4);
#pragma unroll
        for (int w = 0; w < 2 * E; ++w) {
            if (w < words) {
                reinterpret_cast<uint32_t*>(kc)[w] = reinterpret_cast<const uint32_t*>(kr)[w];
                reinterpret_cast<uint32_t*>(vc)[w] = reinterpret_cast<const uint32_t*>(vr)[w];
            }
        }
    } else {
        // one fp16 element
        *reinterpret_cast<uint16_t*>(kc) = *reinterpret_cast<const uint16_t*>(kr);
        *reinterpret_cast<uint16_t*>(vc) = *reinterpret_cast<const uint16_t*>(vr);
    }
}

// Merge the partitions of one (sequence, head): one thread per output element.
// The kernel is latency-bound (a few KiB per workgroup), so the partials of
// the first kMergeBatch partitions are loaded together with the context length,
// before the partition count is known: slots past the count are in the
// workspace (max_parts per row) and their stale contents are masked out.
// Longer rows continue in batches with a running max.
// DT = 0: head_dim from the arguments (the generic variant), one thread per
// element of a block of head_dim rounded up to 64 threads.  B: partitions per
// batch, chosen by the host (8; up to 64 for small calls split finely, such
// as C1's 33 partitions of 16 tokens, which then load all their partials in
// one round).
template <typename IO, int DT, int B>
__global__ __launch_bounds__(DT ? DT : 1024) void decode_reduce_kernel(DecodeArgs a) {
    constexpr int kMergeBatch = B;
    const int s = blockIdx.y;
    const int h = blockIdx.x;
    const int d = threadIdx.x;
    // The partition kernel has finished (same stream): return its claim
    // counters to zero for the next call.
    if (s == 0 && h == 0 && d < kClaimSequences) a.counters[d * kCounterStride] = 0;
    const int D = DT ? DT : a.head_dim;
    if (DT == 0 && d >= D) return;
    const int G = a.num_heads / a.num_kv_heads;
    const int kvh = h / G;
    if (a.fkey && h == kvh * G) store_new_token<1>(a, s, kvh, d, D);
    const int64_t slot0 = (int64_t(s) * a.num_kv_heads + kvh) * a.max_parts * G + (h - kvh * G);
    const float* ml = a.part_ml + slot0 * 2;
    const float* o = a.part_o + slot0 * D + d;
    float bm[kMergeBatch], bl[kMergeBatch], bo[kMergeBatch];
    auto load_batch = [&](int i0) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < kMergeBatch; ++k) {
            const int i = i0 + k < a.max_parts ? i0 + k : a.max_parts - 1;  // in-bounds slot
            bm[k] = ml[int64_t(i) * G * 2];
            bl[k] = ml[int64_t(i) * G * 2 + 1];
            bo[k] = o[int64_t(i) * G * D];
        }
    };
    // A prefill sequence of a mixed call is not decoded here: leave before
    // loading its (stale) partial slots, which a call without single-token
    // rows would otherwise read for every (sequence, head).
    if (a.qsl && a.qsl[s + 1] - a.qsl[s] != 1) return;
    load_batch(0);
    const int ctx = row_context(a, s);
    const int P = a.num_cands > 1 ? __builtin_amdgcn_readfirstlane(a.counters[kChosenPartitionSlot]) : a.P;
    const int np = ctx > 0 ? (ctx + P - 1) / P : 0;
    float m = -INFINITY, l = 0.0f, acc = 0.0f;
    for (int i0 = 0; i0 < np; i0 += kMergeBatch) {
        if (i0 > 0) load_batch(i0);
        float bmax = -INFINITY;
#pragma unroll
        for (int k = 0; k < kMergeBatch; ++k)
            if (i0 + k < np) bmax = fmaxf(bmax, bm[k]);
        const float mn = fmaxf(m, bmax);
        const float alpha = __builtin_amdgcn_exp2f(m - mn);  // 0 on the first batch
        l *= alpha;
        acc *= alpha;
#pragma unroll
        for (int k = 0; k < kMergeBatch; ++k) {
            if (i0 + k < np) {
                const float w = __builtin_amdgcn_exp2f(bm[k] - mn);
                l = fmaf(w, bl[k], l);
                acc = fmaf(w, bo[k], acc);
            }
        }
        m = mn;
    }
    const float r0 = np > 0 ? acc / l : 0.0f;
    IO* out = static_cast<IO*>(a.out) + (query_row(a, s) * a.num_heads + h) * D + d;
    const float r = a.accumulate ? r0 + static_cast<float>(*out) : r0;
    *out = static_cast<IO>(r);
}

// Building with -DVKV_DECODE_MFMA=0 selects the VALU QK^T variant everywhere
// (an A/B switch for measurements; the shipped library uses matrix cores).
#ifndef VKV_DECODE_MFMA
#define VKV_DECODE_MFMA 1
#endif
constexpr int mfma_enabled() { return VKV_DECODE_MFMA; }

template <typename IO, int KVT, int D, int G>
void launch_g(DecodeArgs& args, int grid_x, int grid_y, int grid_z, size_t lds, hipStream_t st) {
    // Matrix-core QK^T for fp16 query and keys at D = 128 with blocks of a
    // multiple of 16 tokens; the VALU variant covers everything else.
    constexpr bool kMfmaShape = std::is_same<IO, _Float16>::value && KVT != kF32 && D == 128;
    // grid_x arrives as the number of item groups (an upper bound).  One workgroup per resident slot: the variant's workgroups per CU by
    // registers (queried once per variant), bounded by the LDS the rows'
    // prefix takes, and never more than there are item groups.  Groups
    // beyond the grid are claimed through the counters as workgroups finish
    // (each workgroup scans the rows once, where a grid of every group pays
    // that scan per group: C5's batch measured 361 us against 382 us).  The
    // resident wave count also feeds the partition choice.
    // Static small-call variants exist for fp16 queries (the serving case).
    constexpr bool kStatic = std::is_same<IO, _Float16>::value;
    static std::atomic<int> reg_blocks[2];
    auto run = [&](auto kernel, auto static_kernel, int variant) {
        const int cus = device_cu_count();
        int per_cu = reg_blocks[variant].load(std::memory_order_relaxed);
        if (per_cu <= 0) {
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kWave * kWavesPerBlock, 0) !=
                    hipSuccess || per_cu <= 0)
                per_cu = 1;
            reg_blocks[variant].store(per_cu, std::memory_order_relaxed);
        }
        const int by_lds = kLdsPerCu / int(lds + 4096);  // + an allowance for the static LDS
        if (by_lds < per_cu) per_cu = by_lds > 0 ? by_lds : 1;
        per_cu = blocks_per_cu(per_cu);
        const int64_t wgs = int64_t(cus) * per_cu;
        int gx = int(wgs < grid_x ? wgs : grid_x);
        if (!kStatic) args.static_parts = 0;
        if (args.static_parts > 0) {
            // one item per wave, all resident at once, or the claim loop
            const int64_t groups = (int64_t(args.num_rows) * args.static_parts * args.num_kv_heads +
                                    kWavesPerBlock - 1) / kWavesPerBlock;
            if (groups <= wgs) {
                gx = int(groups);
                args.num_cands = 1;
            } else {
                args.static_parts = 0;
            }
        }
        args.wave_slots = (gx > 0 ? gx : 1) * kWavesPerBlock;
        args.level_waves = (gx > 0 ? (gx < cus ? gx : cus) : 1) * kWavesPerBlock;
        // When even the longest possible contexts give at most one wave of
        // default-size items per SIMD, the default stands and the kernels
        // (this one and the merge, which reads these args) skip the choice.
        if (args.num_cands > 1 && args.static_parts == 0) {
            const int64_t worst = int64_t(args.num_rows) * ((int64_t(args.max_ctx) + args.P - 1) / args.P) *
                                  args.num_kv_heads;
            if (worst <= args.level_waves) args.num_cands = 1;
        }
        if (args.static_parts > 0)
            hipLaunchKernelGGL(static_kernel, dim3(gx > 0 ? gx : 1, grid_y, grid_z), dim3(kBlockThreads), lds, st, args);
        else
            hipLaunchKernelGGL(kernel, dim3(gx > 0 ? gx : 1, grid_y, grid_z), dim3(kBlockThreads), lds, st, args);
    };
    if (kMfmaShape && args.bs_log2 >= 4 && args.mfma_enabled)
        run(decode_partition_kernel<IO, KVT, D, G, kMfmaShape, false>,
            decode_partition_kernel<IO, KVT, D, G, kMfmaShape, kStatic>, 1);
    else
        run(decode_partition_kernel<IO, KVT, D, G, false, false>, decode_partition_kernel<IO, KVT, D, G, false, kStatic>, 0);
}


template <typename IO, int KVT, int D>
int dispatch_g(int G, DecodeArgs& args, int grid_x, int Hkv, int S, size_t lds, hipStream_t st) {
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
int dispatch_d(int D, int G, DecodeArgs& args, int grid_x, int Hkv, int S, size_t lds,
               hipStream_t st) {
    switch (D) {
        case 64: return dispatch_g<IO, KVT, 64>(G, args, grid_x, Hkv, S, lds, st);
        case 128: return dispatch_g<IO, KVT, 128>(G, args, grid_x, Hkv, S, lds, st);
        case 256: return dispatch_g<IO, KVT, 256>(G, args, grid_x, Hkv, S, lds, st);
        default: return VKV_ERR_UNSUPPORTED;
    }
}

// The same merge at head_dim DT = 128 or 256 with one wave per (sequence,
// head) and E = DT / 64 consecutive elements per lane: measured C2 0.2-0.4 us
// and C5 1-2 us faster than a thread per element (at DT = 64 a thread per
// element is one wave already, and stays).  The wave reads the context length
// first and then loads only the row's own partials: measured C2 0.4-0.8 us and
// C5 1-1.5 us faster than loading the first B slots beside the context length
// (their bytes, twice the partials' at C5, cost more than the round trip).
template <typename IO, int DT, int B>
__global__ __launch_bounds__(kWave) void decode_reduce_wave_kernel(DecodeArgs a) {
    constexpr int E = DT / kWave;
    static_assert(E == 2 || E == 4, "head_dim 128 or 256");
    typedef float fE __attribute__((ext_vector_type(E)));
    const int s = blockIdx.y;
    const int h = blockIdx.x;
    const int d = int(threadIdx.x) * E;
    if (s == 0 && h == 0 && threadIdx.x < kClaimSequences) a.counters[threadIdx.x * kCounterStride] = 0;
    const int G = a.num_heads / a.num_kv_heads;
    const int kvh = h / G;
    if (a.fkey && h == kvh * G) store_new_token<E>(a, s, kvh, d, DT);
    const int64_t slot0 = (int64_t(s) * a.num_kv_heads + kvh) * a.max_parts * G + (h - kvh * G);
    const float* ml = a.part_ml + slot0 * 2;
    const float* o = a.part_o + slot0 * DT + d;
    if (a.qsl && a.qsl[s + 1] - a.qsl[s] != 1) return;
    const int ctx = row_context(a, s);
    const int P = a.num_cands > 1 ? __builtin_amdgcn_readfirstlane(a.counters[kChosenPartitionSlot]) : a.P;
    const int np = ctx > 0 ? (ctx + P - 1) / P : 0;
    // partials of batch i0 (slots past np are neither loaded nor read)
    float bm[B], bl[B];
    fE bo[B];
    auto load_batch = [&](int i0) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < B; ++k) {
            if (i0 + k < np) {
                bm[k] = ml[int64_t(i0 + k) * G * 2];
                bl[k] = ml[int64_t(i0 + k) * G * 2 + 1];
                bo[k] = *reinterpret_cast<const fE*>(o + int64_t(i0 + k) * G * DT);
            }
        }
    };
    load_batch(0);
    float m = -INFINITY, l = 0.0f;
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = 0.0f;
    for (int i0 = 0; i0 < np; i0 += B) {
        if (i0 > 0) load_batch(i0);
        float bmax = -INFINITY;
#pragma unroll
        for (int k = 0; k < B; ++k)
            if (i0 + k < np) bmax = fmaxf(bmax, bm[k]);
        const float mn = fmaxf(m, bmax);
        const float alpha = __builtin_amdgcn_exp2f(m - mn);  // 0 on the first batch
        l *= alpha;
#pragma unroll
        for (int e = 0; e < E; ++e) acc[e] *= alpha;
#pragma unroll
        for (int k = 0; k < B; ++k) {
            if (i0 + k < np) {
                const float w = __builtin_amdgcn_exp2f(bm[k] - mn);
                l = fmaf(w, bl[k], l);
#pragma unroll
                for (int e = 0; e < E; ++e) acc[e] = fmaf(w, bo[k][e], acc[e]);
            }
        }
        m = mn;
    }
    IO* out = static_cast<IO*>(a.out) + (query_row(a, s) * a.num_heads + h) * DT + d;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float r0 = np > 0 ? acc[e] / l : 0.0f;
        const float r = a.accumulate ? r0 + static_cast<float>(out[e]) : r0;
        out[e] = static_cast<IO>(r);
    }
}

template <typename IO, int B>
int launch_reduce_b(int D, const DecodeArgs& args, int H, int S, hipStream_t st) {
    switch (D) {
        case 64: hipLaunchKernelGGL((decode_reduce_kernel<IO, 64, B>), dim3(H, S), dim3(64), 0, st, args); return 0;
        case 128: hipLaunchKernelGGL((decode_reduce_wave_kernel<IO, 128, B>), dim3(H, S), dim3(kWave), 0, st, args); return 0;
        case 256: hipLaunchKernelGGL((decode_reduce_wave_kernel<IO, 256, B>), dim3(H, S), dim3(kWave), 0, st, args); return 0;
        default:
            if (D < 1 || D > 1024) return VKV_ERR_UNSUPPORTED;
            hipLaunchKernelGGL((decode_reduce_kernel<IO, 0, B>), dim3(H, S), dim3((D + 63) / 64 * 64), 0, st, args);
            return 0;
    }
}

template <typename IO>
int launch_reduce(int D, const DecodeArgs& args, int H, int S, hipStream_t st) {
    // Small (static) calls split finely load every partial in one round;
    // the others keep batches of 8 (their rows have few partitions, and
    // wider batches measured slower at C2's batch).
    if (args.static_parts == 0 || args.max_parts <= 8) return launch_reduce_b<IO, 8>(D, args, H, S, st);
    if (args.max_parts <= 16) return launch_reduce_b<IO, 16>(D, args, H, S, st);
    if (args.max_parts <= 32) return launch_reduce_b<IO, 32>(D, args, H, S, st);
    return launch_reduce_b<IO, 64>(D, args, H, S, st);
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
    int64_t max_ctx = p->max_context_len;
    const int64_t table_tokens = int64_t(p->max_blocks_per_seq) * bs;
    if (max_ctx > table_tokens) max_ctx = table_tokens;
    if (max_ctx < 0) max_ctx = 0;
    // Default 768 tokens: the best of a 384..1024 sweep for both the C2
    // (B=64, ctx U[512,4096]) and C5 (B=256, lognormal ctx) decode batches.
    // Small batches split finer (halving, not below 16 tokens, then down to a
    // block multiple) until the longest possible contexts would give kMinItems
    // work items, or a row more than kMaxSplitParts partitions: a wave walks
    // its partition serially, so 8 items of 512 tokens (C1) leave the GPU idle
    // while short items finish together (C1's decode: 15.3 us at 48 tokens,
    // 14.2 at 32, 13.9 at 16, 32.8 at 256), but the merge walks a row's
    // partitions in batches, one after the other (one sequence of 4 096
    // tokens: 29.6 us at 16 tokens, 19.7 at 32, 16.5 at 64 and 128).
    int P = p->partition_size > 0 ? p->partition_size : 768;
    if (p->partition_size <= 0) {
        const int64_t per_part = int64_t(p->num_seqs) * p->num_kv_heads;
        while (P / 2 >= 16 && per_part * ((max_ctx + P - 1) / P) < kMinItems &&
               (max_ctx + P / 2 - 1) / (P / 2) <= kMaxSplitParts)
            P /= 2;
    }
    // A partition starts on a block boundary and holds at most 64 blocks
    // (one block id per lane).
    if (P < bs) P = bs;
    P = (P / bs) * bs;
    if (P > 64 * bs) P = 64 * bs;
    plan.partition_size = P;
    plan.num_candidates = 1;
    for (int i = 0; i < kMaxPartitionCandidates; ++i) plan.candidates[i] = P;
    int smallest = P;
    const bool fixed = fixed_decode_shape(p->head_dim, p->num_heads / p->num_kv_heads, bs, p->key_cache,
                                          p->value_cache);
    if (p->partition_size <= 0 && p->num_seqs <= kAdaptMaxRows && fixed) {
        // the kernels pick the size per call among these (ascending)
        auto block_multiple = [&](int num, int den) {
            const int c = (P * num / den) / bs * bs;
            return c < bs ? bs : (c > 64 * bs ? 64 * bs : c);
        };
        int n = 0;
        for (int i = 0; i < kMaxPartitionCandidates; ++i) {
            const int c = block_multiple(kCandNum[i], kCandDen[i]);
            if (n == 0 || c != plan.candidates[n - 1]) plan.candidates[n++] = c;
        }
        // Slots freed by the 64-block cap take finer sizes just below the default.
        for (int i = 0; i < kFillCandidates && n < kMaxPartitionCandidates; ++i) {
            const int c = block_multiple(kFillNum[i], kFillDen[i]);
            int at = 0;
            while (at < n && plan.candidates[at] < c) ++at;
            if (at < n && plan.candidates[at] == c) continue;
            for (int j = n; j > at; --j) plan.candidates[j] = plan.candidates[j - 1];
            plan.candidates[at] = c;
            ++n;
        }
        for (int i = n; i < kMaxPartitionCandidates; ++i) plan.candidates[i] = plan.candidates[n - 1];
        plan.num_candidates = n;
        smallest = plan.candidates[0];
    }
    plan.max_parts = int((max_ctx + smallest - 1) / smallest);
    if (plan.max_parts < 1) plan.max_parts = 1;
    plan.workspace_bytes = kWorkspaceHeader + size_t(launch_rows_max(p->num_seqs)) * p->num_heads * plan.max_parts *
                                                  (p->head_dim + 2) * sizeof(float);
    return plan;
}

// Query row r of a prefill step: its sequence and the number of keys it sees
// (the reference's prefill is one decode per position, src/core/engine.cpp:157-164).
__global__ __launch_bounds__(kBlockThreads) void prefill_rows_kernel(const int32_t* qsl, const int32_t* cl, int32_t num_seqs,
                                                           int32_t rows, int32_t max_ctx, int32_t* row_seq,
                                                           int32_t* row_ctx) {
    const int r = blockIdx.x * kBlockThreads + threadIdx.x;
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
                const int32_t* row_ctx, const int32_t* qsl, hipStream_t st, const FusedAppend* fa = nullptr) {
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
    a.qsl = qsl;
    const int rows = launch_rows_max(p->num_seqs);
    const size_t o_elems = size_t(rows) * p->num_heads * plan.max_parts * p->head_dim;
    a.counters = static_cast<int*>(workspace);
    a.part_o = reinterpret_cast<float*>(static_cast<char*>(workspace) + kWorkspaceHeader);
    a.part_ml = a.part_o + o_elems;
    a.mfma_enabled = mfma_enabled();
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
    a.num_cands = plan.num_candidates;
    for (int i = 0; i < kMaxPartitionCandidates; ++i) a.cands[i] = plan.candidates[i];
    a.wave_slots = 0;  // set per variant at launch
    a.level_waves = 0;
    a.scale_log2 = logit_scale_log2(p->scale);
    a.accumulate = p->accumulate;
    a.static_parts = 0;
    a.fkey = fa ? fa->key : nullptr;
    a.fval = fa ? fa->value : nullptr;
    a.fkey_stride = fa ? fa->key_stride : 0;
    a.fval_stride = fa ? fa->value_stride : 0;
    a.fbytes = fa ? fa->elem_bytes : 0;
    a.fslots = fa ? fa->slots : nullptr;
    a.fnum_slots = fa ? fa->num_slots : 0;

    const int G = p->num_heads / p->num_kv_heads;
    const int D = p->head_dim;
    const int io_eb = p->io_dtype == VKV_DTYPE_F32 ? 4 : 2;
    const bool fixed = fixed_decode_shape(D, G, p->block_size, p->key_cache, p->value_cache);
    a.head_dim = D;
    a.block_size = p->block_size;
    set_block_div(a, p->block_size);
    a.io_f32 = p->io_dtype == VKV_DTYPE_F32;
    {
        const int kv_eb = p->kv_dtype == VKV_DTYPE_F32 ? 4 : (p->kv_dtype == VKV_DTYPE_F16 ? 2 : 1);
        const int vec_bytes = p->kv_dtype == VKV_DTYPE_FP8_E4M3 ? 8 : 16;
        const uintptr_t bases = reinterpret_cast<uintptr_t>(p->key_cache) | reinterpret_cast<uintptr_t>(p->value_cache);
        a.vec_loads = (int64_t(D) * kv_eb) % vec_bytes == 0 && (bases % uintptr_t(vec_bytes)) == 0;
    }
    // Consecutive ranges of at most kMaxRowsPerLaunch rows, each a partition
    // launch and a merge launch on the stream; the ranges reuse the partials.
    for (int r0 = 0; r0 < p->num_seqs; r0 += kMaxRowsPerLaunch) {
        const int n = p->num_seqs - r0 < kMaxRowsPerLaunch ? p->num_seqs - r0 : kMaxRowsPerLaunch;
        DecodeArgs c = a;
        c.num_rows = n;
        // Small plain decode calls (at most one (row, kv head) pair per CU):
        // a static grid over the partitions of the default size, if its waves
        // are all resident at once (decided at launch).
        if (fixed && !qsl && !row_seq && p->io_dtype == VKV_DTYPE_F16 &&
            int64_t(n) * p->num_kv_heads <= device_cu_count())
            c.static_parts = int32_t((int64_t(c.max_ctx) + c.P - 1) / c.P > 0 ? (int64_t(c.max_ctx) + c.P - 1) / c.P : 1);
        if (qsl) {
            // rows are sequences; their query rows (qsl values) stay absolute
            c.qsl = qsl + r0;
            c.cl = a.cl + r0;
            c.bt = a.bt + int64_t(r0) * p->max_blocks_per_seq;
        } else {
            c.q = static_cast<const char*>(a.q) + int64_t(r0) * a.q_stride * io_eb;
            c.out = static_cast<char*>(a.out) + int64_t(r0) * p->num_heads * D * io_eb;
            if (row_seq) {
                // rows are query tokens; their sequences index the tables
                c.row_seq = row_seq + r0;
                c.row_ctx = row_ctx + r0;
            } else {
                c.cl = a.cl + r0;
                c.bt = a.bt + int64_t(r0) * p->max_blocks_per_seq;
            }
            if (fa) {
                c.fkey = a.fkey + int64_t(r0) * a.fkey_stride;
                c.fval = a.fval + int64_t(r0) * a.fval_stride;
                c.fslots = a.fslots + r0;
            }
        }
        // Persistent grid (sized in launch_g from the kernel's occupancy), never
        // more workgroups than item groups.
        const int64_t max_items = int64_t(n) * plan.max_parts * p->num_kv_heads;
        int64_t item_wgs = (max_items + kWavesPerBlock - 1) / kWavesPerBlock;
        if (item_wgs > (int64_t(1) << 30)) item_wgs = int64_t(1) << 30;
        const int grid_x = int(item_wgs < 1 ? 1 : item_wgs);
        const size_t lds = (size_t(n) + 1) * sizeof(int) + lpt_lds_bytes(n);
        int rc;
        if (!fixed) {
            rc = launch_decode_generic(c, p->kv_dtype, int64_t(n) * plan.max_parts, lds, st);
            if (!rc) rc = p->io_dtype == VKV_DTYPE_F32 ? launch_reduce<float>(D, c, p->num_heads, n, st)
                                                       : launch_reduce<_Float16>(D, c, p->num_heads, n, st);
        } else if (p->io_dtype == VKV_DTYPE_F32) {
            switch (p->kv_dtype) {
                case VKV_DTYPE_F32: rc = dispatch_d<float, kF32>(D, G, c, grid_x, 1, 1, lds, st); break;
                case VKV_DTYPE_F16: rc = dispatch_d<float, kF16>(D, G, c, grid_x, 1, 1, lds, st); break;
                case VKV_DTYPE_FP8_E4M3: rc = dispatch_d<float, kFp8>(D, G, c, grid_x, 1, 1, lds, st); break;
                default: return VKV_ERR_UNSUPPORTED;
            }
            if (!rc) rc = launch_reduce<float>(D, c, p->num_heads, n, st);
        } else {
            switch (p->kv_dtype) {
                case VKV_DTYPE_F16: rc = dispatch_d<_Float16, kF16>(D, G, c, grid_x, 1, 1, lds, st); break;
                case VKV_DTYPE_FP8_E4M3: rc = dispatch_d<_Float16, kFp8>(D, G, c, grid_x, 1, 1, lds, st); break;
                default: return VKV_ERR_UNSUPPORTED;
            }
            if (!rc) rc = launch_reduce<_Float16>(D, c, p->num_heads, n, st);
        }
        if (rc) return rc;
    }
    return 0;
}

int launch_decode(const vkv_decode_params* p, const DecodePlan& plan, void* workspace, hipStream_t st) {
    return launch_rows(p, plan, workspace, nullptr, nullptr, nullptr, st);
}

bool decode_append_fusable(const vkv_append_params* ap, const vkv_decode_params* p) {
    const bool f16 = ap->src_dtype == VKV_DTYPE_F16 && ap->cache_dtype == VKV_DTYPE_F16;
    const bool f32 = ap->src_dtype == VKV_DTYPE_F32 && ap->cache_dtype == VKV_DTYPE_F32;
    const int64_t eb = f32 ? 4 : 2;
    const int64_t row = int64_t(ap->num_kv_heads) * ap->head_dim;
    const int64_t ks = (ap->key_stride ? ap->key_stride : row) * eb;
    const int64_t vs = (ap->value_stride ? ap->value_stride : row) * eb;
    const uintptr_t src = reinterpret_cast<uintptr_t>(ap->key) | reinterpret_cast<uintptr_t>(ap->value);
    return ap->num_tokens == p->num_seqs && p->num_seqs > 0 && ap->key_cache == p->key_cache &&
           ap->value_cache == p->value_cache && (f16 || f32) && p->kv_dtype == ap->cache_dtype &&
           ap->num_kv_heads == p->num_kv_heads && ap->head_dim == p->head_dim &&
           ap->block_size == p->block_size && ap->num_blocks == p->num_blocks && (src & 15u) == 0 &&
           ks % 16 == 0 && vs % 16 == 0 &&
           fixed_decode_shape(p->head_dim, p->num_heads / p->num_kv_heads, p->block_size, p->key_cache,
                              p->value_cache);
}

int launch_decode_append(const vkv_append_params* ap, const vkv_decode_params* p, const DecodePlan& plan,
                         void* workspace, hipStream_t st) {
    const int eb = ap->cache_dtype == VKV_DTYPE_F32 ? 4 : 2;
    const int64_t row = int64_t(ap->num_kv_heads) * ap->head_dim;
    FusedAppend fa;
    fa.key = static_cast<const char*>(ap->key);
    fa.value = static_cast<const char*>(ap->value);
    fa.key_stride = (ap->key_stride ? ap->key_stride : row) * eb;
    fa.value_stride = (ap->value_stride ? ap->value_stride : row) * eb;
    fa.elem_bytes = eb;
    fa.slots = ap->slot_mapping;
    fa.num_slots = int64_t(ap->num_blocks) * ap->block_size;
    return launch_rows(p, plan, workspace, nullptr, nullptr, nullptr, st, &fa);
}

// Decode parameters for the rows of a prefill call: one row per query token
// (row_map) or one per sequence (mixed batch, decoding the single-token ones).
vkv_decode_params prefill_as_decode(const vkv_prefill_params* p, bool per_sequence) {
    vkv_decode_params d{};
    d.output = p->output;
    d.query = p->query;
    d.key_cache = p->key_cache;
    d.value_cache = p->value_cache;
    d.key_scales = p->key_scales;
    d.value_scales = p->value_scales;
    d.block_tables = p->block_tables;
    d.context_lens = p->context_lens;
    d.query_stride = p->query_stride ? p->query_stride : int64_t(p->num_heads) * p->head_dim;
    d.num_seqs = per_sequence ? p->num_seqs : p->num_query_tokens;
    d.num_heads = p->num_heads;
    d.num_kv_heads = p->num_kv_heads;
    d.head_dim = p->head_dim;
    d.block_size = p->block_size;
    d.max_context_len = p->max_context_len > 0 ? p->max_context_len : 0x7FFFFFFF;
    d.max_blocks_per_seq = p->max_blocks_per_seq;
    d.num_blocks = p->num_blocks;
    d.scale = p->scale;
    d.io_dtype = p->io_dtype;
    d.kv_dtype = p->kv_dtype;
    d.accumulate = 0;
    return d;
}

DecodePlan plan_prefill(const vkv_prefill_params* p) {
    if (prefill_mfma_supported(p)) {
        // single-token sequences through split-K decode, one row per sequence
        const vkv_decode_params d = prefill_as_decode(p, true);
        DecodePlan plan = plan_decode(&d);
        // the matrix-core kernel's work list follows the partials
        plan.workspace_bytes = (plan.workspace_bytes + 255) / 256 * 256 + prefill_items_bytes(p);
        return plan;
    }
    const vkv_decode_params d = prefill_as_decode(p, false);
    DecodePlan plan = plan_decode(&d);
    // row_seq and row_ctx follow the partials
    plan.workspace_bytes += size_t(p->num_query_tokens) * 2 * sizeof(int32_t);
    return plan;
}

int launch_prefill(const vkv_prefill_params* p, const DecodePlan& plan, void* workspace, hipStream_t st) {
    if (prefill_mfma_supported(p)) {
        // Mixed batch: the matrix-core kernel takes every sequence with two or
        // more query tokens, the decode kernels the single-token ones; each
        // writes only its own output rows.  All on the caller's stream, one
        // after the other: the decode kernels on a side stream forked from it
        // and joined back were slower (C3's mixed call 339 us against 319 us,
        // its prefill rows alone 127 us against 105 us), and so was giving the
        // prefill kernel 64-192 of the 256 CUs with the decode rows beside it
        // on a side stream (333-348 us against 324 us): neither kernel's waves
        // fit beside the other's on a CU, and the decode rows need nearly every
        // CU to keep enough bytes in flight.
        const size_t items_off = plan.workspace_bytes - prefill_items_bytes(p);
        const vkv_decode_params d = prefill_as_decode(p, true);
        const int rc = launch_prefill_mfma(p, static_cast<char*>(workspace) + items_off, st);
        // (the caller's promise of no single-token sequence spares the decode
        // pass: its kernels cost ~9 us even when they find no row)
        if (rc || p->multi_token_only) return rc;
        return launch_rows(&d, plan, workspace, nullptr, nullptr, p->query_start_loc, st);
    }
    // Every query row decoded like a sequence of a decode call, each with its
    // causal context (the reference's prefill is one decode per position,
    // src/core/engine.cpp:157-164).
    const vkv_decode_params d = prefill_as_decode(p, false);
    const size_t partial_bytes = plan.workspace_bytes - size_t(p->num_query_tokens) * 2 * sizeof(int32_t);
    int32_t* row_seq = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + partial_bytes);
    int32_t* row_ctx = row_seq + p->num_query_tokens;
    int64_t max_keys = int64_t(p->max_blocks_per_seq) * p->block_size;
    if (p->max_context_len > 0 && p->max_context_len < max_keys) max_keys = p->max_context_len;
    const int32_t max_ctx = int32_t(max_keys > 0x7FFFFFFF ? 0x7FFFFFFF : max_keys);
    hipLaunchKernelGGL(prefill_rows_kernel, dim3((p->num_query_tokens + kBlockThreads - 1) / kBlockThreads),
                       dim3(kBlockThreads), 0, st,
                       p->query_start_loc, p->context_lens, p->num_seqs, p->num_query_tokens, max_ctx, row_seq,
                       row_ctx);
    return launch_rows(&d, plan, workspace, row_seq, row_ctx, nullptr, st);
}

}  // namespace vkv
