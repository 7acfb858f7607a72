// prefill.hip — causal chunked-prefill attention on the matrix cores (gfx950).
//
// Semantics follow the reference's prefill, which runs one decode per prompt
// position (src/core/engine.cpp:157-164 over src/attention/paged_attention.cu:13-82):
// query row j of a sequence with q_len new tokens and ctx keys (context_lens,
// this step's tokens included) attends keys 0 .. ctx - q_len + j of the
// sequence's paged cache, i.e. causal attention over the prior context plus
// the chunk.  Keys are gathered through the block table like decode.
//
// The kernels share the matrix-core layout below: prefill_w64_kernel (fp16
// caches at head_dim 128) and prefill_wide_kernel (fp16 caches at head_dim 64
// with groups below 4 heads): work items of (token, head) rows, tiles staged
// by direct global->LDS loads; prefill_wide8_kernel for FP8 caches at head_dim
// 128 (the same, with the code tiles converted to fp16 in LDS once per
// workgroup); prefill_mfma_kernel for the rest of head_dim 64.  In the last a
// workgroup owns (sequence, kv head, block of kBQ = 32 query tokens); wave w
// computes query head kvh * G + w for those 32 tokens as two 16-row MFMA
// tiles, so the G heads that share a kv head share every K/V tile staged in
// LDS.  In both, keys are staged kBK = 64 at a time and computed in 32-key
// steps:
//   S^T = K Q^T   v_mfma_f32_16x16x32_f16, A = K rows (LDS), B = Q (registers);
//                 lane l holds row (query token) l % 16 for keys 4 (l / 16) + e
//                 of each 16-key half: softmax state (max, sum) is lane-local
//                 per row after a two-step exchange across the lane groups.
//   O^T += V^T P^T  A = V^T, read from row-major V with ds_read_b64_tr_b16,
//                 B = P^T straight from the S^T registers (the MFMA k index
//                 runs over keys in the order the S^T layout holds them), so P
//                 never leaves the wave.
// The output tile is O^T, again one row per lane, normalised at the end.
//
// Staging of FP8 caches (prefill_mfma_kernel): each of the first 256 threads
// loads its share of the next tile's K and V rows into registers while the
// current tile is computed, then writes them row-major into LDS (rows padded
// by 16 bytes to spread the banks), dequantised on the way (code x per-token
// scale, fp32 -> fp16).  Block ids of the sequence are cached in LDS, 1024 at
// a time.
#include <algorithm>
#include <functional>
#include <queue>
#include <utility>
#include <type_traits>
#include <vector>

#include "common.hpp"
#include "launch.hpp"

// Building with -DVKV_PREFILL_W64=0 runs fp16 caches at head_dim 128 on the
// 8-wave kernel instead of the one-wave-per-SIMD kernel (an A/B switch).
#ifndef VKV_PREFILL_W64
#define VKV_PREFILL_W64 1
#endif
// Building with -DVKV_PREFILL_D64_WIDE=1 runs fp16 caches at head_dim 64 on
// the 8-wave direct-load kernel for every group size (an A/B switch; by
// default groups of 4 and more take the register-staged kernel).
#ifndef VKV_PREFILL_D64_WIDE
#define VKV_PREFILL_D64_WIDE 0
#endif

namespace vkv {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBQ = 32;        // query tokens per workgroup
constexpr int kRT = kBQ / 16;  // 16-row MFMA tiles per wave
constexpr int kBK = 64;        // keys staged per tile (computed 32 at a time)
constexpr int kMaxWaves = 8;   // heads per workgroup (more: grid.z splits the group)
constexpr int kMinWaves = 4;   // staging always has >= 256 threads
constexpr int kBtCache = 1024; // block ids cached in LDS at a time

struct PrefillArgs {
    _Float16* out;
    const char* q;
    const char* kc;
    const char* vc;
    const float* ks;
    const float* vs;
    const int32_t* bt;
    const int32_t* cl;
    const int32_t* qsl;
    int64_t q_stride;  // elements between query rows
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t group;  // G = H / Hkv
    int32_t heads_per_wg;
    int32_t bs_log2;
    int32_t max_blocks_per_seq;
    int32_t num_blocks;
    int32_t table_tokens;
    int32_t qblocks;  // row blocks per sequence, at most (bounds the number of items)
    int32_t num_seqs;
    const int2* items;       // work list (s, b * Hkv + kvh), b the sequence's row block
    int32_t* item_count;     // [0] items, [1 + z] claim counter of head group z (zeroed by the list kernel)
    float scale_log2;
    // direct-load kernels, calls of at most kInlineBlocks row blocks: every
    // workgroup orders the blocks itself (no list kernel)
    int32_t inline_list;
    int32_t rows_per_item;
    int32_t nbins;
    // host-built schedule (vkv_prefill_work_list_host), or nullptr
    const int32_t* work_list;
    int32_t work_list_words;  // its length (bounds every index read from it)
    int32_t num_query_tokens;
    // division by the group size G: n / G = (n + mulhi(n, m)) >> s for 0 <= n < 2^31
    uint32_t group_div_m;
    int32_t group_div_s;
};

// The query token of row rho (rows are (token, head) pairs, token-major).
__device__ __forceinline__ int row_token(const PrefillArgs& a, const int rho) {
    return int((uint32_t(rho) + __umulhi(uint32_t(rho), a.group_div_m)) >> a.group_div_s);
}

// One work item: row block b of sequence s at kv head kvh, with the
// sequence's first query row q0, its query length and its prior context
// (context length - query length).
struct PrefillItem {
    int s, b, kvh, q0, qlen, prior;
};

template <int D, int KVT>
struct Stage {
    static constexpr int EB = KvTraits<KVT>::bytes;
    static constexpr int COLS = D / 8;                // 8-dim columns per token row
    static constexpr int UNITS = kBK * COLS;          // (key, column) units of a K or V tile
    static constexpr int UPT = UNITS / (64 * kMinWaves);  // units per staging thread
    static constexpr int STR = D * 2 + 16;            // bytes per K or V row in LDS
    static_assert(UNITS % (64 * kMinWaves) == 0, "a tile must split evenly over 256 threads");
    // fp16: the 16 loaded bytes; FP8: 8 code bytes in .xy and the token's scale
    // (bits) in .z, dequantised only when written to LDS so that the loads stay
    // in flight while the current tile is computed.
    u32x4 k[UPT];
    u32x4 v[UPT];
};

// Eight elements of one token as loaded: 16 fp16 bytes, or 8 FP8 code bytes
// with the token's scale beside them.
template <int KVT>
__device__ __forceinline__ u32x4 load8(const char* p, const float* scale) {
    if constexpr (KVT == kF16) {
        return load16_nt(p);
    } else {
        const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
        return u32x4{w[0], w[1], __builtin_bit_cast(uint32_t, *scale), 0u};
    }
}

// Eight fp16 values for LDS: fp16 bytes as they are, FP8 codes dequantised with
// the token's scale (code * scale in fp32, rounded to fp16).  The codes widen
// exactly to fp32 two at a time (gfx950's v_cvt_pk_f32_fp8, OCP e4m3fn).
template <int KVT>
__device__ __forceinline__ u32x4 to_half8(u32x4 raw) {
    if constexpr (KVT == kF16) {
        return raw;
    } else {
        typedef float float2_t __attribute__((ext_vector_type(2)));
        const float sc = as_f32(raw[2]);
        u32x4 r;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(int(raw[i]), false);  // b0, b1
            const float2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8(int(raw[i]), true);   // b2, b3
            const half2_t x0 = {static_cast<_Float16>(lo[0] * sc), static_cast<_Float16>(lo[1] * sc)};
            const half2_t x1 = {static_cast<_Float16>(hi[0] * sc), static_cast<_Float16>(hi[1] * sc)};
            r[2 * i] = __builtin_bit_cast(uint32_t, x0);
            r[2 * i + 1] = __builtin_bit_cast(uint32_t, x1);
        }
        return r;
    }
}

// Max over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four key groups of one query
// row): gfx950's permlane swaps exchange rows of 16 lanes (xor 16) and wave
// halves (xor 32) on the VALU; swapping a value with itself leaves both
// partners' values, one in each result.
__device__ __forceinline__ float row_group_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(as_u32(x), as_u32(x), false, false);
    x = fmaxf(as_f32(a[0]), as_f32(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(as_u32(x), as_u32(x), false, false);
    return fmaxf(as_f32(b[0]), as_f32(b[1]));
}

constexpr float kLazy = 8.0f;  // rescale threshold of the running max, log2 units

// ds_read_b64_tr_b16: 8 bytes per lane, transposed across 16-lane groups.
__device__ __forceinline__ u32x2 tr_read(const char* lds) {
    typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
    typedef __attribute__((address_space(3))) fp16x4_t* lds_ptr;
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_ptr)(lds)));
}

// One work item: query block qb (kBQ tokens) of sequence s against kv head kvh.
template <int D, int KVT>
__device__ __forceinline__ void prefill_block(const PrefillArgs& a, const int s, const int qb, const int kvh,
                                              char* klds, char* vlds, int* btc) {
    using St = Stage<D, KVT>;
    constexpr int EB = St::EB;
    constexpr int kTileBytes = kBK * St::STR;  // one K (or V) tile buffer in LDS
    constexpr int DT = D / 16;  // output dim tiles
    constexpr int KS = D / 32;  // MFMA k-steps of Q K^T

    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col = lane & 15;   // query row within a 16-row tile
    const int grp = lane >> 4;   // key group: keys 4 grp .. 4 grp + 3 of a 16-key half
    const int g = blockIdx.z * a.heads_per_wg + wave;  // head within the GQA group
    const bool computes = wave < a.heads_per_wg && g < a.group;

    const int q0 = a.qsl[s];
    const int qlen = a.qsl[s + 1] - q0;
    if (qlen < 2 || qb * kBQ >= qlen) return;  // (the item list holds none of these)
    const int prior = a.cl[s] - qlen;
    const int jmax = min(qlen, qb * kBQ + kBQ);  // query rows j in [qb*kBQ, jmax)
    int kend = prior + jmax;                     // keys any row of the block may see
    kend = kend < a.table_tokens ? kend : a.table_tokens;
    const int ntiles = kend > 0 ? (kend + kBK - 1) / kBK : 0;
    const int h = kvh * a.group + g;

    // ---------------- Q (B operand of S^T = K Q^T) and per-row context
    const bool neg_scale = a.scale_log2 < 0.0f;
    const float sc = neg_scale ? -a.scale_log2 : a.scale_log2;
    half8_t qop[kRT][KS];
    int rctx[kRT];
#pragma unroll
    for (int r = 0; r < kRT; ++r) {
        const int j = qb * kBQ + 16 * r + col;
        int c = prior + j + 1;
        c = c < 0 ? 0 : (c > a.table_tokens ? a.table_tokens : c);
        rctx[r] = (j < qlen) ? c : 0;
#pragma unroll
        for (int i = 0; i < KS; ++i) {
            // Unconditional load (row 0 / head 0 stand in for absent rows, then
            // zeroed): a load under a branch makes the compiler wait for every
            // outstanding load before the first use of Q inside the key loop,
            // which would serialise the staging prefetch with the MFMAs.
            const bool ok = computes && j < qlen;
            const int64_t qrow = ok ? int64_t(q0) + j : int64_t(q0);
            const int64_t qcol = ok ? int64_t(h) * D : 0;
            u32x4 w = load16(a.q + (qrow * a.q_stride + qcol + 32 * i + 8 * grp) * 2);
            const uint32_t keep = ok ? 0xFFFFFFFFu : 0u;
            const uint32_t flip = neg_scale ? 0x80008000u : 0u;
            w = (w ^ u32x4{flip, flip, flip, flip}) & u32x4{keep, keep, keep, keep};
            qop[r][i] = __builtin_bit_cast(half8_t, w);
        }
    }

    // ---------------- staging
    const int bs_mask = (1 << a.bs_log2) - 1;
    const int64_t row_bytes = int64_t(a.num_kv_heads) * D * EB;  // one slot (token) of the cache
    const int32_t* table = a.bt + int64_t(s) * a.max_blocks_per_seq;
    int win = -1;  // first block id index held in btc
    auto ensure_window = [&](int first_block) __attribute__((always_inline)) {
        // uniform across the workgroup; callers are between barriers
        if (win < 0 || first_block < win || first_block + (kBK >> a.bs_log2) + 1 > win + kBtCache) {
            __syncthreads();
            win = first_block;
            for (int i = tid; i < kBtCache; i += nthr) {
                const int b = win + i;
                int id = 0;
                if (b < a.max_blocks_per_seq) {
                    id = table[b];
                    if (a.num_blocks > 0 && unsigned(id) >= unsigned(a.num_blocks)) id = 0;
                }
                btc[i] = id;
            }
            __syncthreads();
        }
    };
    // Keys past kend (the tail of the last tile) load the row of key kend - 1
    // instead: every query row masks them, so no branch is needed around the
    // loads and they all issue back to back.
    auto fetch = [&](St& st, int k0) __attribute__((always_inline)) {
        int64_t off[St::UPT];
#pragma unroll
        for (int i = 0; i < St::UPT; ++i) {
            const int u = tid + i * 64 * kMinWaves;
            int k = k0 + u / St::COLS;
            k = k < kend ? k : kend - 1;
            const int blk = btc[(k >> a.bs_log2) - win];
            off[i] = ((int64_t(blk) << a.bs_log2) + (k & bs_mask));  // slot
        }
#pragma unroll
        for (int i = 0; i < St::UPT; ++i) {
            const int c = (tid + i * 64 * kMinWaves) % St::COLS;
            const int64_t bytes = off[i] * row_bytes + int64_t(kvh) * D * EB + c * 8 * EB;
            const int64_t sidx = off[i] * a.num_kv_heads + kvh;
            st.k[i] = load8<KVT>(a.kc + bytes, KVT == kFp8 ? a.ks + sidx : nullptr);
            st.v[i] = load8<KVT>(a.vc + bytes, KVT == kFp8 ? a.vs + sidx : nullptr);
        }
    };
    auto put = [&](const St& st, char* kbuf, char* vbuf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < St::UPT; ++i) {
            const int u = tid + i * 64 * kMinWaves;
            const int off = (u / St::COLS) * St::STR + (u % St::COLS) * 16;
            store16(kbuf + off, to_half8<KVT>(st.k[i]));
            store16(vbuf + off, to_half8<KVT>(st.v[i]));
        }
    };

    // ---------------- main loop
    const float lazy = kLazy / sc;  // kLazy in raw (unscaled) logit units
    float m[kRT];
    float4_t lsum[kRT];  // row sums (every element the same), see below
    float4_t o[kRT][DT];
    const half8_t kOnes = {1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16};
#pragma unroll
    for (int r = 0; r < kRT; ++r) {
        m[r] = -INFINITY;
        lsum[r] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < DT; ++t) o[r][t] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }

    // Two LDS tile buffers and one staging register set: tile kt is computed
    // from buffer kt & 1 while the registers (tile kt + 1, loaded during the
    // previous tile) go to the other buffer and are refilled with tile kt + 2.
    // One barrier per tile: it publishes buffer (kt + 1) & 1, and every wave
    // has left tile kt - 1 (the previous user of that buffer) before it.
    St st;
    const bool stager = tid < 64 * kMinWaves;
    if (ntiles > 0) {
        ensure_window(0);
        if (stager) {
            fetch(st, 0);
            put(st, klds, vlds);
        }
        if (ntiles > 1) {
            ensure_window(kBK >> a.bs_log2);
            if (stager) fetch(st, kBK);
        }
        __syncthreads();
    }
    // One 32-key step in three parts, so that a tile's second S^T (matrix
    // pipe) is issued before the first step's softmax (VALU) and overlaps it.
    auto qk = [&](const char* kb, const int sub, float4_t (&sv)[kRT][2]) __attribute__((always_inline)) {
        // S^T of both row tiles; each K operand (one LDS read) feeds both.
#pragma unroll
        for (int r = 0; r < kRT; ++r) sv[r][0] = sv[r][1] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int i = 0; i < KS; ++i) {
                const half8_t kop = __builtin_bit_cast(
                    half8_t, *reinterpret_cast<const u32x4*>(kb + (32 * sub + 16 * hh + col) * St::STR + (32 * i + 8 * grp) * 2));
#pragma unroll
                for (int r = 0; r < kRT; ++r)
                    sv[r][hh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, qop[r][i], sv[r][hh], 0, 0, 0);
            }
    };
    auto softmax = [&](const int kbase, const float4_t (&sv)[kRT][2], half8_t (&pop)[kRT]) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < kRT; ++r) {
            // causal / context mask (key kbase + 16 hh + 4 grp + e < rctx), only
            // on tiles that reach past some row's context (wave-uniform test)
            float x[8];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int e = 0; e < 4; ++e) x[4 * hh + e] = sv[r][hh][e];
            if (__builtin_amdgcn_ballot_w64(kbase + 32 > rctx[r])) {
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (kbase + 16 * hh + 4 * grp + e >= rctx[r]) x[4 * hh + e] = -INFINITY;
            }
            float mx = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
            mx = row_group_max(mx);
            // Rescale only when some row's max exceeds the one in use by more
            // than kLazy (log2 units): below that the weights exp2((x - m) sc)
            // stay under 2^kLazy, well inside fp16 for P and fp32 for the sums,
            // and the result is the same softmax.  The first key always sets m.
            if (__builtin_amdgcn_ballot_w64(mx > m[r] + lazy)) {
                const float mn = fmaxf(m[r], mx);
                const float alpha = mn > m[r] ? __builtin_amdgcn_exp2f((m[r] - mn) * sc) : 1.0f;
                m[r] = mn;
                lsum[r] *= alpha;
#pragma unroll
                for (int t = 0; t < DT; ++t) o[r][t] *= alpha;
            }
            const float mref = m[r] == -INFINITY ? 0.0f : m[r];  // rows with no key yet
            const float msc = mref * sc;
            // P^T operand: k slot (grp, e) = key 4 grp + e, slot (grp, 4 + e) = key 16 + 4 grp + e
#pragma unroll
            for (int e = 0; e < 8; ++e) pop[r][e] = static_cast<_Float16>(__builtin_amdgcn_exp2f(fmaf(x[e], sc, -msc)));
            // row sums on the matrix pipe: a V^T tile of ones gives sum_k p in every lane
            lsum[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kOnes, pop[r], lsum[r], 0, 0, 0);
        }
    };
    auto pv = [&](const char* vb, const int sub, const half8_t (&pop)[kRT]) __attribute__((always_inline)) {
        // O^T += V^T P^T; each V^T operand (two transpose reads of row-major V:
        // within each 16-lane group, lane i receives element i % 4 of the 8-byte
        // chunks addressed by lanes i / 4 + 4 e, e = 0..3, so lane m of group
        // grp addresses key 4 grp + m / 4 (+16), dims 16 t + 4 (m % 4) .. +3)
        // feeds both row tiles.
        const int vrow = 32 * sub + 4 * grp + (col >> 2);
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            const int dcol = (16 * t + 4 * (col & 3)) * 2;
            const u32x2 lo = tr_read(vb + vrow * St::STR + dcol);
            const u32x2 hi = tr_read(vb + (16 + vrow) * St::STR + dcol);
            const half8_t vop = __builtin_bit_cast(half8_t, u32x4{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
            for (int r = 0; r < kRT; ++r) o[r][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, pop[r], o[r][t], 0, 0, 0);
        }
    };
    static_assert(kBK == 64, "the tile loop below computes two 32-key steps");
    for (int kt = 0; kt < ntiles; ++kt) {
        const char* kcur = klds + (kt & 1) * kTileBytes;
        const char* vcur = vlds + (kt & 1) * kTileBytes;
        if (computes) {
            const bool second = kt * kBK + 32 < kend;
            float4_t sa[kRT][2], sb[kRT][2];
            half8_t pa[kRT], pb[kRT];
            qk(kcur, 0, sa);
            if (second) qk(kcur, 1, sb);
            softmax(kt * kBK, sa, pa);
            pv(vcur, 0, pa);
            if (second) {
                softmax(kt * kBK + 32, sb, pb);
                pv(vcur, 1, pb);
            }
        }
        if (kt + 1 < ntiles) {
            if (stager) put(st, klds + ((kt + 1) & 1) * kTileBytes, vlds + ((kt + 1) & 1) * kTileBytes);
            __syncthreads();
            if (kt + 2 < ntiles) {
                ensure_window(((kt + 2) * kBK) >> a.bs_log2);
                if (stager) fetch(st, (kt + 2) * kBK);
            }
        }
    }
    __syncthreads();  // LDS is free for the next item

    // ---------------- output: lane (row col) holds dims 16 t + 4 grp + e
    if (!computes) return;  // (after the loop's last barrier)
#pragma unroll
    for (int r = 0; r < kRT; ++r) {
        const float lt = lsum[r][0];  // already summed over every key of the row
        const int j = qb * kBQ + 16 * r + col;
        if (j >= qlen) continue;
        const float inv = (rctx[r] > 0 && lt > 0.0f) ? 1.0f / lt : 0.0f;
        _Float16* orow = a.out + ((int64_t(q0) + j) * a.num_heads + h) * D;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            const half2_t lo = {static_cast<_Float16>(o[r][t][0] * inv), static_cast<_Float16>(o[r][t][1] * inv)};
            const half2_t hi = {static_cast<_Float16>(o[r][t][2] * inv), static_cast<_Float16>(o[r][t][3] * inv)};
            *reinterpret_cast<u32x2*>(orow + 16 * t + 4 * grp) =
                u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
        }
    }
}

// Persistent workgroups claim items of the list (built by
// prefill_items_kernel, longest first) one at a time through a counter, so a
// workgroup that finishes a short item takes the next one (greedy
// longest-processing-time balance).  Every item ends with a barrier, so LDS is
// free for the next one; every workgroup leaves once the list is exhausted.
template <int D, int KVT>
__global__ __launch_bounds__(64 * kMaxWaves) void prefill_mfma_kernel(PrefillArgs a) {
    using St = Stage<D, KVT>;
    __shared__ __attribute__((aligned(16))) char klds[2 * kBK * St::STR];  // two tile buffers each
    __shared__ __attribute__((aligned(16))) char vlds[2 * kBK * St::STR];
    __shared__ int btc[kBtCache];
    __shared__ int claimed;
    const int count = a.item_count[0];
    for (;;) {
        if (threadIdx.x == 0) claimed = atomicAdd(a.item_count + 1 + blockIdx.z, 1);
        __syncthreads();
        const int it = claimed;
        __syncthreads();  // every thread has read `claimed` before thread 0 may overwrite it
        if (it >= count) break;
        const int2 item = a.items[it];
        prefill_block<D, KVT>(a, item.x, item.y / a.num_kv_heads, item.y % a.num_kv_heads, klds, vlds, btc);
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// fp16 caches: tiles staged by direct global->LDS loads.
//
// A direct load writes 1 KiB of LDS per wave instruction (lane L -> bytes
// 16 L), so tile rows are unpadded: 16-byte chunk c of key row r sits at slot
// c ^ (r % CH) (CH chunks per row), which spreads the reads of one chunk
// column by 16 lanes over the banks.
template <int D>
struct DmaTile {
    static constexpr int ROW = D * 2;        // bytes per key row
    static constexpr int CH = ROW / 16;      // 16-byte chunks per row
    static constexpr int RPI = 1024 / ROW;   // rows per wave instruction
    static constexpr int INST = kBK / RPI;   // wave instructions per K (or V) tile
    static constexpr int BYTES = kBK * ROW;  // one K (or V) tile
    // LDS byte of (row, chunk)
    __device__ static __forceinline__ int off(int row, int chunk) { return row * ROW + ((chunk ^ (row % CH)) << 4); }
};

// FP8 caches on the same kernel (D = 128): the codes reach LDS by direct
// loads in rows of D bytes (same swizzle), the token scales by one 4-byte
// direct load per wave (waves of one parity load the same 64 K or V scales),
// and the workgroup converts each tile once into the fp16 tile that the fp16
// path computes from (code x scale in fp32, rounded to fp16, as the
// register-staged kernel does).
template <int D>
struct DmaTile8 {
    static constexpr int ROW = D;
    static constexpr int CH = ROW / 16;
    static constexpr int RPI = 1024 / ROW;
    static constexpr int INST = kBK / RPI;
    static constexpr int BYTES = kBK * ROW;
    __device__ static __forceinline__ int off(int row, int chunk) { return row * ROW + ((chunk ^ (row % CH)) << 4); }
};

// Workgroup barrier without a vector-memory wait (LDS writes published).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory"); }

// s_waitcnt with only the vector-memory count limited (GFX9 encoding: vmcnt
// bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier that publishes a tile: each wave first waits until at
// most N of its vector-memory operations are outstanding (its direct loads of
// the tile landed in LDS, the next tile's may still be in flight) and for all
// of its LDS operations, then meets the others.  Written as one asm block:
// with a release fence the compiler waits for every direct load in flight
// instead.  The memory clobber keeps LDS accesses on their side of it.
template <int N>
__device__ __forceinline__ void tile_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

// max(a, b, c) as v_maximum3_f32 (NaN-propagating, so no canonicalising
// v_max_f32 x, x, x is inserted for operands that come from the matrix cores)
__device__ __forceinline__ float vmax3(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

// ---------------------------------------------------------------------------
// fp16 caches: work items of (token, head) rows.
//
// A workgroup of kWideWaves waves owns (sequence, kv head, block of
// Wide<D>::ROWS rows), where the rows of a (sequence, kv head) are its
// (query token, head) pairs in the order j * G + g: each wave computes RT
// 16-row MFMA tiles of any mix of heads and tokens, since every row keeps its
// own context length and softmax state in its lane.  So every wave computes
// whatever the group size (G = 1 included), and the G heads of a token still
// share each K/V tile staged in LDS.  Each wave issues 1 / kWideWaves of the
// direct global->LDS loads of every tile (tile t + 2 while tile t is
// computed; the block ids one tile earlier still) and counts its own loads of
// tile t + 1 out with s_waitcnt vmcnt before the barrier that publishes it.
constexpr int kWideWaves = 8;  // two per SIMD
constexpr int kWideStages = 3;
constexpr int kWideBtc = 2048;  // block ids held in LDS at a time
// 16-row tiles per wave (what fits 256 registers) and (token, head) rows per item
template <int D>
struct Wide {
    static constexpr int RT = D == 128 ? 2 : 4;
    static constexpr int ROWS = kWideWaves * RT * 16;
};

// K and V tile buffers of the three stages: six LDS objects, so that the
// compiler can tell the direct loads into one stage from the reads of
// another (with one shared array it waits for every load in flight before
// each LDS read, which would undo the loads' lead).
struct WideBuffers {
    char* k[3];    // fp16 tiles (FP8: k[0] / v[0], the converted tile)
    char* v[3];
    int* btc;      // block ids of the item (kWideBtc)
    char* f8k[3];  // FP8: the code tiles of the three stages
    char* f8v[3];
    float* sc[3];  // FP8: 64 key scales, then 64 value scales, per stage
};

// Row blocks of a sequence with q query tokens (row_mult rows per token,
// rows_per_item per block; single-token sequences belong to decode), at most
// max_qblocks (max_query_len bounds q: caller contract).
__device__ __forceinline__ int seq_row_blocks(int q, int row_mult, int rows_per_item, int max_qblocks) {
    const int n = q >= 2 ? int((int64_t(q) * row_mult + rows_per_item - 1) / rows_per_item) : 0;
    return n < max_qblocks ? n : max_qblocks;
}
// Bin of row block b: nbins - 1 - (key tiles it stages, capped), so that the
// ascending bin order is the longest-first order.  Block b sees keys
// 0 .. kend - 1, kend = prior + its last token + 1 (clamped to the table).
__device__ __forceinline__ int row_block_bin(int prior, int q, int b, int row_mult, int rows_per_item,
                                             int table_tokens, int nbins) {
    const int64_t last = (int64_t(b + 1) * rows_per_item - 1) / row_mult + 1;
    int64_t kend = prior + (last < q ? last : q);
    kend = kend < table_tokens ? kend : table_tokens;
    const int64_t tiles = kend > 0 ? (kend + kBK - 1) / kBK : 0;
    return nbins - 1 - int(tiles < nbins - 1 ? tiles : nbins - 1);
}

// Output rows through LDS.  A wave's RT row tiles of O (accumulator layout:
// lane (row col) holds dims 16 t + 4 grp + e of row 16 r + col), scaled by
// inv[r] and rounded to fp16, go to its 16 RT rows x D region ob, then are
// read back as 16-byte pieces of rows: every store writes whole rows (the
// accumulator layout stores 8 bytes to each of 16 rows per instruction).
// Piece q of row R sits at R * 2D + (q ^ (R % P)) * 16, P pieces per row.
// Rows rho0 + R at or past nrows are not stored.
template <int D, int RT>
__device__ __forceinline__ void store_rows_lds(const PrefillArgs& a, char* ob, const float4_t (&o)[RT][D / 16],
                                               const float (&inv)[RT], const int rho0, const int nrows, const int q0,
                                               const int kvh, const int lane_in) {
    constexpr int ROW = D * 2;
    constexpr int P = ROW / 16;   // 16-byte pieces per row
    constexpr int RPI = 64 / P;   // rows per wave instruction
    // (the lane index through an opaque copy: the compiler would otherwise
    // compute these addresses once before the item loop and hold them in
    // registers across it)
    int lane = lane_in;
    asm volatile("" : "+v"(lane));
    const int col = lane & 15, grp = lane >> 4;
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int row = 16 * r + col;
#pragma unroll
        for (int t = 0; t < D / 16; ++t) {
            const half2_t lo = {static_cast<_Float16>(o[r][t][0] * inv[r]), static_cast<_Float16>(o[r][t][1] * inv[r])};
            const half2_t hi = {static_cast<_Float16>(o[r][t][2] * inv[r]), static_cast<_Float16>(o[r][t][3] * inv[r])};
            const int q = 2 * t + (grp >> 1);
            *reinterpret_cast<u32x2*>(ob + row * ROW + ((q ^ (row & (P - 1))) << 4) + (grp & 1) * 8) =
                u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
        }
    }
    // (a wave's LDS accesses complete in order: its own rows need no barrier)
    const int pq = lane % P;
#pragma unroll
    for (int i = 0; i < 16 * RT / RPI; ++i) {
        const int row = RPI * i + lane / P;
        const u32x4 v = *reinterpret_cast<const u32x4*>(ob + row * ROW + ((pq ^ (row & (P - 1))) << 4));
        const int rho = rho0 + row;
        if (rho < nrows) {
            const int j = row_token(a, rho);
            const int h = kvh * a.group + rho - j * a.group;
            store16(a.out + ((int64_t(q0) + j) * a.num_heads + h) * D + pq * 8, v);
        }
    }
}

template <int D, bool FP8>
__device__ __forceinline__ void prefill_block_wide(const PrefillArgs& a, const PrefillItem& it,
                                                   const WideBuffers& buf) {
    using T = DmaTile<D>;  // the fp16 tile the MFMAs read
    using L = typename std::conditional<FP8, DmaTile8<D>, DmaTile<D>>::type;  // the tile the loads fill
    constexpr int EB = FP8 ? 1 : 2;
    constexpr int DT = D / 16;  // output dim tiles
    constexpr int KS = D / 32;  // MFMA k-steps of Q K^T
    constexpr int RT = Wide<D>::RT;
    constexpr int kWideRows = Wide<D>::ROWS;
    constexpr int JW = L::INST / kWideWaves;  // direct loads per K (or V) tile and wave
    constexpr int NLOAD = 2 * JW + (FP8 ? 1 : 0);  // vector-memory operations per tile and wave
    static_assert(L::INST % kWideWaves == 0, "the loads of a tile must split evenly over the waves");
    static_assert(!FP8 || D == 128, "FP8 conversion maps 512 threads to 64 rows x 8 chunks");

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col = lane & 15;
    const int grp = lane >> 4;
    const int G = a.group;
    int* btc = buf.btc;

    const int s = it.s, b = it.b, kvh = it.kvh;
    const int q0 = it.q0;
    const int qlen = it.qlen;
    const int nrows = qlen * G;
    if (qlen < 2 || b * kWideRows >= nrows) return;  // (the item list holds none of these)
    const int prior = it.prior;
    const int last_row = min(nrows, (b + 1) * kWideRows) - 1;
    int kend = prior + last_row / G + 1;  // keys any row of the block may see
    kend = kend < a.table_tokens ? kend : a.table_tokens;
    const int ntiles = kend > 0 ? (kend + kBK - 1) / kBK : 0;

    // ---------------- loads of tile t, through block ids held in LDS
    const int bs_mask = (1 << a.bs_log2) - 1;
    const uint32_t row_bytes32 = uint32_t(a.num_kv_heads) * D * EB;
    // this lane's bytes within the cache row of its load j: the kv head and
    // the chunk that the swizzle puts at its LDS slot (the same in every tile)
    uint32_t lane_off[JW];
#pragma unroll
    for (int j = 0; j < JW; ++j) {
        const int row = (wave * JW + j) * L::RPI + lane / L::CH;
        lane_off[j] = uint32_t(kvh) * D * EB + uint32_t(((lane % L::CH) ^ (row % L::CH)) * 16);
    }
    const int32_t* table = a.bt + int64_t(s) * a.max_blocks_per_seq;
    // key of this lane's row in load j of tile t (keys past the end: kend - 1
    // again, masked; key 0 for an item with no keys at all, whose loads are
    // still issued so that the vmcnt counts below stay exact)
    auto load_key = [&](const int t, const int j) __attribute__((always_inline)) {
        int k = t * kBK + (wave * JW + j) * L::RPI + lane / L::CH;
        k = k < kend ? k : kend - 1;
        return k > 0 ? k : 0;
    };
    // The item's block ids (range-checked) sit in LDS, kWideBtc from block
    // `win` on.  Block ids read from global memory inside the tile loop would
    // be vector-memory results among the direct loads, and the compiler,
    // unable to count those apart, would wait for every load in flight
    // before using one.  Callers synchronise the workgroup after a fill.
    const int nblk = kend > 0 ? ((kend - 1) >> a.bs_log2) + 1 : 1;
    int win = 0;
    auto fill_window = [&](const int first) __attribute__((always_inline)) {
        win = first;
        const int n = nblk - first < kWideBtc ? nblk - first : kWideBtc;
        for (int i = tid; i < n; i += 64 * kWideWaves) {
            int id = table[first + i];
            if (a.num_blocks > 0 && unsigned(id) >= unsigned(a.num_blocks)) id = 0;
            btc[i] = id;
        }
    };
    // (slots are int32 in the API: slot_mapping, num_blocks * block_size)
    auto load_tile = [&](auto stage, const int t) __attribute__((always_inline)) {
        constexpr int S = decltype(stage)::value;
        char* kdst = FP8 ? buf.f8k[S] : buf.k[S];
        char* vdst = FP8 ? buf.f8v[S] : buf.v[S];
#pragma unroll
        for (int j = 0; j < JW; ++j) {
            const int jj = wave * JW + j;
            const int k = load_key(t, j);
            const int id = btc[(k >> a.bs_log2) - win];
            const uint32_t slot = (uint32_t(id) << a.bs_log2) + uint32_t(k & bs_mask);
            const uint64_t off = uint64_t(slot) * row_bytes32 + lane_off[j];
            __builtin_amdgcn_global_load_lds(a.kc + off, (__attribute__((address_space(3))) void*)(kdst + jj * 1024),
                                             16, 0, 0);
            __builtin_amdgcn_global_load_lds(a.vc + off, (__attribute__((address_space(3))) void*)(vdst + jj * 1024),
                                             16, 0, 0);
        }
        if constexpr (FP8) {
            // lane l: the scale of key t * 64 + l (clamped like the rows);
            // even waves the key scales, odd waves the value scales
            int k = t * kBK + lane;
            k = k < kend ? k : kend - 1;
            k = k > 0 ? k : 0;
            const int id = btc[(k >> a.bs_log2) - win];
            const uint32_t slot = (uint32_t(id) << a.bs_log2) + uint32_t(k & bs_mask);
            const float* src = ((wave & 1) ? a.vs : a.ks) + (uint64_t(slot) * a.num_kv_heads + kvh);
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(buf.sc[S] + 64 * (wave & 1)),
                                             4, 0, 0);
        }
    };
    // FP8: the codes of stage S into the fp16 tile (thread: key row tid / 8,
    // 16 codes of chunk tid % 8, i.e. fp16 chunks 2 c and 2 c + 1)
    auto convert = [&](auto stage) __attribute__((always_inline)) {
        constexpr int S = decltype(stage)::value;
        const int r = tid >> 3, c = tid & 7;
        const int src = L::off(r, c);
        const uint32_t ksb = __builtin_bit_cast(uint32_t, buf.sc[S][r]);
        const uint32_t vsb = __builtin_bit_cast(uint32_t, buf.sc[S][64 + r]);
        const u32x4 kw = *reinterpret_cast<const u32x4*>(buf.f8k[S] + src);
        const u32x4 vw = *reinterpret_cast<const u32x4*>(buf.f8v[S] + src);
        *reinterpret_cast<u32x4*>(buf.k[0] + T::off(r, 2 * c)) = to_half8<kFp8>(u32x4{kw[0], kw[1], ksb, 0u});
        *reinterpret_cast<u32x4*>(buf.k[0] + T::off(r, 2 * c + 1)) = to_half8<kFp8>(u32x4{kw[2], kw[3], ksb, 0u});
        *reinterpret_cast<u32x4*>(buf.v[0] + T::off(r, 2 * c)) = to_half8<kFp8>(u32x4{vw[0], vw[1], vsb, 0u});
        *reinterpret_cast<u32x4*>(buf.v[0] + T::off(r, 2 * c + 1)) = to_half8<kFp8>(u32x4{vw[2], vw[3], vsb, 0u});
    };

    fill_window(0);
    __syncthreads();

    // ---------------- Q (B operand of S^T = K Q^T) and per-row context; row
    // rho = b * ROWS + 16 (RT wave + r) + col is (token rho / G, head rho % G)
    const bool neg_scale = a.scale_log2 < 0.0f;
    const float sc = neg_scale ? -a.scale_log2 : a.scale_log2;
    half8_t qop[RT][KS];
    int rctx[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int rho = b * kWideRows + 16 * RT * wave + 16 * r + col;
        const bool ok = rho < nrows;
        const int j = ok ? rho / G : 0;
        const int h = kvh * G + (ok ? rho - j * G : 0);
        int c = prior + j + 1;
        c = c < 0 ? 0 : (c > a.table_tokens ? a.table_tokens : c);
        rctx[r] = ok ? c : 0;
        const int64_t qbase = (int64_t(q0) + j) * a.q_stride + int64_t(h) * D;
#pragma unroll
        for (int i = 0; i < KS; ++i) {
            u32x4 w = load16(a.q + (qbase + 32 * i + 8 * grp) * 2);
            const uint32_t keep = ok ? 0xFFFFFFFFu : 0u;
            const uint32_t flip = neg_scale ? 0x80008000u : 0u;
            w = (w ^ u32x4{flip, flip, flip, flip}) & u32x4{keep, keep, keep, keep};
            qop[r][i] = __builtin_bit_cast(half8_t, w);
        }
    }

    // Loads of tiles 0 and 1 (every wave issues its share, also for tiles past
    // the end, so that the vmcnt counts below are exact).
    load_tile(std::integral_constant<int, 0>(), 0);
    load_tile(std::integral_constant<int, 1>(), 1);

    const float lazy = kLazy / sc;  // kLazy in raw (unscaled) logit units
    float m[RT], mlim[RT], msc[RT];
    float4_t lsum[RT];  // row sums (every element the same)
    float4_t o[RT][DT];
    const half8_t kOnes = {1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16};
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        m[r] = -INFINITY;
        mlim[r] = -INFINITY;  // m + lazy
        msc[r] = 0.0f;        // m * sc, 0 while the row has no key
        lsum[r] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < DT; ++t) o[r][t] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }

    // This lane's LDS byte offsets within a step's K (V) rows.  The swizzle of
    // row r depends on r % CH only, and the rows this lane reads differ by
    // multiples of 16 (CH divides 16), so the other row halves and steps are
    // constant offsets.  K operand: row col (+16 hh), chunk 4 i + grp.  V^T
    // operand (transposed reads; lane m of group grp: key row 4 grp + m / 4
    // (+16), dims 16 t + 4 (m % 4) .. +3): chunk 2 t + (m % 4) / 2.
    int koff[KS], voff[DT];
    const int vrow = 4 * grp + (col >> 2);
#pragma unroll
    for (int i = 0; i < KS; ++i) koff[i] = T::off(col, 4 * i + grp);
#pragma unroll
    for (int t = 0; t < DT; ++t) voff[t] = T::off(vrow, 2 * t + ((col & 3) >> 1)) + 8 * (col & 1);

    auto qk = [&](const char* kb, float4_t (&sv)[RT][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < RT; ++r) sv[r][0] = sv[r][1] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < KS; ++i)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const half8_t kop =
                    __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4*>(kb + koff[i] + 16 * hh * T::ROW));
#pragma unroll
                for (int r = 0; r < RT; ++r)
                    sv[r][hh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, qop[r][i], sv[r][hh], 0, 0, 0);
            }
    };
    auto softmax = [&](auto masked, const int kbase, float4_t (&sv)[RT][2], half8_t (&pop)[RT])
                       __attribute__((always_inline)) {
        // causal / context mask, on the tiles of the masked tail only, and
        // there on steps that reach past some row's context (wave-uniform
        // test): key kbase + 16 hh + 4 grp + e < rctx
        bool edge = false;
#pragma unroll
        for (int r = 0; r < RT; ++r) edge = edge || kbase + 32 > rctx[r];
        if (decltype(masked)::value && __builtin_amdgcn_ballot_w64(edge)) {
#pragma unroll
            for (int r = 0; r < RT; ++r)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (kbase + 16 * hh + 4 * grp + e >= rctx[r]) sv[r][hh][e] = -INFINITY;
        }
        // This lane's max decides whether the row max is needed at all: it is
        // only when some lane exceeds the lazy limit m + kLazy (then the max
        // over the row's four key groups resets m and rescales).  Below the
        // limit the weights exp2((x - m) sc) stay under 2^kLazy, well inside
        // fp16 for P and fp32 for the sums: the same softmax.
        float lmx[RT];
        bool over = false;
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            lmx[r] = vmax3(vmax3(sv[r][0][0], sv[r][0][1], sv[r][0][2]), vmax3(sv[r][0][3], sv[r][1][0], sv[r][1][1]),
                           vmax3(sv[r][1][2], sv[r][1][3], sv[r][1][3]));
            over = over || lmx[r] > mlim[r];
        }
        if (__builtin_amdgcn_ballot_w64(over)) {
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                if (__builtin_amdgcn_ballot_w64(lmx[r] > mlim[r])) {
                    const float mx = row_group_max(lmx[r]);
                    const float mn = fmaxf(m[r], mx);
                    const float alpha = mn > m[r] ? __builtin_amdgcn_exp2f((m[r] - mn) * sc) : 1.0f;
                    m[r] = mn;
                    mlim[r] = mn + lazy;
                    msc[r] = (mn == -INFINITY ? 0.0f : mn) * sc;
                    lsum[r] *= alpha;
#pragma unroll
                    for (int t = 0; t < DT; ++t) o[r][t] *= alpha;
                }
            }
        }
        // P^T operand: k slot (grp, e) = key 4 grp + e, slot (grp, 4 + e) = key 16 + 4 grp + e
#pragma unroll
        for (int r = 0; r < RT; ++r) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    pop[r][4 * hh + e] =
                        static_cast<_Float16>(__builtin_amdgcn_exp2f(fmaf(sv[r][hh][e], sc, -msc[r])));
            // row sums on the matrix pipe: a V^T tile of ones gives sum_k p in every lane
            lsum[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kOnes, pop[r], lsum[r], 0, 0, 0);
        }
    };
    auto pv = [&](const char* vb, const half8_t (&pop)[RT]) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            const u32x2 lo = tr_read(vb + voff[t]);
            const u32x2 hi = tr_read(vb + voff[t] + 16 * T::ROW);
            const half8_t vop = __builtin_bit_cast(half8_t, u32x4{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
            for (int r = 0; r < RT; ++r) o[r][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, pop[r], o[r][t], 0, 0, 0);
        }
    };

    // One tile t in buffer S = t % kWideStages (a compile-time constant, so
    // that every LDS address is a per-lane register plus an immediate);
    // masked: the causal / context mask may cut into the tile.
    auto tile = [&](auto stage, auto masked, const int t) __attribute__((always_inline)) {
        constexpr int S = decltype(stage)::value;
        tile_barrier<NLOAD>();  // tile t published (t + 1 in flight); every wave has left tile t - 1
        {
            // the block ids of tile t + 2 must be in the window (every wave has
            // issued tile t + 1's loads, the last reads of the old window)
            const int last = (t + 3) * kBK - 1 < kend - 1 ? (t + 3) * kBK - 1 : kend - 1;
            if (last > 0 && (last >> a.bs_log2) - win >= kWideBtc) {
                fill_window(((t + 2) * kBK) >> a.bs_log2);
                __syncthreads();
            }
        }
        load_tile(std::integral_constant<int, (S + 2) % kWideStages>(), t + 2);  // buffer of tile t - 1
        if constexpr (FP8) {
            convert(stage);  // every wave has left the fp16 tile (barrier above)
            lds_barrier();
        }
        const char* kcur = FP8 ? buf.k[0] : buf.k[S];
        const char* vcur = FP8 ? buf.v[0] : buf.v[S];
        float4_t sv[RT][2];
        half8_t pop[RT];
        qk(kcur, sv);
        softmax(masked, t * kBK, sv, pop);
        pv(vcur, pop);
        if (!decltype(masked)::value || t * kBK + 32 < kend) {
            qk(kcur + 32 * T::ROW, sv);
            softmax(masked, t * kBK + 32, sv, pop);
            pv(vcur + 32 * T::ROW, pop);
        }
    };
    using C0 = std::integral_constant<int, 0>;
    using C1 = std::integral_constant<int, 1>;
    using C2 = std::integral_constant<int, 2>;
    static_assert(kWideStages == 3, "the main loop below is unrolled over three buffers");
    // Tiles below every row's context need no mask: the first row of the item
    // has the shortest context.
    const int ctx_min = min(prior + (b * kWideRows) / G + 1, kend);
    const int tfull = ctx_min / kBK;
    int t = 0;
    for (; t + 3 <= tfull; t += 3) {
        tile(C0(), std::false_type(), t);
        tile(C1(), std::false_type(), t + 1);
        tile(C2(), std::false_type(), t + 2);
    }
    for (; t < ntiles; ++t) {
        const int sidx = t % kWideStages;
        if (sidx == 0) tile(C0(), std::true_type(), t);
        else if (sidx == 1) tile(C1(), std::true_type(), t);
        else tile(C2(), std::true_type(), t);
    }
    wait_vmcnt<0>();  // no load of this item may land in the next item's buffers

    if constexpr (D == 128) {
        // ---------------- output through LDS, 8 KiB per wave: FP8, the six
        // code buffers and the two fp16 tiles; fp16, the halves of the six
        // tile buffers
        static_assert(16 * RT * D * 2 == 8192 && DmaTile8<D>::BYTES == 8192 && T::BYTES == 16384,
                      "8 KiB of output rows per wave");
        __syncthreads();  // every wave's loads have landed and no wave reads a tile
        // (constant indices only: a buffer array indexed by a variable would
        // be materialised in memory)
        char* ob;
        if constexpr (FP8) {
            ob = wave == 0 ? buf.f8k[0] : wave == 1 ? buf.f8k[1] : wave == 2 ? buf.f8k[2] : wave == 3 ? buf.f8v[0]
               : wave == 4 ? buf.f8v[1] : wave == 5 ? buf.f8v[2] : wave == 6 ? buf.k[0] : buf.v[0];
        } else {
            const int h2 = wave >> 1;
            ob = (h2 == 0 ? buf.k[0] : h2 == 1 ? buf.k[1] : h2 == 2 ? buf.k[2] : buf.v[0]) + (wave & 1) * 8192;
        }
        float inv[RT];
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const float lt = lsum[r][0];
            inv[r] = (rctx[r] > 0 && lt > 0.0f) ? 1.0f / lt : 0.0f;
        }
        store_rows_lds<D, RT>(a, ob, o, inv, b * kWideRows + 16 * RT * wave, nrows, q0, kvh, lane);
        return;
    }
    // ---------------- output: lane (row col) holds dims 16 t + 4 grp + e
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int rho = b * kWideRows + 16 * RT * wave + 16 * r + col;
        if (rho >= nrows) continue;
        const int j = rho / G;
        const int h = kvh * G + rho - j * G;
        const float lt = lsum[r][0];
        const float inv = (rctx[r] > 0 && lt > 0.0f) ? 1.0f / lt : 0.0f;
        _Float16* orow = a.out + ((int64_t(q0) + j) * a.num_heads + h) * D;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            const half2_t lo = {static_cast<_Float16>(o[r][t][0] * inv), static_cast<_Float16>(o[r][t][1] * inv)};
            const half2_t hi = {static_cast<_Float16>(o[r][t][2] * inv), static_cast<_Float16>(o[r][t][3] * inv)};
            *reinterpret_cast<u32x2*>(orow + 16 * t + 4 * grp) =
                u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
        }
    }
}

// In-kernel work list of a small call, built by every workgroup of the fp16
// kernel alike (so no list kernel runs before it): the row blocks are
// numbered in (sequence, block) order, each block's sort key is (bin, number)
// and its place in the longest-first order is the count of smaller keys.  The
// keys are distinct, so every workgroup computes the same order; the ranking
// is quadratic, which at kInlineBlocks blocks is a few hundred LDS reads per
// thread.  Returns the number of blocks; lblk holds them in order.
constexpr int kInlineBlocks = 512;
template <int NT>
__device__ int inline_row_blocks(const PrefillArgs& a, int2* lblk) {
    constexpr int NW = NT / 64;
    constexpr int PER = kInlineBlocks / NT;  // blocks ranked per thread
    static_assert(kInlineBlocks % NT == 0, "blocks must split evenly over the threads");
    __shared__ int key[kInlineBlocks];
    __shared__ int wave_tot[NW];
    __shared__ int carry;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) carry = 0;
    __syncthreads();
    // number the blocks: sequences in chunks of one per thread, block counts
    // scanned across the workgroup
    for (int s0 = 0; s0 < a.num_seqs; s0 += NT) {
        const int s = s0 + tid;
        int q = 0, prior = 0, n = 0;
        if (s < a.num_seqs) {
            q = a.qsl[s + 1] - a.qsl[s];
            prior = a.cl[s] - q;
            n = seq_row_blocks(q, a.group, a.rows_per_item, a.qblocks);
        }
        const int incl = wave_incl_scan(n);
        if (lane == 63) wave_tot[wave] = incl;
        __syncthreads();
        int before = carry;
        for (int w = 0; w < wave; ++w) before += wave_tot[w];
        for (int b = 0; b < n; ++b) {
            const int i = before + incl - n + b;
            if (i < kInlineBlocks) {  // (the host bound keeps every call within)
                key[i] = (row_block_bin(prior, q, b, a.group, a.rows_per_item, a.table_tokens, a.nbins) << 9) | i;
                lblk[i] = int2{s, b};
            }
        }
        __syncthreads();
        if (tid == 0) {
            int t = carry;
            for (int w = 0; w < NW; ++w) t += wave_tot[w];
            carry = t;
        }
        __syncthreads();
    }
    const int total = carry < kInlineBlocks ? carry : kInlineBlocks;
    // rank, then place (lblk is read before the barrier and written after it)
    int2 mine[PER];
    int rank[PER];
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const int i = tid + p * NT;
        mine[p] = int2{0, 0};
        rank[p] = 0;
        if (i < total) {
            const int k = key[i];
            mine[p] = lblk[i];
            for (int j = 0; j < total; ++j) rank[p] += key[j] < k ? 1 : 0;
        }
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < PER; ++p)
        if (tid + p * NT < total) lblk[rank[p]] = mine[p];
    __syncthreads();
    return total;
}

// Host-built schedule (vkv_prefill_work_list_host): 32 header words ([0] W
// lists, one per workgroup of the persistent grid; [1] L slots per list; [2]
// the format, kListFormat; [3] N items), then W x L slots of kListItemWords
// words, slot k of list w at k W + w: s, b, kvh, q0, qlen, prior, key tiles, 0
// (s = -1: the list has ended).  The host deals the items to the lists
// longest first, each to the list with the least work so far (a
// longest-processing-time schedule made before the launch), so a workgroup
// knows its next item while it computes the current one; its first item,
// slot w, needs no header word and is requested together with the header.
constexpr int kListHeaderWords = 32;
constexpr int kListFormat = 3;
constexpr int kListItemWords = 8;
// Cost of an item in the host's schedule: its key tiles plus this many for
// its start (the chain of loads before its first tile can be computed).
constexpr int kListItemStartTiles = 5;
constexpr int kListDefaultCus = 256;  // lists when the builder finds no device

// The sequence fields of item (s, b, kvh), read from the call's arrays.
__device__ __forceinline__ PrefillItem load_item(const PrefillArgs& a, const int s, const int b, const int kvh) {
    const int q0 = a.qsl[s];
    const int qlen = a.qsl[s + 1] - q0;
    return PrefillItem{s, b, kvh, q0, qlen, a.cl[s] - qlen};
}

// Persistent loop of the direct-load kernels (NT threads): work items from the
// host-built schedule, the in-kernel list (small calls) or the list kernel's;
// item_fn(it) runs one.  No item is claimed, so no counter needs resetting.
template <int NT, typename Item>
__device__ __forceinline__ void run_items(const PrefillArgs& a, Item item_fn) {
    if (a.work_list) {
        // Workgroup w runs list w (and w + grid, ...), no claims.  Every index
        // read from the list is bounded by its length, and items outside the
        // call's sequences, kv heads and query rows are skipped, so a list
        // from another call gives wrong rows but reads nothing out of bounds.
        const int32_t* wl = a.work_list;
        const int32_t* slots = wl + kListHeaderWords;
        const int64_t cap = (int64_t(a.work_list_words) - kListHeaderWords) / kListItemWords;
        PrefillItem nx;
        auto fetch = [&](const int64_t k) __attribute__((always_inline)) {
            const int32_t* e = slots + k * kListItemWords;
            nx = PrefillItem{e[0], e[1], e[2], e[3], e[4], e[5]};
        };
        auto valid = [&](const PrefillItem& it) __attribute__((always_inline)) {
            return unsigned(it.s) < unsigned(a.num_seqs) && unsigned(it.kvh) < unsigned(a.num_kv_heads) &&
                   it.b >= 0 && it.q0 >= 0 && it.qlen >= 2 && int64_t(it.q0) + it.qlen <= a.num_query_tokens &&
                   int64_t(it.b) * a.rows_per_item < int64_t(it.qlen) * a.group;
        };
        for (int w = blockIdx.x; w < cap; w += gridDim.x) {
            fetch(w);  // (slot 0 of list w, beside the header)
            const int lists = wl[0], len = wl[1];
            if (wl[2] != kListFormat || lists < 1 || len < 0 || int64_t(lists) * len > cap || w >= lists) break;
            for (int k = 0; k < len; ++k) {
                const PrefillItem it = nx;
                if (it.s < 0) break;  // (the list has ended)
                const bool ok = valid(it);
                // the next slot, requested after this one is checked (waiting
                // for this one then waits for nothing else), arrives while
                // this item runs
                asm volatile("" ::: "memory");
                if (k + 1 < len) fetch(int64_t(k + 1) * lists + w);
                if (ok) item_fn(it);
            }
        }
        return;
    }
    // The in-kernel list (every workgroup orders a small call's row blocks
    // itself) or the list kernel's, longest first, dealt to the workgroups in
    // a snake: round r gives item r W + p to workgroup p when r is even and
    // to W - 1 - p when r is odd (W workgroups, all resident: one per CU), so
    // the longest items meet the shortest ones, as a longest-processing-time
    // schedule would put them, with no claims.
    __shared__ int2 lblk[kInlineBlocks];  // inline list: (s, b) of row block i, then in longest-first order
    const int count = a.inline_list ? inline_row_blocks<NT>(a, lblk) * a.num_kv_heads : a.item_count[0];
    const int W = gridDim.x, p = blockIdx.x;
    for (int r = 0;; ++r) {
        const int64_t it = int64_t(r) * W + ((r & 1) ? W - 1 - p : p);
        if (it >= count) break;  // (later rounds are further on)
        // items (row block, kv head), kv head fastest
        int2 item;
        if (a.inline_list) {
            const int2 blk = lblk[it / a.num_kv_heads];
            item = int2{blk.x, blk.y * a.num_kv_heads + int(it % a.num_kv_heads)};
        } else {
            item = a.items[it];
        }
        item_fn(load_item(a, item.x, item.y / a.num_kv_heads, item.y % a.num_kv_heads));
    }
}

template <int D, bool FP8>
__device__ __forceinline__ void wide_items(const PrefillArgs& a, const WideBuffers& buf) {
    run_items<64 * kWideWaves>(a, [&](const PrefillItem& it) __attribute__((always_inline)) {
        prefill_block_wide<D, FP8>(a, it, buf);
    });
}

template <int D>
__global__ __launch_bounds__(64 * kWideWaves) void prefill_wide_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(1024))) char k0[DmaTile<D>::BYTES];
    __shared__ __attribute__((aligned(1024))) char k1[DmaTile<D>::BYTES];
    __shared__ __attribute__((aligned(1024))) char k2[DmaTile<D>::BYTES];
    __shared__ __attribute__((aligned(1024))) char v0[DmaTile<D>::BYTES];
    __shared__ __attribute__((aligned(1024))) char v1[DmaTile<D>::BYTES];
    __shared__ __attribute__((aligned(1024))) char v2[DmaTile<D>::BYTES];
    __shared__ int btc[kWideBtc];
    static_assert(kWideStages == 3, "three K and three V buffers");
    const WideBuffers buf = {{k0, k1, k2}, {v0, v1, v2}, btc, {nullptr, nullptr, nullptr},
                             {nullptr, nullptr, nullptr}, {nullptr, nullptr, nullptr}};
    wide_items<D, false>(a, buf);
}

// ---------------------------------------------------------------------------
// fp16 caches at D = 128, one wave per SIMD: prefill_w64_kernel.
//
// The same work items as prefill_wide_kernel<128> (256 (token, head) rows of
// one sequence and kv head), computed by 4 waves of 64 rows (four 16-row MFMA
// tiles) instead of 8 waves of 32.  Every K or V operand read from LDS then
// feeds four MFMAs instead of two, which halves the LDS bytes per FLOP (the
// operand reads bounded the 8-wave kernel).  A lone wave per SIMD has 512
// registers: the output and row-sum accumulators live in AGPRs (asm MFMAs,
// below) and the scores of two steps in VGPRs, so a wave overlaps its own
// phases: step s's exponentials run on the VALU while step s + 1's Q K^T runs
// on the matrix pipe, and step s's P V while step s + 2's K operands are read
// and step s + 1's maxima computed.  K/V tiles reach LDS by direct loads as in
// the 8-wave kernel, through four stages: with the overlap a wave still reads
// tile t - 1 after the barrier that publishes tile t + 1, so the loads issued
// after that barrier (tile t + 3) go to the buffer of tile t - 1, which every
// wave has left by then.  Tiles whose keys all lie below every row's context
// run this pipeline; the masked tail tiles run one step at a time.
constexpr int kW64Waves = 4;
constexpr int kW64RT = 4;  // 16-row tiles per wave
constexpr int kW64Stages = 4;
static_assert(kW64Waves * kW64RT * 16 == Wide<128>::ROWS, "the same items (and work list) as the 8-wave kernel");

struct W64Buffers {
    char* tiles;  // stage S: K tile at S * 2 * tile bytes, V tile right after it
    int* btc;
};

// One 16-byte direct global->LDS load per lane (LDS address lds + 16 lane),
// in asm: the compiler then does not track these LDS writes, so it neither
// needs a separate LDS object per stage to tell them from the operand reads
// nor waits for them (the tile barrier counts them out with s_waitcnt vmcnt).
// s_nop 0: the wait state between the M0 write and the load reading it.
__device__ __forceinline__ void dma16(const char* g, const uint32_t lds) {
    const uint32_t l = __builtin_amdgcn_readfirstlane(lds);  // (wave-uniform; an SGPR operand)
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(l) : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
    typedef const __attribute__((address_space(3))) char* lds_cptr;
    return uint32_t(size_t((lds_cptr)p));
}

// c_r += A B_r (r = 0..3) on the matrix cores, the accumulators in AGPRs.
// The compiler's own MFMA selection at one wave per SIMD would put every MFMA
// result in AGPRs, the scores included, and copy them out for the softmax;
// asm keeps just these accumulators there.  The compiler inserts no wait
// states around asm: the leading s_nop covers VALU writes of the B operands
// (P) just before, and agpr_fence() the AGPR reads that follow.
__device__ __forceinline__ void mfma4_agpr(float4_t& c0, float4_t& c1, float4_t& c2, float4_t& c3, const half8_t a,
                                           const half8_t b0, const half8_t b1, const half8_t b2, const half8_t b3) {
    asm("s_nop 4\n\t"
        "v_mfma_f32_16x16x32_f16 %0, %4, %5, %0\n\t"
        "v_mfma_f32_16x16x32_f16 %1, %4, %6, %1\n\t"
        "v_mfma_f32_16x16x32_f16 %2, %4, %7, %2\n\t"
        "v_mfma_f32_16x16x32_f16 %3, %4, %8, %3"
        : "+a"(c0), "+a"(c1), "+a"(c2), "+a"(c3)
        : "v"(a), "v"(b0), "v"(b1), "v"(b2), "v"(b3));
}

// Wait states (32) between the asm MFMAs' AGPR writes and any other read of
// those AGPRs: more than the longest XDL write-to-read distance.  Every
// accumulator passes through it, so no read can move above it.
// The accumulators placed in AGPRs once (zero-initialised values would
// otherwise be re-materialised and copied in at every asm MFMA).
template <int RT, int DT>
__device__ __forceinline__ void agpr_pin(float4_t (&o)[RT][DT], float4_t (&l)[RT]) {
    asm volatile("" : "+a"(l[0]), "+a"(l[1]), "+a"(l[2]), "+a"(l[3]));
#pragma unroll
    for (int r = 0; r < RT; ++r)
        asm volatile("" : "+a"(o[r][0]), "+a"(o[r][1]), "+a"(o[r][2]), "+a"(o[r][3]), "+a"(o[r][4]), "+a"(o[r][5]),
                     "+a"(o[r][6]), "+a"(o[r][7]));
}

template <int RT, int DT>
__device__ __forceinline__ void agpr_fence(float4_t (&o)[RT][DT], float4_t (&l)[RT]) {
    asm volatile("s_nop 15\n\ts_nop 15" : "+a"(l[0]), "+a"(l[1]), "+a"(l[2]), "+a"(l[3]));
#pragma unroll
    for (int r = 0; r < RT; ++r)
        asm volatile("" : "+a"(o[r][0]), "+a"(o[r][1]), "+a"(o[r][2]), "+a"(o[r][3]), "+a"(o[r][4]), "+a"(o[r][5]),
                     "+a"(o[r][6]), "+a"(o[r][7]));
}

// s_r = A B_r (first k-step: no accumulator) and s_r += A B_r, r = 0..3, for
// the scores S^T = K Q^T: A = K (VGPRs, from LDS), B = Q (AGPRs, which the
// MFMAs read directly), s in VGPRs.  Early-clobber outputs: the block writes
// s_0 before its last MFMA reads A.
__device__ __forceinline__ void mfma4_first(float4_t& s0, float4_t& s1, float4_t& s2, float4_t& s3, const half8_t a,
                                            const half8_t b0, const half8_t b1, const half8_t b2, const half8_t b3) {
    asm("v_mfma_f32_16x16x32_f16 %0, %4, %5, 0\n\t"
        "v_mfma_f32_16x16x32_f16 %1, %4, %6, 0\n\t"
        "v_mfma_f32_16x16x32_f16 %2, %4, %7, 0\n\t"
        "v_mfma_f32_16x16x32_f16 %3, %4, %8, 0"
        : "=&v"(s0), "=&v"(s1), "=&v"(s2), "=&v"(s3)
        : "v"(a), "a"(b0), "a"(b1), "a"(b2), "a"(b3));
}
__device__ __forceinline__ void mfma4_vacc(float4_t& s0, float4_t& s1, float4_t& s2, float4_t& s3, const half8_t a,
                                           const half8_t b0, const half8_t b1, const half8_t b2, const half8_t b3) {
    asm("v_mfma_f32_16x16x32_f16 %0, %4, %5, %0\n\t"
        "v_mfma_f32_16x16x32_f16 %1, %4, %6, %1\n\t"
        "v_mfma_f32_16x16x32_f16 %2, %4, %7, %2\n\t"
        "v_mfma_f32_16x16x32_f16 %3, %4, %8, %3"
        : "+v"(s0), "+v"(s1), "+v"(s2), "+v"(s3)
        : "v"(a), "a"(b0), "a"(b1), "a"(b2), "a"(b3));
}

// Wait states (8, the distance LLVM keeps between this MFMA's result and a
// VALU read of it) between the asm MFMAs' writes of the scores and their VALU
// reads, with every score passing through it.
__device__ __forceinline__ void score_fence(float4_t (&sv)[4][2]) {
    asm volatile("s_nop 7"
                 : "+v"(sv[0][0]), "+v"(sv[0][1]), "+v"(sv[1][0]), "+v"(sv[1][1]), "+v"(sv[2][0]), "+v"(sv[2][1]),
                   "+v"(sv[3][0]), "+v"(sv[3][1]));
}

// Single MFMAs for hand-placed schedules (each between scheduling barriers):
// s = A B (no accumulator), s += A B with s in VGPRs and B = Q in AGPRs, and
// c += A B with c in AGPRs.  No wait states: the schedule keeps every VALU
// write of an operand at least two instructions ahead of its MFMA.
__device__ __forceinline__ void mfma_first_v(float4_t& s, const half8_t a, const half8_t b) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, 0" : "=&v"(s) : "v"(a), "a"(b));
}
__device__ __forceinline__ void mfma_acc_v(float4_t& s, const half8_t a, const half8_t b) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(s) : "v"(a), "a"(b));
}
__device__ __forceinline__ void mfma_acc_a(float4_t& c, const half8_t a, const half8_t b) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}

// VALU work of the hand-placed slots, also in asm so that it stays where it is
// written (the compiler orders plain arithmetic freely around scheduling
// barriers).  w = exp2(x sc - m): v_fma_f32 then v_exp_f32.
__device__ __forceinline__ float slot_exp2(const float x, const float sc, const float m) {
    float w;
    asm volatile("v_fma_f32 %0, %1, %2, -%3\n\tv_exp_f32 %0, %0" : "=&v"(w) : "v"(x), "s"(sc), "v"(m));
    return w;
}
// Two weights rounded to fp16 (nearest even) in one word.  Placed at least
// two slots after the exps it reads: a trans result (v_exp_f32) needs a wait
// state before another VALU reads it, and reading it sooner stalls the
// wave's in-order issue on the exp's latency (measured: a pack right after
// its exps cost twice as much beside an MFMA).
__device__ __forceinline__ uint32_t slot_pack(const float lo, const float hi) {
    uint32_t r;
    asm volatile("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(r) : "v"(lo), "v"(hi));
    return r;
}
// max(a, b, c), NaN-propagating like v_maximum3_f32
__device__ __forceinline__ float slot_max3(const float a, const float b, const float c) {
    float r;
    asm volatile("v_maximum3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Keys any row of row block b may see (the rows' largest context), clamped to
// the table.
__device__ __forceinline__ int item_kend(const PrefillArgs& a, const PrefillItem& it, const int rows) {
    const int nrows = it.qlen * a.group;
    const int last_row = min(nrows, (it.b + 1) * rows) - 1;
    const int kend = it.prior + last_row / a.group + 1;
    return kend < a.table_tokens ? kend : a.table_tokens;
}

template <int D>
__device__ __forceinline__ void prefill_block_w64(const PrefillArgs& a, const PrefillItem& it,
                                                  const W64Buffers& buf) {
    using T = DmaTile<D>;
    constexpr int EB = 2;
    constexpr int DT = D / 16;  // output dim tiles
    constexpr int KS = D / 32;  // MFMA k-steps of Q K^T
    constexpr int RT = kW64RT;
    constexpr int kRows = kW64Waves * RT * 16;
    constexpr int NT = 64 * kW64Waves;
    constexpr int JW = T::INST / kW64Waves;  // direct loads per K (or V) tile and wave
    constexpr int NLOAD = 2 * JW;            // vector-memory operations per tile and wave
    static_assert(D == 128 && DT == 8 && RT == 4, "the asm accumulator blocks assume four row tiles, eight dim tiles");
    static_assert(T::INST % kW64Waves == 0, "the loads of a tile must split evenly over the waves");

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // (scalar: the loads' LDS addresses are)
    const int col = lane & 15;
    const int grp = lane >> 4;
    const int G = a.group;
    int* btc = buf.btc;

    const int s = it.s, b = it.b, kvh = it.kvh;
    const int q0 = it.q0;
    const int qlen = it.qlen;
    const int nrows = qlen * G;
    if (qlen < 2 || b * kRows >= nrows) return;  // (the item list holds none of these)
    const int prior = it.prior;
    const int kend = item_kend(a, it, kRows);  // keys any row of the block may see
    const int ntiles = kend > 0 ? (kend + kBK - 1) / kBK : 0;

    // ---------------- loads of tile t, through block ids held in LDS (as in prefill_block_wide)
    const int bs_mask = (1 << a.bs_log2) - 1;
    const uint32_t row_bytes32 = uint32_t(a.num_kv_heads) * D * EB;
    uint32_t lane_off[JW];
#pragma unroll
    for (int j = 0; j < JW; ++j) {
        const int row = (wave * JW + j) * T::RPI + lane / T::CH;
        lane_off[j] = uint32_t(kvh) * D * EB + uint32_t(((lane % T::CH) ^ (row % T::CH)) * 16);
    }
    const int32_t* table = a.bt + int64_t(s) * a.max_blocks_per_seq;
    auto load_key = [&](const int t, const int j) __attribute__((always_inline)) {
        int k = t * kBK + (wave * JW + j) * T::RPI + lane / T::CH;
        k = k < kend ? k : kend - 1;
        return k > 0 ? k : 0;
    };
    const int nblk = kend > 0 ? ((kend - 1) >> a.bs_log2) + 1 : 1;
    int win = 0;
    auto fill_window = [&](const int first) __attribute__((always_inline)) {
        win = first;
        const int n = nblk - first < kWideBtc ? nblk - first : kWideBtc;
        for (int i = tid; i < n; i += NT) {
            int id = table[first + i];
            if (a.num_blocks > 0 && unsigned(id) >= unsigned(a.num_blocks)) id = 0;
            btc[i] = id;
        }
    };
    const uint32_t tiles_lds = lds_addr(buf.tiles);
    auto kstage = [&](const int st) __attribute__((always_inline)) { return buf.tiles + st * (2 * T::BYTES); };
    auto vstage = [&](const int st) __attribute__((always_inline)) { return buf.tiles + st * (2 * T::BYTES) + T::BYTES; };
    // This wave's share of tile t's loads: load j of K (or V) fills LDS bytes
    // stage base + (JW wave + j) KiB (+ the tile size for V).
    auto dma_lds = [&](const int st, const int j) __attribute__((always_inline)) {
        return tiles_lds + uint32_t(st * (2 * T::BYTES) + (wave * JW + j) * 1024);
    };
    auto dma_off = [&](const int t, const int j, const int id) __attribute__((always_inline)) {
        const int k = load_key(t, j);
        const uint32_t slot = (uint32_t(id) << a.bs_log2) + uint32_t(k & bs_mask);
        return uint64_t(slot) * row_bytes32 + lane_off[j];
    };
    auto dma_id = [&](const int t, const int j) __attribute__((always_inline)) {
        return btc[(load_key(t, j) >> a.bs_log2) - win];
    };
    auto load_tile = [&](const int st, const int t) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < JW; ++j) {
            const uint64_t off = dma_off(t, j, dma_id(t, j));
            dma16(a.kc + off, dma_lds(st, j));
            dma16(a.vc + off, dma_lds(st, j) + T::BYTES);
        }
    };
    // Barrier publishing tile t (its loads landed, tile t + 1's in flight);
    // the block ids of tile t + 2 are then in the window (every wave has
    // issued tile t + 1's loads, the last reads of the old window).  The
    // caller issues the loads of tile t + 2.
    auto publish_barrier = [&](const int t) __attribute__((always_inline)) {
        tile_barrier<NLOAD>();
        const int last = (t + 3) * kBK - 1 < kend - 1 ? (t + 3) * kBK - 1 : kend - 1;
        if (last > 0 && (last >> a.bs_log2) - win >= kWideBtc) {
            fill_window(((t + 2) * kBK) >> a.bs_log2);
            __syncthreads();
        }
    };

    fill_window(0);
    __syncthreads();


    // Loads of tiles 0 and 1 (every wave issues its share, also for tiles past
    // the end, so that the vmcnt counts are exact).
    load_tile(0, 0);
    load_tile(1, 1);

    // ---------------- Q (B operand of S^T = K Q^T) and per-row context, loaded
    // while the first two tiles load.  Row
    // rho = b * kRows + 16 (RT wave + r) + col is (token rho / G, head rho % G)
    const bool neg_scale = a.scale_log2 < 0.0f;
    const float sc = neg_scale ? -a.scale_log2 : a.scale_log2;
    half8_t qop[RT][KS];
    int rctx[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int rho = b * kRows + 16 * RT * wave + 16 * r + col;
        const bool ok = rho < nrows;
        const int j = ok ? rho / G : 0;
        const int h = kvh * G + (ok ? rho - j * G : 0);
        int c = prior + j + 1;
        c = c < 0 ? 0 : (c > a.table_tokens ? a.table_tokens : c);
        rctx[r] = ok ? c : 0;
        const int64_t qbase = (int64_t(q0) + j) * a.q_stride + int64_t(h) * D;
#pragma unroll
        for (int i = 0; i < KS; ++i) {
            u32x4 w = load16(a.q + (qbase + 32 * i + 8 * grp) * 2);
            const uint32_t keep = ok ? 0xFFFFFFFFu : 0u;
            const uint32_t flip = neg_scale ? 0x80008000u : 0u;
            w = (w ^ u32x4{flip, flip, flip, flip}) & u32x4{keep, keep, keep, keep};
            qop[r][i] = __builtin_bit_cast(half8_t, w);
        }
    }

    const float lazy = kLazy / sc;  // kLazy in raw (unscaled) logit units
    float m[RT], mlim[RT], msc[RT];
    float4_t lsum[RT];    // row sums (every element the same), AGPRs
    float4_t o[RT][DT];   // O^T, AGPRs
    half8_t kOnes = {1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16};
    // held in registers from here on: rematerialised by a move right before
    // an asm MFMA it would lack the VALU-write-to-MFMA-read wait states
    asm volatile("s_nop 1" : "+v"(kOnes));
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        m[r] = -INFINITY;
        mlim[r] = -INFINITY;  // m + lazy
        msc[r] = 0.0f;        // m * sc, 0 while the row has no key
        lsum[r] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < DT; ++t) o[r][t] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    agpr_pin(o, lsum);

    // LDS byte offsets of this lane's operands within a step's K (V) rows, as
    // in prefill_block_wide.
    int koff[KS], voff[DT];
    const int vrow = 4 * grp + (col >> 2);
#pragma unroll
    for (int i = 0; i < KS; ++i) koff[i] = T::off(col, 4 * i + grp);
#pragma unroll
    for (int t = 0; t < DT; ++t) voff[t] = T::off(vrow, 2 * t + ((col & 3) >> 1)) + 8 * (col & 1);

    auto read_k = [&](const char* kb, half8_t (&kop)[KS][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < KS; ++i)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
                kop[i][hh] = __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4*>(kb + koff[i] + 16 * hh * T::ROW));
    };
    // S^T of a step (asm MFMAs; the scores pass score_fence before any VALU read)
    auto qk = [&](const half8_t (&kop)[KS][2], float4_t (&sv)[RT][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
            mfma4_first(sv[0][hh], sv[1][hh], sv[2][hh], sv[3][hh], kop[0][hh], qop[0][0], qop[1][0], qop[2][0],
                        qop[3][0]);
#pragma unroll
        for (int i = 1; i < KS; ++i)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
                mfma4_vacc(sv[0][hh], sv[1][hh], sv[2][hh], sv[3][hh], kop[i][hh], qop[0][i], qop[1][i], qop[2][i],
                           qop[3][i]);
        score_fence(sv);
    };
    // causal / context mask: key kbase + 16 hh + 4 grp + e < rctx
    auto mask = [&](const int kbase, float4_t (&sv)[RT][2]) __attribute__((always_inline)) {
        bool edge = false;
#pragma unroll
        for (int r = 0; r < RT; ++r) edge = edge || kbase + 32 > rctx[r];
        if (__builtin_amdgcn_ballot_w64(edge)) {
#pragma unroll
            for (int r = 0; r < RT; ++r)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (kbase + 16 * hh + 4 * grp + e >= rctx[r]) sv[r][hh][e] = -INFINITY;
        }
    };
    // This lane's max per row tile; true when some row exceeds its lazy limit
    auto lane_max = [&](const float4_t (&sv)[RT][2], float (&lmx)[RT]) __attribute__((always_inline)) {
        bool over = false;
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            lmx[r] = vmax3(vmax3(sv[r][0][0], sv[r][0][1], sv[r][0][2]), vmax3(sv[r][0][3], sv[r][1][0], sv[r][1][1]),
                           vmax3(sv[r][1][2], sv[r][1][3], sv[r][1][3]));
            over = over || lmx[r] > mlim[r];
        }
        return over;
    };
    // The lazy rescale (rows whose max exceeds m + kLazy reset m to the max
    // over their four key groups): rare, outside the overlapped regions.
    auto rescale = [&](const float (&lmx)[RT]) __attribute__((always_inline)) {
        // every row tile in one block (alpha 1 where the max stays): the code
        // sits in each step, so it is kept to one copy
        float alpha[RT];
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            alpha[r] = 1.0f;
            if (__builtin_amdgcn_ballot_w64(lmx[r] > mlim[r])) {
                const float mx = row_group_max(lmx[r]);
                const float mn = fmaxf(m[r], mx);
                alpha[r] = mn > m[r] ? __builtin_amdgcn_exp2f((m[r] - mn) * sc) : 1.0f;
                m[r] = mn;
                mlim[r] = mn + lazy;
                msc[r] = (mn == -INFINITY ? 0.0f : mn) * sc;
            }
        }
        agpr_fence(o, lsum);
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            lsum[r] *= alpha[r];
#pragma unroll
            for (int t = 0; t < DT; ++t) o[r][t] *= alpha[r];
        }
    };
    // ---------------- the tiles, pipelined.  Steps whose keys reach past some
    // row's context are masked: wmin, the smallest context of the wave's rows
    // (rows past the item have context 0 and are masked everywhere; their
    // output is not stored), decides on the scalar unit whether a step needs
    // the per-element test.
    int wmin;
    {
        float mn = 3.0e9f;
#pragma unroll
        for (int r = 0; r < RT; ++r)
            if (b * kRows + 16 * RT * wave + 16 * r + col < nrows) mn = fminf(mn, float(rctx[r]));
        wmin = __builtin_amdgcn_readfirstlane(int(-group_max<64>(-mn)));
    }
    auto mask_if = [&](const int kbase, float4_t (&sv)[RT][2]) __attribute__((always_inline)) {
        if (kbase + 32 > wmin) mask(kbase, sv);
    };
    float4_t sv[RT][2];   // scores of the step being finished
    half8_t kop[KS][2];   // K operands
    // Q lives in AGPRs (the asm MFMAs read it there); wait states between its
    // writes and the first MFMA reads
#pragma unroll
    for (int r = 0; r < RT; ++r)
        asm volatile("s_nop 4" : "+a"(qop[r][0]), "+a"(qop[r][1]), "+a"(qop[r][2]), "+a"(qop[r][3]));
    if (ntiles > 0) {
        publish_barrier(0);
        load_tile(2 % kW64Stages, 2);
        read_k(kstage(0), kop);
        qk(kop, sv);
        mask_if(0, sv);
        float lmx[RT];
        (void)lane_max(sv, lmx);
        // the first maximum: the running max starts at -inf, so this is the
        // rescale with nothing yet to rescale (the accumulators are zero)
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const float mx = row_group_max(lmx[r]);
            m[r] = mx;
            mlim[r] = mx + lazy;
            msc[r] = (mx == -INFINITY ? 0.0f : mx) * sc;
        }
        read_k(kstage(0) + 32 * T::ROW, kop);
    }
    // One step s: at entry the scores of s are computed, masked and rescaled
    // for, and the K operands of step s + 1 are read.  The step is placed by
    // hand, slot by slot (scheduling barriers between slots, its VALU work in
    // asm): one MFMA and a few VALU or LDS instructions per slot, so that the
    // lone wave of the SIMD issues VALU work while its MFMAs run.
    //   X: the V operands of s are read; 32 slots of one Q K^T MFMA of step
    //      s + 1, 24 of them beside one weight exp2(x sc - m sc) of step s
    //      (row tiles 0-2; pairs packed to fp16 a slot later);
    //   the scores of s + 1 wait out the MFMA-to-VALU distance and are masked
    //      where needed; `between` runs here (the barrier publishing the next
    //      tile, when the next K operands lie in it);
    //   Y: 36 slots of one P V (or row-sum) MFMA of step s, row tile by row
    //      tile, beside the K operand reads of step s + 2 (kn2), the weights
    //      of row tile 3 (done before its MFMAs) and this lane's row maxima
    //      of step s + 1;
    //   the rare rescale.
    // check = false discards the look-ahead (past the item's last tile).
    // dma: this step issues the loads of tile dt into stage dst, after the
    // barrier `between` (compile-time: the slots differ).
    auto pstep = [&](const char* vb, const char* kn2, const int kb_next, const bool check, auto between, auto dma,
                     const int dt, const int dst) __attribute__((always_inline)) {
        constexpr bool kDma = decltype(dma)::value;
        uint32_t pw[RT][4];  // weights of step s, fp16 pairs (the P^T operands)
        float wexp[RT][8];
        float4_t svn[RT][2];
        float lmx[RT];
        u32x2 vlo[DT], vhi[DT];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const int i = j >> 3, hh = (j >> 2) & 1, r = j & 3;
            if (i == 0) mfma_first_v(svn[r][hh], kop[0][hh], qop[r][0]);
            else mfma_acc_v(svn[r][hh], kop[i][hh], qop[r][i]);
            // V operands of step s: one transposed read per slot
            if (j < 16) {
                if (j & 1) vhi[j >> 1] = tr_read(vb + voff[j >> 1] + 16 * T::ROW);
                else vlo[j >> 1] = tr_read(vb + voff[j >> 1]);
            }
            // exps n = 3 (j / 4) + j % 4 for j % 4 < 3 (row tile n / 8, slot n % 8),
            // each odd n's pair packed in the next slot
            if ((j & 3) < 3) {
                const int n = 3 * (j >> 2) + (j & 3);
                wexp[n >> 3][n & 7] = slot_exp2(sv[n >> 3][(n & 7) >> 2][n & 3], sc, msc[n >> 3]);
            }
            if (j >= 3 && ((j - 3) & 3) < 3) {  // the pair ending in exp n, three slots later
                const int n = 3 * ((j - 3) >> 2) + ((j - 3) & 3);
                if (n & 1) pw[n >> 3][(n & 7) >> 1] = slot_pack(wexp[n >> 3][n & 6], wexp[n >> 3][n & 7]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // pairs whose pack slot falls past the last slot (n + 1 = 23: exp slot 30)
#pragma unroll
        for (int n = 0; n < 24; n += 2) {
            const int jn = 4 * ((n + 1) / 3) + (n + 1) % 3;
            if (jn + 3 >= 32) pw[n >> 3][(n & 7) >> 1] = slot_pack(wexp[n >> 3][n & 6], wexp[n >> 3][(n & 6) + 1]);
        }
        score_fence(svn);
        if (check) mask_if(kb_next, svn);
        between();
        __builtin_amdgcn_sched_barrier(0);
        half8_t pop[RT], vop[DT];
#pragma unroll
        for (int t = 0; t < DT; ++t) vop[t] = __builtin_bit_cast(half8_t, u32x4{vlo[t][0], vlo[t][1], vhi[t][0], vhi[t][1]});
        int dids[JW];
#pragma unroll
        for (int q = 0; q < 36; ++q) {
            const int r = q / 9, t = q % 9;
            if (t == 0) pop[r] = __builtin_bit_cast(half8_t, u32x4{pw[r][0], pw[r][1], pw[r][2], pw[r][3]});
            if (t == 0) mfma_acc_a(lsum[r], kOnes, pop[r]);
            else mfma_acc_a(o[r][t - 1], vop[t - 1], pop[r]);
            if (q < 8)
                kop[q >> 1][q & 1] = __builtin_bit_cast(
                    half8_t, *reinterpret_cast<const u32x4*>(kn2 + koff[q >> 1] + 16 * (q & 1) * T::ROW));
            // loads of tile dt: block ids read in slots 8-11, loads issued in 16-23
            if (kDma && q >= 8 && q < 8 + JW) dids[q - 8] = dma_id(dt, q - 8);
            if (kDma && q >= 16 && q < 16 + 2 * JW) {
                const int jj = (q - 16) >> 1;
                const uint64_t off = dma_off(dt, jj, dids[jj]);
                if ((q & 1) == 0) dma16(a.kc + off, dma_lds(dst, jj));
                else dma16(a.vc + off, dma_lds(dst, jj) + T::BYTES);
            }
            // row tile 3's weights: exps in slots 0-7, packs three slots after
            // the pair's second exp, in 4-10 (its MFMAs from slot 27)
            if (q < 8) wexp[3][q] = slot_exp2(sv[3][q >> 2][q & 3], sc, msc[3]);
            if (q >= 4 && q < 12 && (q & 1) == 0) pw[3][(q - 4) >> 1] = slot_pack(wexp[3][q - 4], wexp[3][q - 3]);
            // maxima of step s + 1 (lane-local, one row tile per 4 slots from slot 12)
            if (q >= 12 && q < 28) {  // (unused when the look-ahead is discarded)
                const int r2 = (q - 12) >> 2, k = (q - 12) & 3;
                if (k == 0) lmx[r2] = slot_max3(svn[r2][0][0], svn[r2][0][1], svn[r2][0][2]);
                if (k == 1) lmx[r2] = slot_max3(lmx[r2], svn[r2][0][3], svn[r2][1][0]);
                if (k == 2) lmx[r2] = slot_max3(lmx[r2], svn[r2][1][1], svn[r2][1][2]);
                if (k == 3) lmx[r2] = slot_max3(lmx[r2], svn[r2][1][3], svn[r2][1][3]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (check) {
            bool over = false;
#pragma unroll
            for (int r = 0; r < RT; ++r) over = over || lmx[r] > mlim[r];
            if (__builtin_amdgcn_ballot_w64(over)) rescale(lmx);
        }
#pragma unroll
        for (int r = 0; r < RT; ++r) sv[r][0] = svn[r][0], sv[r][1] = svn[r][1];
    };
    // Tile t in stage t % kW64Stages: step 2t (keys 0-31 of the tile), whose
    // look-ahead K operands (step 2t + 2) lie in tile t + 1, published by the
    // barrier between its two halves; then step 2t + 1.  The second step of
    // the last tile may lie wholly past the context: its keys are all masked
    // and add nothing.
    for (int t = 0; t < ntiles; ++t) {
        const int st = t % kW64Stages, st1 = (t + 1) % kW64Stages;
        pstep(vstage(st), kstage(st1), t * kBK + 32, true,
              [&]() __attribute__((always_inline)) { publish_barrier(t + 1); }, std::true_type(), t + 3,
              (t + 3) % kW64Stages);
        pstep(vstage(st) + 32 * T::ROW, kstage(st1) + 32 * T::ROW, t * kBK + kBK, t + 1 < ntiles,
              []() __attribute__((always_inline)) {}, std::false_type(), 0, 0);
    }
    wait_vmcnt<0>();  // no load of this item may land in the next item's buffers

    // ---------------- output through LDS (16 KiB per wave, in the tile buffers)
    __syncthreads();  // every wave's loads have landed and no wave reads a tile
    agpr_fence(o, lsum);
    static_assert(64 * D * EB * kW64Waves <= kW64Stages * 2 * T::BYTES, "the output fits in the tile buffers");
    float inv[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const float lt = lsum[r][0];
        inv[r] = (rctx[r] > 0 && lt > 0.0f) ? 1.0f / lt : 0.0f;
    }
    store_rows_lds<D, RT>(a, buf.tiles + wave * (64 * D * EB), o, inv, b * kRows + 64 * wave, nrows, q0, kvh, lane);
}

template <int D>
__device__ __forceinline__ void w64_items(const PrefillArgs& a, const W64Buffers& buf) {
    run_items<64 * kW64Waves>(a, [&](const PrefillItem& it) __attribute__((always_inline)) {
        prefill_block_w64<D>(a, it, buf);
    });
}

template <int D>
__global__ __launch_bounds__(64 * kW64Waves) __attribute__((amdgpu_waves_per_eu(1, 1)))
void prefill_w64_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(1024))) char tiles[kW64Stages * 2 * DmaTile<D>::BYTES];
    __shared__ int btc[kWideBtc];
    const W64Buffers buf = {tiles, btc};
    w64_items<D>(a, buf);
}

// FP8 caches at D = 128: three stages of code tiles and scales, one fp16 tile.
__global__ __launch_bounds__(64 * kWideWaves) void prefill_wide8_kernel(PrefillArgs a) {
    constexpr int D = 128;
    __shared__ __attribute__((aligned(1024))) char k0[DmaTile<D>::BYTES];
    __shared__ __attribute__((aligned(1024))) char v0[DmaTile<D>::BYTES];
    __shared__ __attribute__((aligned(1024))) char fk0[DmaTile8<D>::BYTES];
    __shared__ __attribute__((aligned(1024))) char fk1[DmaTile8<D>::BYTES];
    __shared__ __attribute__((aligned(1024))) char fk2[DmaTile8<D>::BYTES];
    __shared__ __attribute__((aligned(1024))) char fv0[DmaTile8<D>::BYTES];
    __shared__ __attribute__((aligned(1024))) char fv1[DmaTile8<D>::BYTES];
    __shared__ __attribute__((aligned(1024))) char fv2[DmaTile8<D>::BYTES];
    __shared__ __attribute__((aligned(256))) float sc0[2 * kBK];
    __shared__ __attribute__((aligned(256))) float sc1[2 * kBK];
    __shared__ __attribute__((aligned(256))) float sc2[2 * kBK];
    __shared__ int btc[kWideBtc];
    const WideBuffers buf = {{k0, nullptr, nullptr}, {v0, nullptr, nullptr}, btc, {fk0, fk1, fk2},
                             {fv0, fv1, fv2}, {sc0, sc1, sc2}};
    wide_items<D, true>(a, buf);
}

// Work list of the matrix-core kernels, in one workgroup: items (s, b * Hkv +
// kvh), row block b of every sequence with >= 2 query tokens, ordered by the
// number of key tiles they stage, most first, so that persistent workgroups
// taking them in turn (dealt in a snake by the direct-load kernels, claimed by
// prefill_mfma_kernel) form a longest-processing-time schedule (short items
// fill in at the end).  A row block of rows_per_item rows (query tokens
// times row_mult heads) sees keys 0 .. kend - 1 with kend = prior + its last
// token + 1; a histogram over the tile counts (one bin per possible count,
// at most kMaxLevels: counts past that share the top bin) gives every count's
// offset, and the blocks take their
// slots through LDS atomics (the order within a bin does not matter to the
// results).
constexpr int kMaxLevels = 4096;
constexpr int kMaxHeadGroups = 63;  // claim counters after the item count (256-byte header)

// Exclusive prefix sum of arr[0, n) in LDS by 256 threads (each a contiguous
// tile, tiles combined with DPP wave scans and one LDS step); returns the total.
__device__ int block_exclusive_scan(int* arr, int n, int* wave_tot) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int per = (n + 255) / 256;
    const int b = tid * per;
    int local = 0;
    for (int i = 0; i < per; ++i)
        if (b + i < n) local += arr[b + i];
    const int incl = wave_incl_scan(local);
    if (lane == 63) wave_tot[wave] = incl;
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; ++w) before += wave_tot[w];
    const int total = wave_tot[0] + wave_tot[1] + wave_tot[2] + wave_tot[3];
    int run = before + incl - local;
    for (int i = 0; i < per; ++i) {
        if (b + i < n) {
            const int v = arr[b + i];
            arr[b + i] = run;
            run += v;
        }
    }
    __syncthreads();  // (wave_tot may be reused by the next scan)
    return total;
}

__global__ __launch_bounds__(256) void prefill_items_kernel(const int32_t* qsl, const int32_t* cl, int32_t num_seqs,
                                                            int32_t hkv, int32_t row_mult, int32_t rows_per_item,
                                                            int32_t max_qblocks, int32_t table_tokens, int32_t nbins,
                                                            int2* items, int32_t* count) {
    __shared__ int off[kMaxLevels];   // items per bin, then bin offsets (nbins used)
    __shared__ int fill[kMaxLevels];  // slots taken per bin
    __shared__ int wave_tot[4];
    const int tid = threadIdx.x;
    for (int i = tid; i < nbins; i += 256) off[i] = fill[i] = 0;
    __syncthreads();
    auto blocks = [&](int q) { return seq_row_blocks(q, row_mult, rows_per_item, max_qblocks); };
    auto bin = [&](int prior, int q, int b) {
        return row_block_bin(prior, q, b, row_mult, rows_per_item, table_tokens, nbins);
    };
    for (int s = tid; s < num_seqs; s += 256) {
        const int q = qsl[s + 1] - qsl[s];
        const int prior = cl[s] - q;
        const int n = blocks(q);
        for (int b = 0; b < n; ++b) atomicAdd(&off[bin(prior, q, b)], hkv);
    }
    __syncthreads();
    const int total = block_exclusive_scan(off, nbins, wave_tot);
    if (tid == 0) count[0] = total;
    if (tid < kMaxHeadGroups) count[1 + tid] = 0;  // claim counters of the prefill kernel
    for (int s = tid; s < num_seqs; s += 256) {
        const int q = qsl[s + 1] - qsl[s];
        const int prior = cl[s] - q;
        const int n = blocks(q);
        for (int b = 0; b < n; ++b) {
            const int k0 = bin(prior, q, b);
            const int pos = off[k0] + atomicAdd(&fill[k0], hkv);
            for (int k = 0; k < hkv; ++k) items[pos + k] = int2{s, b * hkv + k};
        }
    }
}

int ilog2i(int x) {
    int r = 0;
    while ((1 << r) < x) ++r;
    return r;
}

}  // namespace

bool prefill_mfma_supported(const vkv_prefill_params* p) {
    // 16-byte direct/vector loads of K, V and Q rows; power-of-two blocks
    const int64_t qs = p->query_stride ? p->query_stride : int64_t(p->num_heads) * p->head_dim;
    const uintptr_t align = reinterpret_cast<uintptr_t>(p->key_cache) | reinterpret_cast<uintptr_t>(p->value_cache) |
                            reinterpret_cast<uintptr_t>(p->query) | uintptr_t(qs * 2);
    const bool pow2_bs = p->block_size >= 1 && p->block_size <= 1024 && (p->block_size & (p->block_size - 1)) == 0;
    return p->io_dtype == VKV_DTYPE_F16 && (p->kv_dtype == VKV_DTYPE_F16 || p->kv_dtype == VKV_DTYPE_FP8_E4M3) &&
           (p->head_dim == 64 || p->head_dim == 128) && p->max_query_len >= 2 && pow2_bs && (align & 15u) == 0 &&
           p->num_kv_heads > 0 && p->num_heads % p->num_kv_heads == 0 &&
           p->num_heads / p->num_kv_heads <= kMaxHeadGroups * kMaxWaves;
}

namespace {

// D = 128, and fp16 caches at D = 64 with groups below 4 heads, run on the
// direct-load kernels, whose items are Wide<D>::ROWS (token, head) rows; the
// rest of D = 64 on prefill_mfma_kernel, whose items are kBQ query tokens of
// every head of a kv head (a wave per head, at least 4 waves: smaller groups
// would leave waves idle).  Measured on C3's chunks at D = 64, fp16 cache:
// groups of 7 73.5 us on the staged kernel against 88.0 on the direct-load
// one, groups of 4 89.2 against 91.7, groups of 1 138.4 against 101.8.
bool wide_path(const vkv_prefill_params* p) {
    if (p->head_dim == 128) return true;
    const int G = p->num_kv_heads > 0 ? p->num_heads / p->num_kv_heads : 1;
    return p->kv_dtype == VKV_DTYPE_F16 && (VKV_PREFILL_D64_WIDE || G < kMinWaves);
}
int rows_per_item(const vkv_prefill_params* p) {
    if (!wide_path(p)) return kBQ;
    return p->head_dim == 128 ? Wide<128>::ROWS : Wide<64>::ROWS;
}
// Row blocks (work items per kv head) of a sequence, at most: with a group of
// G heads a token brings G rows to the direct-load kernels.
int64_t max_row_blocks(const vkv_prefill_params* p) {
    const int64_t row_mult = wide_path(p) ? p->num_heads / p->num_kv_heads : 1;
    const int rows = rows_per_item(p);
    return (int64_t(p->max_query_len) * row_mult + rows - 1) / rows;
}

}  // namespace

size_t prefill_items_bytes(const vkv_prefill_params* p) {
    return 256 + size_t(int64_t(p->num_seqs) * max_row_blocks(p) * p->num_kv_heads) * sizeof(int2);
}

int launch_prefill_mfma(const vkv_prefill_params* p, void* item_space, hipStream_t st) {
    PrefillArgs a;
    a.out = static_cast<_Float16*>(p->output);
    a.q = static_cast<const char*>(p->query);
    a.kc = static_cast<const char*>(p->key_cache);
    a.vc = static_cast<const char*>(p->value_cache);
    a.ks = p->key_scales;
    a.vs = p->value_scales;
    a.bt = p->block_tables;
    a.cl = p->context_lens;
    a.qsl = p->query_start_loc;
    a.q_stride = p->query_stride ? p->query_stride : int64_t(p->num_heads) * p->head_dim;
    a.num_heads = p->num_heads;
    a.num_kv_heads = p->num_kv_heads;
    a.group = p->num_heads / p->num_kv_heads;
    // wide_path(): prefill_w64_kernel / prefill_wide_kernel /
    // prefill_wide8_kernel, Wide<D>::ROWS (token, head) rows per item; else
    // prefill_mfma_kernel, up to kMaxWaves heads x kBQ tokens per item
    const bool wide = wide_path(p);
    const int head_groups = wide ? 1 : (a.group + kMaxWaves - 1) / kMaxWaves;
    a.heads_per_wg = (a.group + head_groups - 1) / head_groups;
    a.bs_log2 = ilog2i(p->block_size);
    a.max_blocks_per_seq = p->max_blocks_per_seq;
    a.num_blocks = p->num_blocks;
    // keys any row may see: the table, and the caller's max_context_len clamp
    int64_t tt = int64_t(p->max_blocks_per_seq) * p->block_size;
    if (p->max_context_len > 0 && p->max_context_len < tt) tt = p->max_context_len;
    a.table_tokens = int32_t(tt > 0x7FFFFFFF ? 0x7FFFFFFF : tt);
    const int row_mult = wide ? a.group : 1;
    const int rpi = rows_per_item(p);
    a.qblocks = int(max_row_blocks(p));
    a.num_seqs = p->num_seqs;
    a.scale_log2 = logit_scale_log2(p->scale);
    int32_t* count = static_cast<int32_t*>(item_space);
    int2* items = reinterpret_cast<int2*>(static_cast<char*>(item_space) + 256);
    a.items = items;
    a.item_count = count;
    // bins: every possible tile count (items past kMaxLevels - 1 tiles share the last)
    const int64_t max_tiles = (int64_t(a.table_tokens) + kBK - 1) / kBK;
    const int nbins = int(max_tiles + 1 < kMaxLevels ? max_tiles + 1 : kMaxLevels);
    a.rows_per_item = rpi;
    a.nbins = nbins;
    // Row blocks, at most: a sequence of q >= 2 tokens has ceil(q G / R) <=
    // q G / R + 1 of them, and there are at most min(S, T / 2) such sequences
    // (T query tokens).  Small calls order them in the kernel itself.
    const int64_t T = p->num_query_tokens;
    const int64_t nseq2 = p->num_seqs < T / 2 ? p->num_seqs : T / 2;
    const int64_t bound = T * row_mult / rpi + nseq2;
    // a host-built list (wide kernels only) replaces both in-kernel orderings
    a.work_list = wide && p->work_list && p->work_list_words > kListHeaderWords ? p->work_list : nullptr;
    a.work_list_words = a.work_list ? p->work_list_words : 0;
    a.num_query_tokens = int32_t(p->num_query_tokens);
    {
        int sh = 0;
        while ((int64_t(1) << sh) < a.group) ++sh;
        const uint64_t m = ((uint64_t(1) << (32 + sh)) + uint64_t(a.group) - 1) / uint64_t(a.group);
        a.group_div_m = uint32_t(m - (uint64_t(1) << 32));
        a.group_div_s = sh;
    }
    a.inline_list = !a.work_list && wide && bound <= kInlineBlocks;
    if (!a.inline_list && !a.work_list)
        hipLaunchKernelGGL(prefill_items_kernel, dim3(1), dim3(256), 0, st, p->query_start_loc, p->context_lens,
                           p->num_seqs, p->num_kv_heads, row_mult, rpi, a.qblocks, a.table_tokens, nbins,
                           items, count);
    // Persistent grid, never more workgroups than there can be items: one per
    // CU for the wide kernel (its LDS and registers fill a CU); two per CU for
    // the FP8 kernel (at D = 128 one is resident, the other starts when a CU
    // frees up).
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const int64_t upper = int64_t(p->num_seqs) * a.qblocks * p->num_kv_heads;
    const int64_t per_cu = wide ? 1 : 2;
    const int64_t wgs = int64_t(cus) * per_cu < upper ? int64_t(cus) * per_cu : upper;
    const bool w64 = VKV_PREFILL_W64 && p->head_dim == 128 && p->kv_dtype == VKV_DTYPE_F16;
    const int waves = w64 ? kW64Waves : wide ? kWideWaves : (a.heads_per_wg < kMinWaves ? kMinWaves : a.heads_per_wg);
    const dim3 grid(unsigned(wgs > 0 ? wgs : 1), 1u, unsigned(head_groups));
    const dim3 block(unsigned(64 * waves));
    if (p->head_dim == 128) {
        if (w64) hipLaunchKernelGGL((prefill_w64_kernel<128>), grid, block, 0, st, a);
        else if (p->kv_dtype == VKV_DTYPE_F16) hipLaunchKernelGGL((prefill_wide_kernel<128>), grid, block, 0, st, a);
        else hipLaunchKernelGGL(prefill_wide8_kernel, grid, block, 0, st, a);
    } else {
        if (wide) hipLaunchKernelGGL((prefill_wide_kernel<64>), grid, block, 0, st, a);
        else if (p->kv_dtype == VKV_DTYPE_F16) hipLaunchKernelGGL((prefill_mfma_kernel<64, kF16>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((prefill_mfma_kernel<64, kFp8>), grid, block, 0, st, a);
    }
    return 0;
}

int64_t prefill_work_list_host(const vkv_prefill_params* p, const int32_t* host_qsl, const int32_t* host_cl,
                               int32_t* out, int64_t capacity) {
    if (!p || !host_qsl || !host_cl) return -1;
    if (p->num_seqs <= 0 || !prefill_mfma_supported(p) || !wide_path(p)) return 0;  // no list for this call
    const int G = p->num_heads / p->num_kv_heads, hkv = p->num_kv_heads;
    const int rpi = rows_per_item(p);
    const int64_t qblocks = max_row_blocks(p);
    int64_t tt = int64_t(p->max_blocks_per_seq) * p->block_size;
    if (p->max_context_len > 0 && p->max_context_len < tt) tt = p->max_context_len;
    // items in (s, b, kvh) order with their key tiles
    struct Item {
        int32_t s, b, kvh, q0, qlen, prior, tiles;
    };
    std::vector<Item> items;
    for (int32_t s = 0; s < p->num_seqs; ++s) {
        const int64_t q = int64_t(host_qsl[s + 1]) - host_qsl[s];
        if (q < 2) continue;
        const int64_t prior = int64_t(host_cl[s]) - q;
        int64_t nb = (q * G + rpi - 1) / rpi;
        nb = nb < qblocks ? nb : qblocks;
        for (int64_t b = 0; b < nb; ++b) {
            const int64_t last = ((b + 1) * rpi - 1) / G + 1;
            int64_t kend = prior + (last < q ? last : q);
            kend = kend < tt ? kend : tt;
            const int32_t tiles = int32_t(kend > 0 ? (kend + kBK - 1) / kBK : 0);
            for (int k = 0; k < hkv; ++k)
                items.push_back(Item{s, int32_t(b), k, host_qsl[s], int32_t(q), int32_t(prior), tiles});
        }
    }
    // one list per workgroup of the persistent grid (one per CU)
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess || cus <= 0) {
        cus = kListDefaultCus;
        (void)hipGetLastError();  // (no device: the default, and no error left behind)
    }
    const int64_t n = int64_t(items.size());
    const int64_t lists = n < cus ? (n > 0 ? n : 1) : cus;
    // Longest first (ties in (s, b, kvh) order), each item to the list with
    // the least work so far (ties: the lowest list).
    std::stable_sort(items.begin(), items.end(), [](const Item& u, const Item& v) { return u.tiles > v.tiles; });
    std::vector<std::vector<int32_t>> dealt{static_cast<size_t>(lists)};
    typedef std::pair<int64_t, int64_t> Load;  // (work, list)
    std::priority_queue<Load, std::vector<Load>, std::greater<Load>> least;
    for (int64_t w = 0; w < lists; ++w) least.push(Load(0, w));
    for (int64_t i = 0; i < n; ++i) {
        Load l = least.top();
        least.pop();
        dealt[size_t(l.second)].push_back(int32_t(i));
        l.first += items[size_t(i)].tiles + kListItemStartTiles;
        least.push(l);
    }
    size_t len = 0;
    for (const auto& d : dealt) len = d.size() > len ? d.size() : len;
    const int64_t words = kListHeaderWords + int64_t(kListItemWords) * lists * int64_t(len);
    if (!out) return words;
    if (capacity < words) return -2;
    std::fill(out, out + words, 0);
    out[0] = int32_t(lists);
    out[1] = int32_t(len);
    out[2] = kListFormat;
    out[3] = int32_t(n);
    for (int64_t w = 0; w < lists; ++w)
        for (size_t k = 0; k < len; ++k) {
            int32_t* e = out + kListHeaderWords + (int64_t(k) * lists + w) * kListItemWords;
            if (k < dealt[size_t(w)].size()) {
                const Item& it = items[size_t(dealt[size_t(w)][k])];
                const int32_t v[kListItemWords] = {it.s, it.b, it.kvh, it.q0, it.qlen, it.prior, it.tiles, 0};
                std::copy(v, v + kListItemWords, e);
            } else {
                e[0] = -1;  // the list has ended
            }
        }
    return words;
}

}  // namespace vkv

