// decode_common.hpp — what the split-K decode kernels of decode.hip (fixed
// shapes) and decode_generic.hip (any head_dim, group size and block size)
// share: the argument block, the row helpers, the per-lane K/V loads, the
// device-side partition choice and the persistent item loop.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>

#include "common.hpp"
#include "launch.hpp"

namespace vkv {
namespace dec {

constexpr int kWavesPerBlock = 4;
static_assert(kWave * kWavesPerBlock == kBlockThreads, "partition kernels launch kBlockThreads threads");
// Workspace layout: a 1 KiB header holding the work-claim counters (zero
// between calls: the merge kernel resets them) and int kChosenPartitionSlot
// (the partition size the partition kernel chose, for the merge kernel),
// followed by the partials.
constexpr size_t kWorkspaceHeader = 1024;
constexpr int kClaimSequences = 8;
constexpr int kCounterStride = 32;  // ints: one 128-byte line per counter
constexpr float kLog2e = 1.4426950408889634f;
// Fixed cost of one item (partial write, merge input, chain start-up) in
// token-equivalents, for the span estimate of the partition choice.
constexpr int kItemOverheadTokens = 128;
// LDS per CU on gfx950, for the resident-wave estimate.
constexpr int kLdsPerCu = 160 * 1024;
// Rows (sequences or query rows) per partition launch: the kernel keeps one
// prefix entry per row in LDS.  Larger calls run as consecutive launches.
constexpr int kMaxRowsPerLaunch = 8192;
// Rows of the largest launch of a call (the partials are sized for it).
inline int launch_rows_max(int num_rows) { return num_rows < kMaxRowsPerLaunch ? num_rows : kMaxRowsPerLaunch; }

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
    // Mixed prefill batch (rows = sequences): query_start_loc.  Only sequences
    // with one query token are decoded here (query row qsl[s]); the others
    // belong to the prefill kernel and have no partitions.
    const int32_t* qsl;
    // Partials, item-major so that one item's G heads are contiguous:
    // slot ((s * Hkv + kvh) * max_parts + part) * G + g for head kvh * G + g.
    float* part_o;   // [S][Hkv][max_parts][G][D]
    float* part_ml;  // [S][Hkv][max_parts][G][2] (max in log2 domain, sum)
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
    int32_t num_rows;         // sequences (decode) or query rows (prefill)
    int* counters;            // the workspace header ints (claim counters zero between calls)
    int32_t mfma_enabled;     // use the matrix-core QK^T variant where it applies
    // num_cands > 1: P is the default size, the kernel picks the partition
    // size among cands (ascending) and records it in the workspace header.
    int32_t num_cands;
    int32_t cands[kMaxPartitionCandidates];
    int32_t wave_slots;       // waves of this launch resident at once (estimate)
    int32_t level_waves;      // waves of one workgroup per CU (one wave per SIMD)
    // generic variant (any head_dim / group size / block size) only
    int32_t head_dim;
    int32_t block_size;
    int32_t io_f32;           // query and output are fp32 (else fp16)
    int32_t vec_loads;        // whole-vector K/V loads (head_dim and cache alignment allow them)
    // n / block_size for 0 <= n < 2^31 as (n + mulhi(n, bs_div_m)) >> bs_div_s
    // (bs_div_s = ceil(log2 block_size), bs_div_m = ceil(2^(32 + s) / block_size)
    // - 2^32: exact for such n, see block_div)
    uint32_t bs_div_m;
    int32_t bs_div_s;
    // > 0: small call, one item per wave of a grid that covers every
    // (row, partition < static_parts, sub-item) at partition size P: no
    // prefix scan, no claims, and items request their block ids together with
    // the context length.  0: the persistent claim loop.
    int32_t static_parts;
    // Append fused into the call (source rows in the cache's element type,
    // fp16 or fp32; fixed shapes): row s's new token is fkey / fval + s *
    // stride (bytes), bound for cache slot fslots[s].  The partition kernel
    // reads row s's last position from these rows when that position's slot
    // is fslots[s] (its K/V as the append would leave them); the merge kernel
    // stores the rows into slots in [0, fnum_slots).  fkey == NULL: no append.
    const char* fkey;
    const char* fval;
    int64_t fkey_stride;
    int64_t fval_stride;
    int32_t fbytes;  // element bytes of the rows and the cache (2 or 4)
    const int32_t* fslots;
    int64_t fnum_slots;
};

// The new token of an appending decode call (see DecodeArgs::fkey).
struct FusedAppend {
    const char* key;
    const char* value;
    int64_t key_stride;  // bytes
    int64_t value_stride;
    int32_t elem_bytes;
    const int32_t* slots;
    int64_t num_slots;
};

// The shapes decode.hip's fixed-shape kernels are built for; every other
// shape runs on decode_generic.hip.
inline bool fixed_decode_shape(int head_dim, int group, int block_size, const void* kc, const void* vc) {
    const bool pow2_bs = block_size > 0 && block_size <= 1024 && (block_size & (block_size - 1)) == 0;
    const bool aligned = ((reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc)) & 15u) == 0;
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) && group >= 1 && group <= 8 && pow2_bs && aligned;
}

// Partition kernel of the generic variant (decode_generic.hip) for one launch
// of rows; max_pairs bounds the (row, partition) pairs.  0 or VKV_ERR_*.
int launch_decode_generic(DecodeArgs& a, int kv_dtype, int64_t max_pairs, size_t lds, hipStream_t st);

// n / block_size by the multiplier of DecodeArgs::bs_div_m: with m = 2^32 +
// bs_div_m = ceil(2^(32+s) / d), n m / 2^(32+s) = n / d + n e / (d 2^(32+s))
// for e = m d - 2^(32+s) < d, and that last term is below 1 / d for n < 2^31,
// so the floor is exact (division by invariant integers, Granlund and
// Montgomery 1994).
__device__ __forceinline__ int block_div(const DecodeArgs& a, const int n) {
    return int((uint32_t(n) + __umulhi(uint32_t(n), a.bs_div_m)) >> a.bs_div_s);
}
inline void set_block_div(DecodeArgs& a, int block_size) {
    int s = 0;
    while ((int64_t(1) << s) < block_size) ++s;
    const uint64_t m = ((uint64_t(1) << (32 + s)) + uint64_t(block_size) - 1) / uint64_t(block_size);
    a.bs_div_m = uint32_t(m - (uint64_t(1) << 32));
    a.bs_div_s = s;
}

// Keys row r attends (clamped to the table) and the query/output row it uses.
__device__ __forceinline__ int row_context(const DecodeArgs& a, int r) {
    int ctx;
    if (a.row_ctx) ctx = a.row_ctx[r];
    else if (a.qsl) ctx = (a.qsl[r + 1] - a.qsl[r] == 1) ? a.cl[r] : 0;
    else ctx = a.cl[r];
    return ctx < a.max_ctx ? ctx : a.max_ctx;
}
__device__ __forceinline__ int64_t query_row(const DecodeArgs& a, int r) { return a.qsl ? a.qsl[r] : r; }

template <int KVT>
struct LaneLoad {
    static constexpr int bytes = KVT == kFp8 ? 8 : 16;  // bytes per lane per load
    static constexpr int words = bytes / 4;
    static constexpr int elems = bytes / KvTraits<KVT>::bytes;
};

// K/V lane loads are non-temporal: every cache byte is read once per call, so
// the stream should not displace other lines (measured: 14% faster gathers).
template <int KVT>
__device__ __forceinline__ void load_lane(const char* p, uint32_t* w) {
    if constexpr (LaneLoad<KVT>::bytes == 16) {
        const u32x4 v = load16_nt(p);
        w[0] = v[0];
        w[1] = v[1];
        w[2] = v[2];
        w[3] = v[3];
    } else {
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
        w[0] = v[0];
        w[1] = v[1];
    }
}

// Unpack one lane load into EPL floats in dimension order.  FP8 values come out
// scaled by 2^-8 (the caller folds 256 into its per-token scale).
template <int KVT>
__device__ __forceinline__ void unpack_lane(const uint32_t* w, float* v) {
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
        for (int i = 0; i < 2; ++i) {
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

// Partition size of a call that left it to the library.  Every workgroup
// evaluates the same candidates over the rows' context lengths (each thread
// brings its row tile's partition count per candidate), so all reach the same
// size.  One workgroup per CU puts one wave on each SIMD (level_waves waves),
// so n items stack ceil(n / level_waves) waves on the busiest SIMDs, and a
// SIMD's waves share its issue slots and memory pipeline: the call takes
// about ceil(items / level_waves) x (P + kItemOverheadTokens), the cost the
// candidates compete on (ties: the smaller size).  Items beyond the
// wave_slots resident waves wait for a wave to finish, which the same count
// covers.  C2's batch (8 kv heads, 64 rows; 1 024 waves per level) measured
// 97.8 us at 656 tokens (2 016 items, cost 2 x 784), 98.4 at 672, 99.5 at
// 688, 102.2 at 448 (2 840 items, 3 x 576), 102.8 at 768 (1 784 items,
// 2 x 896), 106.4 at 512, 110.5 at 544, 113.5 at 576 and 117.7 at 608
// (2 160 items, 3 x 736): time rises with the cost throughout, except that a
// nearly empty extra level costs less (107.5 us at 640: 2 064 items); among
// the candidates it takes 656 (2 016 items, 2 x 784).  C3's decode rows (two
// waves per SIMD resident) take 1 280 tokens (2 044 items, 2 x 1 408), the
// fastest of a sweep: 198.8 us, against 200.7 at 1 152, 210.0 at 768, 212.2
// at 1 536, 223.3 at 960 and 238.0 at 2 048.  Two cases keep the
// default: default-size items of at most one level (small batches, which the
// host already split finer), and beyond two rounds of resident waves, where
// waves that claim items as they finish fill the last round with the short
// final partitions of the rows (C5's batch, 3.3 rounds at 768 tokens:
// 345 us at 768 against 356 at 640 and 354-356 at 896 to 1 536).
__device__ inline int choose_partition(const DecodeArgs& a, const int (&cnt)[kMaxPartitionCandidates]) {
    __shared__ int sums[kWavesPerBlock][kMaxPartitionCandidates];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
#pragma unroll
    for (int c = 0; c < kMaxPartitionCandidates; ++c) {
        const int v = __builtin_amdgcn_readlane(wave_incl_scan(cnt[c]), kWave - 1);
        if (lane == 0) sums[wave][c] = v;
    }
    __syncthreads();
    const unsigned W = a.wave_slots > 0 ? unsigned(a.wave_slots) : 1u;
    const unsigned L = a.level_waves > 0 ? unsigned(a.level_waves) : 1u;
    const unsigned cap = 0x7FFFFFFFu / unsigned(a.num_kv_heads);
    unsigned items0 = 0;
    uint64_t best_cost = ~uint64_t(0);
    int best = a.P;
#pragma unroll
    for (int c = 0; c < kMaxPartitionCandidates; ++c) {
        if (c >= a.num_cands) break;
        unsigned pairs = 0;
#pragma unroll
        for (int w = 0; w < kWavesPerBlock; ++w) pairs += unsigned(sums[w][c]);
        const unsigned items = (pairs < cap ? pairs : cap) * unsigned(a.num_kv_heads);
        if (a.cands[c] == a.P) items0 = items;
        const uint64_t cost = uint64_t((items + L - 1) / L) * unsigned(a.cands[c] + kItemOverheadTokens);
        if (cost < best_cost) {
            best_cost = cost;
            best = a.cands[c];
        }
    }
    return (items0 <= L || items0 > 2 * W) ? a.P : best;
}

// Longest-first order of the pairs of a call whose items take more than one
// round of the resident waves (rows <= kLptMaxRows, so that the host's LDS
// holds the lists below): waves that finish claim the next items, and with
// the rows' short final partitions spread through a row-major list the last
// round ends with long items started late while other waves sit idle (C5's
// batch ran 5 % below the bandwidth of the same batch with every context a
// multiple of the partition).  So the full partitions of every row come
// first (row-major), then each row's short final partition, longest first,
// in kLptBins length classes (rows in order within a class).  Every
// workgroup derives the same order from the context lengths.
constexpr int kLptMaxRows = 512;
constexpr int kLptBins = 64;
// Extra dynamic LDS of a launch of n rows for that order (the row prefix of
// (n + 1) ints comes first).
inline size_t lpt_lds_bytes(int n) { return n <= kLptMaxRows ? size_t(2) * size_t(n) * sizeof(int) : 0; }

// The item loop of the persistent partition kernels.  Items are numbered
// densely, pair-major: pair = (row, partition), items_per_pair items each
// (kv heads, or kv heads x query-head chunks), so no wave is launched for a
// partition that does not exist (the context lengths live on the device, so
// a fixed grid would carry many empty slots for long-tailed batches) and the
// waves of a workgroup hold adjacent items of the same blocks.  Workgroups
// claim item groups dynamically, so all stay busy until the list runs out.
// Nothing waits on another workgroup.  item(P, row, partition, sub) runs
// one item on the calling wave.
// DEAL: items dealt in a snake (no claims); otherwise claimed through the
// workspace counters.
template <bool STATIC = false, bool DEAL = false, class Item>
__device__ __forceinline__ void run_partitions(const DecodeArgs& a, const int items_per_pair, Item&& item) {
    extern __shared__ int prefix[];  // [num_rows + 1] exclusive prefix of partitions per row
    const int lane = threadIdx.x & (kWave - 1);
    const int nrows = a.num_rows;
    // STATIC (small calls, static_parts > 0): one item per wave of a grid
    // covering every (row, partition < static_parts, sub-item), no prefix
    // scan, no claims.
    constexpr bool stat = STATIC;
    const int wave = threadIdx.x / kWave;
    int P = a.P;
    int num_items = nrows * a.static_parts * items_per_pair;
    bool lpt = false;
    int num_full = 0;
    int* shortlist = prefix + (nrows + 1);  // [nrows]: rows of the short final partitions, longest first
    if constexpr (!stat) {
        // Partitions per row and their exclusive prefix, scanned by the whole
        // workgroup: each thread sums a contiguous tile of rows, the 256 tile sums
        // are scanned with DPP wave scans plus one LDS step, then each thread writes
        // its tile's prefix entries.  A call that leaves the partition size to the
        // library counts its tile for every candidate size in the same pass and
        // picks the size first (power-of-two block sizes only).
        __shared__ int wave_total[kWavesPerBlock];
        auto parts_of = [&](int r) {
            const int ctx = row_context(a, r);
            return ctx > 0 ? (ctx + P - 1) / P : 0;
        };
        const int per = (nrows + kBlockThreads - 1) / kBlockThreads;
        const int r0 = int(threadIdx.x) * per;
        int local = 0;
        if (a.num_cands > 1) {
            int cnt[kMaxPartitionCandidates];
#pragma unroll
            for (int c = 0; c < kMaxPartitionCandidates; ++c) cnt[c] = 0;
            for (int i = 0; i < per; ++i) {
                const int ctx = r0 + i < nrows ? row_context(a, r0 + i) : 0;
                if (ctx > 0) {
                    // candidates are block multiples m * bs: ceil(ctx / (m * bs)) = ceil(nb / m)
                    const int nb = ((ctx - 1) >> a.bs_log2) + 1;
#pragma unroll
                    for (int c = 0; c < kMaxPartitionCandidates; ++c) {
                        const int m = a.cands[c] >> a.bs_log2;  // >= 1 (the host pads unused entries)
                        cnt[c] += (nb + m - 1) / m;
                    }
                }
            }
            P = __builtin_amdgcn_readfirstlane(choose_partition(a, cnt));  // wave-uniform: keep it scalar
#pragma unroll
            for (int c = 0; c < kMaxPartitionCandidates; ++c)
                if (a.cands[c] == P) local = cnt[c];
            // for the merge kernel (same stream, after this grid)
            if (blockIdx.x == 0 && threadIdx.x == 0) a.counters[kChosenPartitionSlot] = P;
        } else {
            for (int i = 0; i < per; ++i)
                if (r0 + i < nrows) local += parts_of(r0 + i);
        }
        const int incl = wave_incl_scan(local);
        if (lane == kWave - 1) wave_total[wave] = incl;
        __syncthreads();
        int before = 0;
        for (int w = 0; w < wave; ++w) before += wave_total[w];
        int run = before + incl - local;
        for (int i = 0; i < per; ++i) {
            if (r0 + i < nrows) {
                prefix[r0 + i] = run;
                run += parts_of(r0 + i);
            }
        }
        if (threadIdx.x == kBlockThreads - 1) prefix[nrows] = before + incl;
        __syncthreads();
        const int num_pairs = prefix[nrows];
        num_items = num_pairs * items_per_pair;

        // Longest-first order (above).  prefix becomes the exclusive prefix of the
        // rows' full partitions (the last one counts when it is full); the short
        // final partitions follow in shortlist, their row's partition index being
        // its full count.
        lpt = nrows <= kLptMaxRows && num_items > a.wave_slots;
        int* bins = shortlist + nrows;          // [nrows]: length class of a row's short final partition, -1 none
        if (lpt) {
            int full_r[kLptMaxRows / 256 + 1];  // this thread's rows r = tid + 256 j
#pragma unroll
            for (int j = 0; j * 256 < kLptMaxRows; ++j) {
                const int r = int(threadIdx.x) + 256 * j;
                full_r[j] = 0;
                if (r < nrows) {
                    const int np = prefix[r + 1] - prefix[r];
                    const int ctx = np > 0 ? row_context(a, r) : 0;
                    const int last = ctx - (np - 1) * P;  // tokens of the final partition
                    const bool short_last = np > 0 && last < P;
                    full_r[j] = short_last ? np - 1 : np;
                    bins[r] = short_last ? int((int64_t(last) * kLptBins) / P) : -1;
                }
            }
            __syncthreads();  // every thread has read the partition prefix
            // the full counts into prefix (exclusive, by a block scan of the
            // per-thread tiles of contiguous rows)
            const int per2 = (nrows + kBlockThreads - 1) / kBlockThreads;
#pragma unroll
            for (int j = 0; j * 256 < kLptMaxRows; ++j) {
                const int r = int(threadIdx.x) + 256 * j;
                if (r < nrows) shortlist[r] = full_r[j];  // (shortlist as scratch for the counts)
            }
            __syncthreads();
            const int t0 = int(threadIdx.x) * per2;
            int tile = 0;
            for (int i = 0; i < per2; ++i)
                if (t0 + i < nrows) tile += shortlist[t0 + i];
            const int incl = wave_incl_scan(tile);
            if (lane == kWave - 1) wave_total[threadIdx.x / kWave] = incl;
            __syncthreads();
            int before = 0;
            for (int w = 0; w < int(threadIdx.x) / kWave; ++w) before += wave_total[w];
            int run = before + incl - tile;
            for (int i = 0; i < per2; ++i) {
                if (t0 + i < nrows) {
                    const int c = shortlist[t0 + i];
                    prefix[t0 + i] = run;
                    run += c;
                }
            }
            if (threadIdx.x == kBlockThreads - 1) prefix[nrows] = before + incl;
            __syncthreads();  // prefix complete; the counts in shortlist are no longer needed
            num_full = prefix[nrows];
            // short final partitions by class, longest class first: thread t takes
            // class kLptBins - 1 - t / 4 over the quarter t % 4 of the rows; the
            // (class, quarter) counts in thread order give each its offset
            const int cls = kLptBins - 1 - int(threadIdx.x) / 4;
            const int qlen = (nrows + 3) / 4;
            const int q0 = (int(threadIdx.x) & 3) * qlen;
            const int q1 = q0 + qlen < nrows ? q0 + qlen : nrows;
            int cnt = 0;
            for (int r = q0; r < q1; ++r) cnt += bins[r] == cls ? 1 : 0;
            const int ci2 = wave_incl_scan(cnt);
            __syncthreads();  // every wave has read wave_total above
            if (lane == kWave - 1) wave_total[threadIdx.x / kWave] = ci2;
            __syncthreads();
            int off = ci2 - cnt;
            for (int w = 0; w < int(threadIdx.x) / kWave; ++w) off += wave_total[w];
            for (int r = q0; r < q1; ++r)
                if (bins[r] == cls) shortlist[off++] = r;
            __syncthreads();
        }

    }
    // Item groups of 4 consecutive items go to a workgroup, one item per
    // wave.
    const int num_groups = stat ? int(gridDim.x) : (num_items + kWavesPerBlock - 1) / kWavesPerBlock;
    auto run_group = [&](const int g) __attribute__((always_inline)) {
        const int it = g * kWavesPerBlock + wave;
        if (it < num_items) {
            const int pair = it / items_per_pair;
            const int sub = it - pair * items_per_pair;
            if constexpr (stat) {
                const int row = pair / a.static_parts;
                item(P, row, pair - row * a.static_parts, sub);
            } else if (lpt && pair >= num_full) {
                // a short final partition: its index is the row's full count
                const int row = shortlist[pair - num_full];
                item(P, row, prefix[row + 1] - prefix[row], sub);
            } else {
                int lo = 0, hi = nrows - 1;  // row = last r with prefix[r] <= pair
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (prefix[mid] <= pair) lo = mid;
                    else hi = mid - 1;
                }
                item(P, lo, pair - prefix[lo], sub);
            }
        }
    };
    if constexpr (DEAL) {
        // Dealt in a snake over the grid (every workgroup is resident: the
        // grid holds one per resident slot): round r gives group r W + b to
        // workgroup b when r is even and to W - 1 - b when r is odd, so in the
        // longest-first order the later (shorter) groups go first to the
        // workgroups whose earlier groups were the longest.  Nothing is
        // claimed: a wave starts its next item as soon as it has finished its
        // own, without waiting for its workgroup's other waves or for a
        // counter.  (The matrix-core kernels: their items' times follow their
        // lengths.)
        const int W = int(gridDim.x);
        for (int r = 0;; ++r) {
            const int g = r * W + ((r & 1) ? W - 1 - int(blockIdx.x) : int(blockIdx.x));
            if (g >= num_groups) break;  // (later rounds are further on)
            run_group(g);
        }
        return;
    }
    // Claimed (the VALU kernels, whose items' times vary with what shares
    // their CU).  Round 0 is static: workgroup b takes group b.  Later groups
    // g >= gridDim.x are dealt in 8 interleaved sequences g = gridDim.x + 8k +
    // q, each with its own counter (separate cache lines, so claims on
    // different sequences do not queue on one address).  A workgroup claims
    // from sequence blockIdx.x % 8 first and moves on to the next sequence when
    // one is exhausted, so every group is processed exactly once wherever the
    // workgroups run.  The merge kernel returns the counters to zero.
    __shared__ int next_group;
    const int g0 = int(gridDim.x);
    int g = blockIdx.x;
    int q = blockIdx.x % kClaimSequences;
    int tried = 0;
    while (g < num_groups) {
        run_group(g);
        if (g0 >= num_groups) break;  // the grid covers every group: nothing to claim
        __syncthreads();
        if (threadIdx.x == 0) {
            int next = num_groups;
            while (tried < kClaimSequences) {
                const int k = atomicAdd(a.counters + q * kCounterStride, 1);
                const int cand = g0 + kClaimSequences * k + q;
                if (cand < num_groups) {
                    next = cand;
                    break;
                }
                q = (q + 1) % kClaimSequences;  // this sequence is exhausted
                ++tried;
            }
            next_group = next;
        }
        __syncthreads();
        g = next_group;
    }
}

// Building with -DVKV_DECODE_BLOCKS_PER_CU=<n> fixes the grid's workgroups per
// CU (a tuning switch; default: as many as are resident at once).
#ifndef VKV_DECODE_BLOCKS_PER_CU
#define VKV_DECODE_BLOCKS_PER_CU 0
#endif
inline int blocks_per_cu(int fits) {
    return VKV_DECODE_BLOCKS_PER_CU > 0 ? VKV_DECODE_BLOCKS_PER_CU : fits;
}

inline int device_cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}


}  // namespace dec
}  // namespace vkv
