// ceilings.hip — measured hardware ceilings for the roofline fractions that
// bench.py reports (bench.py --suite ceil).  Measurement code only: the
// product library does not link it.
//
//   vkvc_mfma_loop    dense v_mfma_f32_16x16x32_f16 (the prefill kernels'
//                     instruction), 8 independent accumulator chains per wave,
//                     operands in registers: the matrix-core ceiling.
//   vkvc_read_stream  read-only sweep of a contiguous buffer (16-byte loads,
//                     8 in flight per lane), one 4-byte XOR per lane written
//                     at the end: the sequential HBM read ceiling.
//   vkvc_read_blocks  read-only gather of whole KV blocks (K and V pools of
//                     one layer) in the order of a block-id list: the decode's
//                     byte set without its math.
//   vkvc_read_heads   the decode's read pattern without its math: per (row,
//                     partition, kv head) wave, that head's slice of every
//                     token row of the partition, through the block table.
//   vkvc_copy         hipMemcpyAsync (pinned host <-> device in bench.py's
//                     host-link rows).
//
// Every entry point returns 0 or a hipError_t and launches on `stream`.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

// One MFMA with the accumulator in VGPRs, written as an instruction so that
// the compiler keeps the loop free of accumulator copies.
__device__ __forceinline__ void mfma(float4_t& c, half8_t a, half8_t b) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}

// 32 MFMAs per iteration over 8 accumulators: every MFMA's accumulator was
// last written 8 instructions earlier, so the chains never wait on each
// other and the matrix pipe issues back to back.
__global__ __launch_bounds__(kThreads) void mfma_loop_kernel(float* out, int iters) {
    const int lane = threadIdx.x & 63;
    half8_t a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = static_cast<_Float16>(0.001f * (lane + i));
        b[i] = static_cast<_Float16>(0.002f * (lane - i));
    }
    float4_t acc[8];
    for (int i = 0; i < 8; ++i) acc[i] = float4_t{0.f, 0.f, 0.f, 0.f};
    asm volatile("s_nop 4" ::: "memory");  // VALU writes of the operands -> first MFMA
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 32; ++j)
            mfma(acc[j & 7], a, b);
    }
    asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");  // MFMA results -> VALU reads
    float s = 0.f;
    for (int i = 0; i < 8; ++i) s += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
    out[blockIdx.x * kThreads + threadIdx.x] = s;
}

template <bool NT>
__device__ __forceinline__ uint4 load16(const uint4* p) {
    if constexpr (NT) {
        uint4 v;
        v.x = __builtin_nontemporal_load(&p->x);
        v.y = __builtin_nontemporal_load(&p->y);
        v.z = __builtin_nontemporal_load(&p->z);
        v.w = __builtin_nontemporal_load(&p->w);
        return v;
    } else {
        return *p;
    }
}

__device__ __forceinline__ uint32_t fold(uint4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

template <bool NT>
__global__ __launch_bounds__(kThreads) void read_stream_kernel(const uint4* __restrict__ src, int64_t n16,
                                                               uint32_t* __restrict__ out) {
    constexpr int kUnroll = 8;
    const int64_t stride = int64_t(gridDim.x) * kThreads;
    int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    uint32_t x = 0;
    for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
        uint4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) v[u] = load16<NT>(src + i + u * stride);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) x ^= fold(v[u]);
    }
    for (; i < n16; i += stride) x ^= fold(load16<NT>(src + i));
    out[int64_t(blockIdx.x) * kThreads + threadIdx.x] = x;
}

// One workgroup per listed block at a time (grid-stride over the list); a
// block of `block16` 16-byte words is read from both pools, 8 loads in
// flight per lane and pool.
template <bool NT>
__global__ __launch_bounds__(kThreads) void read_blocks_kernel(const uint4* __restrict__ k, const uint4* __restrict__ v,
                                                               const int32_t* __restrict__ ids, int n_ids,
                                                               int block16, uint32_t* __restrict__ out) {
    constexpr int kUnroll = 8;
    uint32_t x = 0;
    for (int w = blockIdx.x; w < n_ids; w += gridDim.x) {
        const int64_t base = int64_t(ids[w]) * block16;
        int i = threadIdx.x;
        for (; i + (kUnroll - 1) * kThreads < block16; i += kUnroll * kThreads) {
            uint4 a[kUnroll], b[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) a[u] = load16<NT>(k + base + i + u * kThreads);
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) b[u] = load16<NT>(v + base + i + u * kThreads);
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) x ^= fold(a[u]) ^ fold(b[u]);
        }
        for (; i < block16; i += kThreads) x ^= fold(load16<NT>(k + base + i)) ^ fold(load16<NT>(v + base + i));
    }
    out[int64_t(blockIdx.x) * kThreads + threadIdx.x] = x;
}

// The decode's own read pattern without its math: items (row, partition of P
// tokens, kv head), kv head fastest, one per wave (4 per workgroup), each
// reading its partition's K and V head slices (head_bytes of every token,
// through the block table) with 16-byte non-temporal loads.  As in the
// decode, the partition's block ids are loaded once, one per lane (P / bs <=
// 64), and each lane keeps U loads per pool in flight.
__global__ __launch_bounds__(kThreads) void read_heads_kernel(const char* __restrict__ k, const char* __restrict__ v,
                                                              const int32_t* __restrict__ bt,
                                                              const int32_t* __restrict__ cl, int S, int MB, int Hkv,
                                                              int bs, int row_bytes, int head_bytes, int P,
                                                              int max_parts, uint32_t* __restrict__ out) {
    constexpr int U = 8;
    const int lane = threadIdx.x & 63;
    const int64_t item = int64_t(blockIdx.x) * (kThreads / 64) + threadIdx.x / 64;
    uint32_t x = 0;
    if (item < int64_t(S) * max_parts * Hkv) {
        const int h = int(item % Hkv);
        const int part = int((item / Hkv) % max_parts);
        const int s = int(item / (int64_t(Hkv) * max_parts));
        const int ctx = cl[s];
        const int t0 = part * P;  // a multiple of bs
        const int n = ctx - t0 < P ? ctx - t0 : P;
        const int nb = n > 0 ? (n + bs - 1) / bs : 0;
        const int my_block = lane < nb ? bt[int64_t(s) * MB + t0 / bs + lane] : 0;
        const int lpt = head_bytes / 16;  // lanes per token
        const int tpl = 64 / lpt;         // tokens per wave-wide load
        const int sub = lane % lpt, grp = lane / lpt;
        for (int c = 0; c < n; c += U * tpl) {
            uint4 a[U], b[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int rel = c + u * tpl + grp;
                const int blk = __shfl(my_block, (rel / bs) & 63);
                a[u] = b[u] = uint4{0, 0, 0, 0};
                if (rel < n) {
                    const int64_t off = (int64_t(blk) * bs + rel % bs) * row_bytes + int64_t(h) * head_bytes + sub * 16;
                    a[u] = load16<true>(reinterpret_cast<const uint4*>(k + off));
                    b[u] = load16<true>(reinterpret_cast<const uint4*>(v + off));
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) x ^= fold(a[u]) ^ fold(b[u]);
        }
    }
    out[int64_t(blockIdx.x) * kThreads + threadIdx.x] = x;
}

}  // namespace

extern "C" {

// out: blocks * 256 floats.  FLOPs = blocks * 4 waves * iters * 32 * 16384.
int vkvc_mfma_loop(float* out, int blocks, int iters, hipStream_t stream) {
    if (!out || blocks <= 0 || iters <= 0) return int(hipErrorInvalidValue);
    mfma_loop_kernel<<<blocks, kThreads, 0, stream>>>(out, iters);
    return int(hipGetLastError());
}

// src: `bytes` (multiple of 16, 16-byte aligned); out: blocks * 256 words.
int vkvc_read_stream(const void* src, int64_t bytes, uint32_t* out, int blocks, int nontemporal,
                     hipStream_t stream) {
    if (!src || !out || blocks <= 0 || bytes <= 0 || (bytes & 15) || (reinterpret_cast<uintptr_t>(src) & 15))
        return int(hipErrorInvalidValue);
    const uint4* s = static_cast<const uint4*>(src);
    if (nontemporal)
        read_stream_kernel<true><<<blocks, kThreads, 0, stream>>>(s, bytes / 16, out);
    else
        read_stream_kernel<false><<<blocks, kThreads, 0, stream>>>(s, bytes / 16, out);
    return int(hipGetLastError());
}

// k, v: pools of blocks of `block_bytes` (multiple of 16); ids: n_ids block
// indices (each < the pools' block count, checked by the caller); out:
// blocks * 256 words.
int vkvc_read_blocks(const void* k, const void* v, const int32_t* ids, int n_ids, int64_t block_bytes,
                     uint32_t* out, int blocks, int nontemporal, hipStream_t stream) {
    if (!k || !v || !ids || !out || n_ids <= 0 || blocks <= 0 || block_bytes <= 0 || (block_bytes & 15) ||
        block_bytes / 16 > INT32_MAX)
        return int(hipErrorInvalidValue);
    const int b16 = static_cast<int>(block_bytes / 16);
    const uint4* kp = static_cast<const uint4*>(k);
    const uint4* vp = static_cast<const uint4*>(v);
    if (nontemporal)
        read_blocks_kernel<true><<<blocks, kThreads, 0, stream>>>(kp, vp, ids, n_ids, b16, out);
    else
        read_blocks_kernel<false><<<blocks, kThreads, 0, stream>>>(kp, vp, ids, n_ids, b16, out);
    return int(hipGetLastError());
}

// The decode pattern (read_heads_kernel): bt [S][MB] and cl [S] on the
// device, every table entry a valid block of the pools, cl <= MB * bs; P a
// multiple of bs with P / bs <= 64; head_bytes a multiple of 16 dividing
// 1 024; out: ceil(S * max_parts * Hkv / 4) * 256 words.
int vkvc_read_heads(const void* k, const void* v, const int32_t* bt, const int32_t* cl, int S, int MB, int Hkv,
                    int bs, int row_bytes, int head_bytes, int P, int max_parts, uint32_t* out, hipStream_t stream) {
    if (!k || !v || !bt || !cl || !out || S <= 0 || MB <= 0 || Hkv <= 0 || bs <= 0 || P <= 0 || max_parts <= 0 ||
        head_bytes < 16 || (head_bytes & 15) || 1024 % head_bytes || row_bytes < Hkv * head_bytes || P % bs ||
        P / bs > 64)
        return int(hipErrorInvalidValue);
    const int64_t items = int64_t(S) * max_parts * Hkv;
    const int64_t blocks = (items + 3) / 4;
    if (blocks > INT32_MAX) return int(hipErrorInvalidValue);
    read_heads_kernel<<<int(blocks), kThreads, 0, stream>>>(static_cast<const char*>(k), static_cast<const char*>(v),
                                                           bt, cl, S, MB, Hkv, bs, row_bytes, head_bytes, P,
                                                           max_parts, out);
    return int(hipGetLastError());
}

int vkvc_copy(void* dst, const void* src, int64_t bytes, hipStream_t stream) {
    if (!dst || !src || bytes <= 0) return int(hipErrorInvalidValue);
    return int(hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), hipMemcpyDefault, stream));
}

}  // extern "C"
