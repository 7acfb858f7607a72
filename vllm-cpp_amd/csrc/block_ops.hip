// block_ops.hip — copy_blocks (copy-on-write on fork) and swap_blocks
// (HBM <-> pinned host) for gfx950.
//
// Neither exists in the reference (its only hooks are BlockManager::inc_ref,
// src/core/block_manager.cpp:37-41, and the "for preemption / swap"
// BlockTable::to_id_list declaration, include/vllm/core/block_manager.hpp:39-40).
//
// Both are streaming copies: a work unit is one 16 KiB piece of one
// (pair, plane, layer) block; 256 lanes each move 4 x 16 bytes with
// non-temporal loads/stores (the data is not reused, so it should not
// displace anything in L2/MALL).  A grid-stride loop over units keeps the grid
// at a fixed size regardless of the pair count: copy fills the chip, swap
// takes a few workgroups.  Swap reads or writes host memory that hipHostMalloc
// mapped into the device address space, so the same loop drives the PCIe/host
// link directly from the CUs.
#include <cstdlib>

#include "common.hpp"
#include "launch.hpp"

namespace vkv {
namespace {

constexpr int kUnitBytes = 16384;          // bytes per work unit
constexpr int kThreads = 256;
constexpr int kVecPerThread = kUnitBytes / (16 * kThreads);  // 4

struct BlockCopyArgs {
    PlaneSet planes;
    const int32_t* pairs;
    char* host_base;
    int64_t host_block_bytes;
    int64_t host_plane_off[4];  // byte offset of plane p inside a host block
    int64_t units_per_block[4]; // per plane: ceil(block_bytes / kUnitBytes)
    int64_t units_per_pair;     // sum over planes of layers * units_per_block
    int64_t total_units;
    int32_t num_layers;
    int32_t num_dev_blocks;
    int32_t num_host_blocks;
    int32_t direction;          // swap only: 0 out (dev -> host), 1 in
};

// Copies bytes [off, off + kUnitBytes) clipped to len from src to dst.  When
// both pointers and len are 16-byte aligned (the normal case) every lane moves
// whole 16-byte vectors; otherwise it falls back to bytes.
__device__ __forceinline__ void copy_unit(char* dst, const char* src, int64_t off, int64_t len,
                                          bool aligned16) {
    const int64_t end = off + kUnitBytes < len ? off + kUnitBytes : len;
    if (aligned16) {
        u32x4 v[kVecPerThread];
#pragma unroll
        for (int i = 0; i < kVecPerThread; ++i) {
            const int64_t b = off + (int64_t(i) * kThreads + threadIdx.x) * 16;
            if (b < end) v[i] = load16_nt(src + b);
        }
#pragma unroll
        for (int i = 0; i < kVecPerThread; ++i) {
            const int64_t b = off + (int64_t(i) * kThreads + threadIdx.x) * 16;
            if (b < end) store16_nt(dst + b, v[i]);
        }
    } else {
        for (int64_t b = off + threadIdx.x; b < end; b += kThreads) dst[b] = src[b];
    }
}

// Decode a unit index into (pair, plane, layer, byte offset inside the block).
struct Unit {
    int64_t pair;
    int plane;
    int layer;
    int64_t off;
};

__device__ __forceinline__ Unit decode_unit(const BlockCopyArgs& a, int64_t u) {
    Unit r;
    r.pair = u / a.units_per_pair;
    int64_t rem = u - r.pair * a.units_per_pair;
    r.plane = 0;
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        const int64_t span = a.units_per_block[p] * a.num_layers;
        if (r.plane == p && p + 1 < a.planes.num_planes && rem >= span) {
            rem -= span;
            r.plane = p + 1;
        }
    }
    const int64_t upb = a.units_per_block[r.plane];
    r.layer = int(rem / upb);
    r.off = (rem - int64_t(r.layer) * upb) * kUnitBytes;
    return r;
}

__global__ __launch_bounds__(kThreads) void copy_blocks_kernel(BlockCopyArgs a) {
    for (int64_t u = blockIdx.x; u < a.total_units; u += gridDim.x) {
        const Unit w = decode_unit(a, u);
        const int32_t src = a.pairs[2 * w.pair];
        const int32_t dst = a.pairs[2 * w.pair + 1];
        if (unsigned(src) >= unsigned(a.num_dev_blocks) || unsigned(dst) >= unsigned(a.num_dev_blocks)) continue;
        const int64_t bb = a.planes.block_bytes[w.plane];
        char* layer = a.planes.base[w.plane] + int64_t(w.layer) * a.planes.layer_stride[w.plane];
        const bool aligned = ((reinterpret_cast<uintptr_t>(layer) | uintptr_t(bb)) & 15u) == 0;
        copy_unit(layer + int64_t(dst) * bb, layer + int64_t(src) * bb, w.off, bb, aligned);
    }
}

__global__ __launch_bounds__(kThreads) void swap_blocks_kernel(BlockCopyArgs a) {
    for (int64_t u = blockIdx.x; u < a.total_units; u += gridDim.x) {
        const Unit w = decode_unit(a, u);
        const int32_t src = a.pairs[2 * w.pair];
        const int32_t dst = a.pairs[2 * w.pair + 1];
        const int32_t dev = a.direction == 0 ? src : dst;
        const int32_t host = a.direction == 0 ? dst : src;
        if (unsigned(dev) >= unsigned(a.num_dev_blocks) || unsigned(host) >= unsigned(a.num_host_blocks)) continue;
        const int64_t bb = a.planes.block_bytes[w.plane];
        char* d = a.planes.base[w.plane] + int64_t(w.layer) * a.planes.layer_stride[w.plane] + int64_t(dev) * bb;
        char* h = a.host_base + int64_t(host) * a.host_block_bytes + a.host_plane_off[w.plane] + int64_t(w.layer) * bb;
        const bool aligned = ((reinterpret_cast<uintptr_t>(d) | reinterpret_cast<uintptr_t>(h) | uintptr_t(bb)) & 15u) == 0;
        if (a.direction == 0) copy_unit(h, d, w.off, bb, aligned);
        else copy_unit(d, h, w.off, bb, aligned);
    }
}

BlockCopyArgs make_args(const PlaneSet& planes, int32_t num_layers, const int32_t* pairs, int32_t num_pairs) {
    BlockCopyArgs a{};
    a.planes = planes;
    a.pairs = pairs;
    a.num_layers = num_layers;
    a.units_per_pair = 0;
    int64_t off = 0;
    for (int p = 0; p < 4; ++p) {
        if (p < planes.num_planes) {
            a.units_per_block[p] = (planes.block_bytes[p] + kUnitBytes - 1) / kUnitBytes;
            a.units_per_pair += a.units_per_block[p] * num_layers;
            a.host_plane_off[p] = off;
            off += planes.block_bytes[p] * num_layers;
        } else {
            a.units_per_block[p] = 1;
            a.host_plane_off[p] = off;
        }
    }
    a.total_units = a.units_per_pair * num_pairs;
    return a;
}

int grid_for_units(int64_t units, int64_t cap) {
    int64_t g = units < cap ? units : cap;
    return int(g < 1 ? 1 : g);
}

// Copy: HBM-bound, so the grid fills the chip (16 workgroups per CU on a
// 256-CU part).
constexpr int64_t kCopyWorkgroups = int64_t(256) * 16;

// Swap: bound by the host link (~55 GB/s), which a few workgroups keep busy;
// the rest of the chip stays free for the decode a side-stream swap runs
// beside.  Writes to host memory (out) reach 49 GB/s with 8 workgroups, with
// C2's decode beside them 6 % slower; reads of host memory (in) wait longer
// per request and need more in flight (8: 19 GB/s, 16: 38 GB/s, 24-32:
// 54-57 GB/s).  More workgroups than these slow a decode beside the swap far
// more than they speed the swap (16 writing workgroups: decode 1.6x slower).
// Building with -DVKV_SWAP_WORKGROUPS=<n> fixes both (a tuning switch).
#ifndef VKV_SWAP_WORKGROUPS
#define VKV_SWAP_WORKGROUPS 0
#endif
constexpr int64_t kSwapOutWorkgroups = 8;
constexpr int64_t kSwapInWorkgroups = 24;
int64_t swap_workgroups(int32_t direction) {
    if (VKV_SWAP_WORKGROUPS > 0) return VKV_SWAP_WORKGROUPS;
    return direction == 0 ? kSwapOutWorkgroups : kSwapInWorkgroups;
}

}  // namespace

int launch_copy_blocks(const PlaneSet& planes, int32_t num_layers, int32_t num_blocks, const int32_t* pairs,
                       int32_t num_pairs, hipStream_t st) {
    BlockCopyArgs a = make_args(planes, num_layers, pairs, num_pairs);
    a.num_dev_blocks = num_blocks;
    if (a.total_units == 0) return 0;
    hipLaunchKernelGGL(copy_blocks_kernel, dim3(grid_for_units(a.total_units, kCopyWorkgroups)), dim3(kThreads), 0,
                       st, a);
    return 0;
}

int launch_swap_blocks(const PlaneSet& planes, int32_t num_layers, int32_t num_dev_blocks, char* host_base,
                       int64_t host_block_bytes, int32_t num_host_blocks, const int32_t* pairs, int32_t num_pairs,
                       int32_t direction, hipStream_t st) {
    BlockCopyArgs a = make_args(planes, num_layers, pairs, num_pairs);
    a.host_base = host_base;
    a.host_block_bytes = host_block_bytes;
    a.num_dev_blocks = num_dev_blocks;
    a.num_host_blocks = num_host_blocks;
    a.direction = direction;
    if (a.total_units == 0) return 0;
    hipLaunchKernelGGL(swap_blocks_kernel, dim3(grid_for_units(a.total_units, swap_workgroups(direction))), dim3(kThreads), 0,
                       st, a);
    return 0;
}

}  // namespace vkv
