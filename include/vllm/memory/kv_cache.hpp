// kv_cache.hpp — KV storage geometry and ownership, API kept as in the
// reference (include/vllm/memory/kv_cache.hpp:11-48 of jiamumuzhao/vllm-cpp).
//
// Layout (unchanged): for each layer, K and V are separate arrays of
// [num_blocks][block_size][num_kv_heads][head_dim]; layer i of K starts
// i * layer_bytes after layer 0, likewise V.  The element type, which the
// reference fixes to float, is a trailing constructor argument defaulting to
// fp32, so existing callers compile and behave as before.  FP8 caches carry one
// fp32 scale per (slot, kv head) in two more per-layer arrays.
//
// Differences from the reference: a self-allocated cache is freed by the
// destructor (the reference leaks it), and the K/V operations of the paged
// path (append, block copy, swap) are available as methods.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "vllm_kv_amd.h"

namespace vllm {

enum class KVDtype : int32_t {
    kF32 = VKV_DTYPE_F32,
    kF16 = VKV_DTYPE_F16,
    kFP8E4M3 = VKV_DTYPE_FP8_E4M3,
};

size_t kv_dtype_bytes(KVDtype dtype);

class KVCache {
  public:
    // external_k / external_v: caller-owned device buffers of layer_bytes() *
    // num_layers each; when either is null the cache allocates (and zeroes) its
    // own.  FP8 scales likewise come from external_*_scales or are allocated.
    KVCache(size_t num_layers, size_t num_blocks, size_t block_size, size_t num_kv_heads, size_t head_dim,
            void* external_k = nullptr, void* external_v = nullptr, KVDtype dtype = KVDtype::kF32,
            float* external_k_scales = nullptr, float* external_v_scales = nullptr);
    ~KVCache();

    KVCache(const KVCache&) = delete;
    KVCache& operator=(const KVCache&) = delete;

    // Device address of block physical_block of a layer (K or V).
    void* k_ptr(size_t layer, size_t physical_block);
    void* v_ptr(size_t layer, size_t physical_block);
    // FP8 only: scales of the block's slots, [block_size][num_kv_heads] floats.
    float* k_scale_ptr(size_t layer, size_t physical_block);
    float* v_scale_ptr(size_t layer, size_t physical_block);

    // Zero one block of one layer (K, V and, for FP8, their scales); synchronous.
    void clear_block(size_t layer, size_t physical_block);

    size_t num_layers() const { return num_layers_; }
    size_t num_blocks() const { return num_blocks_; }
    size_t block_size() const { return block_size_; }
    size_t num_kv_heads() const { return num_kv_heads_; }
    size_t head_dim() const { return head_dim_; }
    KVDtype dtype() const { return dtype_; }

    // Total device bytes of K, V and scales over all layers.
    size_t total_bytes() const;

    size_t block_bytes() const;        // one block of one layer, K or V
    size_t scale_block_bytes() const;  // one block of one layer's scales (FP8), else 0
    size_t layer_bytes() const { return block_bytes() * num_blocks_; }

    // --- paged-path operations (stream-ordered, no synchronisation) ---

    // Write num_tokens K/V rows (src_dtype F32/F16, [tokens][num_kv_heads][head_dim])
    // of one layer into the slots of slot_mapping (device, -1 skips).
    void append(size_t layer, const void* key, const void* value, const int32_t* slot_mapping, int32_t num_tokens,
                KVDtype src_dtype, hipStream_t stream);

    // Copy-on-write: for each (src, dst) pair (device memory) and every layer,
    // block dst <- block src, K, V and scales.
    void copy_blocks(const int32_t* block_pairs, int32_t num_pairs, hipStream_t stream);

    // Bytes of one swapped block in host memory (all layers, K, V, scales).
    size_t host_block_bytes() const;
    // Swap between this cache and a hipHostMalloc buffer of num_host_blocks *
    // host_block_bytes(); direction VKV_SWAP_OUT or VKV_SWAP_IN.
    void swap_blocks(void* host, int32_t num_host_blocks, const int32_t* block_pairs, int32_t num_pairs,
                     int32_t direction, hipStream_t stream);

    // Plane descriptors (K, V[, K scales, V scales]) for the C ABI.
    int32_t planes(vkv_block_plane out[4]);

  private:
    size_t num_layers_;
    size_t num_blocks_;
    size_t block_size_;
    size_t num_kv_heads_;
    size_t head_dim_;
    KVDtype dtype_;
    bool owns_kv_ = false;
    bool owns_scales_ = false;

    // One device pointer per layer, as in the reference.
    std::vector<void*> k_buffers_;
    std::vector<void*> v_buffers_;
    std::vector<float*> k_scale_buffers_;
    std::vector<float*> v_scale_buffers_;
};

}  // namespace vllm
