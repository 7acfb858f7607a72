// kv_cache.cpp — KVCache (reference: src/memory/kv_cache.cpp:8-62).
#include "vllm/memory/kv_cache.hpp"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#include "vllm/utils/hip_utils.hpp"

namespace vllm {

size_t kv_dtype_bytes(KVDtype dtype) {
    switch (dtype) {
        case KVDtype::kF32: return 4;
        case KVDtype::kF16: return 2;
        case KVDtype::kFP8E4M3: return 1;
    }
    return 4;
}

KVCache::KVCache(size_t num_layers, size_t num_blocks, size_t block_size, size_t num_kv_heads, size_t head_dim,
                 void* external_k, void* external_v, KVDtype dtype, float* external_k_scales,
                 float* external_v_scales)
    : num_layers_(num_layers),
      num_blocks_(num_blocks),
      block_size_(block_size),
      num_kv_heads_(num_kv_heads),
      head_dim_(head_dim),
      dtype_(dtype) {
    const size_t per_layer = layer_bytes();
    void* k_all = external_k;
    void* v_all = external_v;
    if (!k_all || !v_all) {
        const size_t total = per_layer * num_layers_;
        VLLM_HIP_CHECK(hipMalloc(&k_all, total ? total : 1));
        VLLM_HIP_CHECK(hipMalloc(&v_all, total ? total : 1));
        VLLM_HIP_CHECK(hipMemset(k_all, 0, total));
        VLLM_HIP_CHECK(hipMemset(v_all, 0, total));
        owns_kv_ = true;
    }
    k_buffers_.resize(num_layers_);
    v_buffers_.resize(num_layers_);
    for (size_t i = 0; i < num_layers_; ++i) {
        k_buffers_[i] = static_cast<uint8_t*>(k_all) + i * per_layer;
        v_buffers_[i] = static_cast<uint8_t*>(v_all) + i * per_layer;
    }
    if (dtype_ == KVDtype::kFP8E4M3) {
        const size_t scale_layer = scale_block_bytes() * num_blocks_;
        float* ks = external_k_scales;
        float* vs = external_v_scales;
        if (!ks || !vs) {
            const size_t total = scale_layer * num_layers_;
            VLLM_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&ks), total ? total : 1));
            VLLM_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&vs), total ? total : 1));
            VLLM_HIP_CHECK(hipMemset(ks, 0, total));
            VLLM_HIP_CHECK(hipMemset(vs, 0, total));
            owns_scales_ = true;
        }
        k_scale_buffers_.resize(num_layers_);
        v_scale_buffers_.resize(num_layers_);
        for (size_t i = 0; i < num_layers_; ++i) {
            k_scale_buffers_[i] = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(ks) + i * scale_layer);
            v_scale_buffers_[i] = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(vs) + i * scale_layer);
        }
    }
}

KVCache::~KVCache() {
    // Buffers passed in by the caller stay the caller's; only our own are freed.
    if (owns_kv_ && !k_buffers_.empty()) {
        (void)hipFree(k_buffers_[0]);
        (void)hipFree(v_buffers_[0]);
    }
    if (owns_scales_ && !k_scale_buffers_.empty()) {
        (void)hipFree(k_scale_buffers_[0]);
        (void)hipFree(v_scale_buffers_[0]);
    }
}

size_t KVCache::block_bytes() const { return block_size_ * num_kv_heads_ * head_dim_ * kv_dtype_bytes(dtype_); }

size_t KVCache::scale_block_bytes() const {
    return dtype_ == KVDtype::kFP8E4M3 ? block_size_ * num_kv_heads_ * sizeof(float) : 0;
}

void* KVCache::k_ptr(size_t layer, size_t physical_block) {
    return static_cast<uint8_t*>(k_buffers_[layer]) + physical_block * block_bytes();
}

void* KVCache::v_ptr(size_t layer, size_t physical_block) {
    return static_cast<uint8_t*>(v_buffers_[layer]) + physical_block * block_bytes();
}

float* KVCache::k_scale_ptr(size_t layer, size_t physical_block) {
    if (dtype_ != KVDtype::kFP8E4M3) return nullptr;
    return k_scale_buffers_[layer] + physical_block * block_size_ * num_kv_heads_;
}

float* KVCache::v_scale_ptr(size_t layer, size_t physical_block) {
    if (dtype_ != KVDtype::kFP8E4M3) return nullptr;
    return v_scale_buffers_[layer] + physical_block * block_size_ * num_kv_heads_;
}

void KVCache::clear_block(size_t layer, size_t physical_block) {
    VLLM_HIP_CHECK(hipMemset(k_ptr(layer, physical_block), 0, block_bytes()));
    VLLM_HIP_CHECK(hipMemset(v_ptr(layer, physical_block), 0, block_bytes()));
    if (dtype_ == KVDtype::kFP8E4M3) {
        VLLM_HIP_CHECK(hipMemset(k_scale_ptr(layer, physical_block), 0, scale_block_bytes()));
        VLLM_HIP_CHECK(hipMemset(v_scale_ptr(layer, physical_block), 0, scale_block_bytes()));
    }
}

size_t KVCache::total_bytes() const {
    return 2 * num_layers_ * num_blocks_ * (block_bytes() + scale_block_bytes());
}

void KVCache::append(size_t layer, const void* key, const void* value, const int32_t* slot_mapping,
                     int32_t num_tokens, KVDtype src_dtype, hipStream_t stream) {
    vkv_append_params p{};
    p.key = key;
    p.value = value;
    p.key_cache = k_buffers_[layer];
    p.value_cache = v_buffers_[layer];
    if (dtype_ == KVDtype::kFP8E4M3) {
        p.key_scales = k_scale_buffers_[layer];
        p.value_scales = v_scale_buffers_[layer];
    }
    p.slot_mapping = slot_mapping;
    p.num_tokens = num_tokens;
    p.num_kv_heads = int32_t(num_kv_heads_);
    p.head_dim = int32_t(head_dim_);
    p.block_size = int32_t(block_size_);
    p.num_blocks = int32_t(num_blocks_);
    p.src_dtype = int32_t(src_dtype);
    p.cache_dtype = int32_t(dtype_);
    VLLM_KV_CHECK(vkv_reshape_and_cache(&p, reinterpret_cast<vkv_stream_t>(stream)));
}

int32_t KVCache::planes(vkv_block_plane out[4]) {
    const int64_t stride = int64_t(layer_bytes());
    out[0] = {k_buffers_.empty() ? nullptr : k_buffers_[0], stride, int64_t(block_bytes())};
    out[1] = {v_buffers_.empty() ? nullptr : v_buffers_[0], stride, int64_t(block_bytes())};
    if (dtype_ != KVDtype::kFP8E4M3) return 2;
    const int64_t sstride = int64_t(scale_block_bytes() * num_blocks_);
    out[2] = {k_scale_buffers_[0], sstride, int64_t(scale_block_bytes())};
    out[3] = {v_scale_buffers_[0], sstride, int64_t(scale_block_bytes())};
    return 4;
}

void KVCache::copy_blocks(const int32_t* block_pairs, int32_t num_pairs, hipStream_t stream) {
    vkv_block_plane pl[4];
    const int32_t n = planes(pl);
    VLLM_KV_CHECK(vkv_copy_blocks(pl, n, int32_t(num_layers_), int32_t(num_blocks_), block_pairs, num_pairs,
                                  reinterpret_cast<vkv_stream_t>(stream)));
}

size_t KVCache::host_block_bytes() const { return 2 * num_layers_ * (block_bytes() + scale_block_bytes()); }

void KVCache::swap_blocks(void* host, int32_t num_host_blocks, const int32_t* block_pairs, int32_t num_pairs,
                          int32_t direction, hipStream_t stream) {
    vkv_block_plane pl[4];
    const int32_t n = planes(pl);
    VLLM_KV_CHECK(vkv_swap_blocks(pl, n, int32_t(num_layers_), int32_t(num_blocks_), host, num_host_blocks,
                                  block_pairs, num_pairs, direction, reinterpret_cast<vkv_stream_t>(stream)));
}

}  // namespace vllm
