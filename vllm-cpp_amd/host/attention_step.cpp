// attention_step.cpp — AttentionMetadata and PagedAttentionLayer (the batched
// form of the reference's AttentionLayer::forward attention core,
// src/layers/attention.cpp:78-129).
#include "vllm/attention/attention_step.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "vllm/utils/hip_utils.hpp"
#include "vllm_kv_amd.h"

namespace vllm {

namespace {

[[noreturn]] void die(const char* msg, long long a, long long b) {
    std::fprintf(stderr, "AttentionMetadata: %s (%lld, %lld)\n", msg, a, b);
    std::abort();
}

}  // namespace

AttentionMetadata::AttentionMetadata(int32_t max_seqs, int32_t max_tokens, int32_t max_blocks_per_seq,
                                     int32_t block_size)
    : max_seqs_(max_seqs), max_tokens_(max_tokens), max_blocks_per_seq_(max_blocks_per_seq), block_size_(block_size) {
    if (max_seqs <= 0 || max_tokens <= 0 || max_blocks_per_seq <= 0 || block_size <= 0)
        die("capacities must be positive", max_seqs, max_tokens);
    // One int32 image: slots | positions | tables | context_lens | query_start_loc,
    // each section 16-byte aligned.
    auto round4 = [](size_t n) { return (n + 3) & ~size_t(3); };
    off_slots_ = 0;
    off_positions_ = off_slots_ + round4(size_t(max_tokens));
    off_tables_ = off_positions_ + round4(size_t(max_tokens));
    off_context_ = off_tables_ + round4(size_t(max_seqs) * size_t(max_blocks_per_seq));
    off_qsl_ = off_context_ + round4(size_t(max_seqs));
    words_ = off_qsl_ + round4(size_t(max_seqs) + 1);
    for (int i = 0; i < 2; ++i) {
        VLLM_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&host_[i]), words_ * sizeof(int32_t), hipHostMallocDefault));
        std::memset(host_[i], 0, words_ * sizeof(int32_t));
        VLLM_HIP_CHECK(hipEventCreateWithFlags(&uploaded_[i], hipEventDisableTiming));
    }
    VLLM_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&dev_), words_ * sizeof(int32_t)));
    VLLM_HIP_CHECK(hipMemset(dev_, 0, words_ * sizeof(int32_t)));
}

AttentionMetadata::~AttentionMetadata() {
    for (int i = 0; i < 2; ++i) {
        if (uploaded_[i]) {
            if (pending_[i]) (void)hipEventSynchronize(uploaded_[i]);
            (void)hipEventDestroy(uploaded_[i]);
        }
        if (host_[i]) (void)hipHostFree(host_[i]);
    }
    // Kernels queued before destruction may still read the device copy.
    if (dev_) {
        (void)hipDeviceSynchronize();
        (void)hipFree(dev_);
    }
}

void AttentionMetadata::build(const std::vector<StepSequence>& seqs, hipStream_t stream) {
    const int32_t S = int32_t(seqs.size());
    if (S > max_seqs_) die("more sequences than the capacity", S, max_seqs_);
    int32_t* h = host_[cur_];
    if (pending_[cur_]) {  // the upload of two builds ago may still be reading this buffer
        VLLM_HIP_CHECK(hipEventSynchronize(uploaded_[cur_]));
        pending_[cur_] = false;
    }
    int32_t* slots = h + off_slots_;
    int32_t* positions = h + off_positions_;
    int32_t* tables = h + off_tables_;
    int32_t* context = h + off_context_;
    int32_t* qsl = h + off_qsl_;
    int32_t t = 0, max_q = 0, singles = 0;
    qsl[0] = 0;
    for (int32_t s = 0; s < S; ++s) {
        const StepSequence& q = seqs[size_t(s)];
        if (q.num_new_tokens < 1 || q.context_len < 0) die("a sequence needs >= 1 new token", s, q.num_new_tokens);
        if (q.num_blocks > max_blocks_per_seq_) die("block table longer than max_blocks_per_seq", s, q.num_blocks);
        if (int64_t(t) + q.num_new_tokens > max_tokens_) die("more tokens than the capacity", t, q.num_new_tokens);
        for (int32_t j = 0; j < q.num_new_tokens; ++j, ++t) {
            const int64_t pos = int64_t(q.context_len) + j;
            const int64_t logical = pos / block_size_;
            if (logical >= q.num_blocks) die("KV block table missing position", s, pos);
            slots[t] = int32_t(int64_t(q.block_table[logical]) * block_size_ + pos % block_size_);
            positions[t] = int32_t(pos);
        }
        int32_t* row = tables + size_t(s) * size_t(max_blocks_per_seq_);
        std::copy(q.block_table, q.block_table + q.num_blocks, row);
        std::fill(row + q.num_blocks, row + max_blocks_per_seq_, 0);
        context[s] = q.context_len + q.num_new_tokens;
        qsl[s + 1] = t;
        max_q = std::max(max_q, q.num_new_tokens);
        singles += q.num_new_tokens == 1 ? 1 : 0;
    }
    // One copy of the whole image (unused tails included: one transfer beats several).
    VLLM_HIP_CHECK(hipMemcpyAsync(dev_, h, words_ * sizeof(int32_t), hipMemcpyHostToDevice, stream));
    VLLM_HIP_CHECK(hipEventRecord(uploaded_[cur_], stream));
    pending_[cur_] = true;
    cur_ ^= 1;
    num_seqs_ = S;
    num_tokens_ = t;
    max_query_len_ = max_q;
    single_token_seqs_ = singles;
}

PagedAttentionLayer::PagedAttentionLayer(int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                         int32_t max_seq_len)
    : num_heads_(num_heads), num_kv_heads_(num_kv_heads), head_dim_(head_dim), max_seq_len_(max_seq_len) {}

void PagedAttentionLayer::attach_rope_table(const float* cos_sin, int32_t max_position) {
    cos_sin_ = cos_sin;
    max_position_ = max_position;
}

void PagedAttentionLayer::forward(void* out, void* q, void* k, const void* v, KVDtype io_dtype, KVCache& cache,
                                  const AttentionMetadata& md, size_t layer, hipStream_t stream) const {
    const int32_t T = md.num_tokens();
    if (T == 0) return;
    if (int32_t(cache.num_kv_heads()) != num_kv_heads_ || int32_t(cache.head_dim()) != head_dim_ ||
        int32_t(cache.block_size()) != md.block_size()) {
        std::fprintf(stderr, "PagedAttentionLayer: cache geometry does not match the layer/metadata\n");
        std::abort();
    }
    const bool fp8 = cache.dtype() == KVDtype::kFP8E4M3;
    void* kc = cache.k_ptr(layer, 0);
    void* vc = cache.v_ptr(layer, 0);
    float* ks = fp8 ? cache.k_scale_ptr(layer, 0) : nullptr;
    float* vs = fp8 ? cache.v_scale_ptr(layer, 0) : nullptr;
    const auto st = reinterpret_cast<vkv_stream_t>(stream);

    // 1. RoPE + append (the reference's :79 and :84-102), one launch.
    if (cos_sin_) {
        vkv_rope_append_params p{};
        p.query = q;
        p.key = k;
        p.value = v;
        p.cos_sin = cos_sin_;
        p.positions = md.positions();
        p.max_position = max_position_;
        p.key_cache = kc;
        p.value_cache = vc;
        p.key_scales = ks;
        p.value_scales = vs;
        p.slot_mapping = md.slot_mapping();
        p.num_tokens = T;
        p.num_heads = num_heads_;
        p.num_kv_heads = num_kv_heads_;
        p.head_dim = head_dim_;
        p.block_size = int32_t(cache.block_size());
        p.num_blocks = int32_t(cache.num_blocks());
        p.src_dtype = int32_t(io_dtype);
        p.cache_dtype = int32_t(cache.dtype());
        VLLM_KV_CHECK(vkv_rope_reshape_and_cache(&p, st));
    } else {
        cache.append(layer, k, v, md.slot_mapping(), T, io_dtype, stream);
    }

    // 2. Attention over context + this step's tokens (:105-129), one call.
    const int32_t nb = int32_t(cache.num_blocks());
    const int32_t max_ctx = int32_t(std::min<int64_t>(max_seq_len_, int64_t(nb) * int64_t(cache.block_size())));
    const float scale = 1.0f / sqrtf(float(head_dim_));
    if (md.max_query_len() == 1) {
        vkv_decode_params d{};
        d.output = out;
        d.query = q;
        d.key_cache = kc;
        d.value_cache = vc;
        d.key_scales = ks;
        d.value_scales = vs;
        d.block_tables = md.block_tables();
        d.context_lens = md.context_lens();
        d.num_seqs = md.num_seqs();
        d.num_heads = num_heads_;
        d.num_kv_heads = num_kv_heads_;
        d.head_dim = head_dim_;
        d.block_size = int32_t(cache.block_size());
        d.max_context_len = max_ctx;
        d.max_blocks_per_seq = md.max_blocks_per_seq();
        d.num_blocks = nb;
        d.scale = scale;
        d.io_dtype = int32_t(io_dtype);
        d.kv_dtype = int32_t(cache.dtype());
        d.accumulate = 0;  // the reference zeroes, then adds (:128-129)
        VLLM_KV_CHECK(vkv_paged_decode(&d, st));
    } else {
        // Every row's keys are clamped as in decode (the reference's
        // max_context_len); a step without decode rows skips their pass.
        vkv_prefill_params p{};
        p.output = out;
        p.query = q;
        p.key_cache = kc;
        p.value_cache = vc;
        p.key_scales = ks;
        p.value_scales = vs;
        p.block_tables = md.block_tables();
        p.context_lens = md.context_lens();
        p.query_start_loc = md.query_start_loc();
        p.num_seqs = md.num_seqs();
        p.num_query_tokens = T;
        p.max_query_len = md.max_query_len();
        p.num_heads = num_heads_;
        p.num_kv_heads = num_kv_heads_;
        p.head_dim = head_dim_;
        p.block_size = int32_t(cache.block_size());
        p.max_blocks_per_seq = md.max_blocks_per_seq();
        p.num_blocks = nb;
        p.scale = scale;
        p.io_dtype = int32_t(io_dtype);
        p.kv_dtype = int32_t(cache.dtype());
        p.max_context_len = max_ctx;
        p.multi_token_only = md.single_token_seqs() == 0 ? 1 : 0;
        VLLM_KV_CHECK(vkv_paged_prefill(&p, st));
    }
}

}  // namespace vllm
