// attention_step.hpp — the attention core of one scheduler step for every
// running sequence at once, over the C ABI of vllm_kv_amd.h.
//
// The reference runs AttentionLayer::forward (src/layers/attention.cpp:62-140)
// per sequence and per token: RoPE on q/k (:79), two cudaMemcpyAsync per token
// to place K and V (:84-102), two pageable H2D uploads of context_lens and the
// block table per layer (:105-110), a memset and one decode launch (:128-129).
// Here the step's metadata (slot mapping, positions, block tables, context
// lengths, query offsets) is packed on the host once per step and uploaded
// with one copy that every layer shares (AttentionMetadata); each layer then
// makes one fused RoPE + append launch and one attention call for all
// sequences (PagedAttentionLayer).  The q/k/v projections, the output
// projection and the residual add of the reference's layer are not part of the
// KV path and stay with the caller.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <vector>

#include "vllm/memory/kv_cache.hpp"

namespace vllm {

// One sequence's share of a step.  block_table holds the sequence's physical
// block ids (BlockManager), already grown to cover context_len + num_new_tokens
// positions (Scheduler: ensure_sequence_capacity, src/core/scheduler.cpp:99-100).
struct StepSequence {
    const int32_t* block_table;
    int32_t num_blocks;       // entries of block_table
    int32_t context_len;      // tokens already in the cache
    int32_t num_new_tokens;   // tokens of this step: 1 = decode, more = a prefill chunk
};

class AttentionMetadata {
  public:
    // Capacity of one step: sequences, tokens (sum of num_new_tokens) and
    // block-table row length.  Allocates two pinned host staging buffers and
    // one device buffer; nothing is allocated later.
    AttentionMetadata(int32_t max_seqs, int32_t max_tokens, int32_t max_blocks_per_seq, int32_t block_size);
    ~AttentionMetadata();
    AttentionMetadata(const AttentionMetadata&) = delete;
    AttentionMetadata& operator=(const AttentionMetadata&) = delete;

    // Packs the step on the host and uploads it with one hipMemcpyAsync on
    // `stream`; kernels that use the metadata must run on that stream (or after
    // it).  Token t of sequence s sits at position context_len + j and slot
    // block_table[pos / block_size] * block_size + pos % block_size (the
    // reference's placement, src/layers/attention.cpp:85-94).  Aborts, as the
    // reference does (:87-90), when a table does not cover a position, and on
    // a step larger than the capacity.  The staging buffer written here was
    // last read by the upload two builds earlier, which is waited for first.
    void build(const std::vector<StepSequence>& seqs, hipStream_t stream);

    int32_t num_seqs() const { return num_seqs_; }
    int32_t num_tokens() const { return num_tokens_; }
    int32_t max_query_len() const { return max_query_len_; }
    // sequences with exactly one new token (decode rows of a mixed step)
    int32_t single_token_seqs() const { return single_token_seqs_; }
    int32_t max_blocks_per_seq() const { return max_blocks_per_seq_; }
    int32_t block_size() const { return block_size_; }

    // Device arrays of the last build().
    const int32_t* slot_mapping() const { return dev_ + off_slots_; }        // [num_tokens]
    const int32_t* positions() const { return dev_ + off_positions_; }      // [num_tokens]
    const int32_t* block_tables() const { return dev_ + off_tables_; }      // [num_seqs][max_blocks_per_seq]
    const int32_t* context_lens() const { return dev_ + off_context_; }     // [num_seqs], this step's tokens included
    const int32_t* query_start_loc() const { return dev_ + off_qsl_; }      // [num_seqs + 1]

  private:
    int32_t max_seqs_, max_tokens_, max_blocks_per_seq_, block_size_;
    size_t off_slots_, off_positions_, off_tables_, off_context_, off_qsl_, words_;
    int32_t* host_[2] = {nullptr, nullptr};
    hipEvent_t uploaded_[2] = {nullptr, nullptr};
    bool pending_[2] = {false, false};
    int cur_ = 0;
    int32_t* dev_ = nullptr;
    int32_t num_seqs_ = 0, num_tokens_ = 0, max_query_len_ = 0, single_token_seqs_ = 0;
};

// Attention of one layer for a whole step.  q/out: [num_tokens][num_heads][head_dim],
// k/v: [num_tokens][num_kv_heads][head_dim], the tokens of the step in the order
// of AttentionMetadata::build's sequences, io_dtype F32 or F16 (F32 needs an
// F32 or F16 cache).
class PagedAttentionLayer {
  public:
    // max_seq_len bounds attended context as in the reference
    // (max_context_len = min(max_seq_len, num_blocks * block_size),
    // src/layers/attention.cpp:123-124); scale = 1/sqrtf(head_dim) (:126).
    PagedAttentionLayer(int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t max_seq_len);

    // cos_sin: device table [max_position][head_dim/2][2] fp32 (vkv_rope_cos_sin_host
    // builds the reference's); without a table forward() applies no rotation.
    void attach_rope_table(const float* cos_sin, int32_t max_position);

    // RoPE (q in place) fused with the K/V append of every token of the step
    // into layer `layer` of `cache` (one launch), then attention of every
    // sequence over its context including this step's tokens, written to out:
    // one split-K decode launch when every sequence has one new token,
    // otherwise the chunked-prefill path (causal within each chunk).
    // k is not modified; aborts on a HIP or argument error.
    void forward(void* out, void* q, void* k, const void* v, KVDtype io_dtype, KVCache& cache,
                 const AttentionMetadata& md, size_t layer, hipStream_t stream) const;

    int32_t num_heads() const { return num_heads_; }
    int32_t num_kv_heads() const { return num_kv_heads_; }
    int32_t head_dim() const { return head_dim_; }

  private:
    int32_t num_heads_, num_kv_heads_, head_dim_, max_seq_len_;
    const float* cos_sin_ = nullptr;
    int32_t max_position_ = 0;
};

}  // namespace vllm
