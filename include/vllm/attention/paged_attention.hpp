// paged_attention.hpp — the reference's decode-attention entry point, kept
// field for field (include/vllm/attention/paged_attention.hpp:9-28 of
// jiamumuzhao/vllm-cpp) so callers recompile unchanged; cudaStream_t becomes
// hipStream_t.  The implementation calls vkv_paged_decode (vllm_kv_amd.h) with
// fp32 query/cache/output and the reference's `out +=` semantics.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace vllm {

// Field order, types and meaning are the reference's; all pointers are device memory.
struct PagedAttentionParams {
    float* output;                // per sequence: num_heads x head_dim results (added into)
    const float* query;           // per sequence: num_heads x head_dim
    const float* key_cache;       // one layer: blocks x block_size x num_kv_heads x head_dim
    const float* value_cache;     // same shape as key_cache
    const int32_t* block_tables;  // num_seqs rows of max_blocks_per_seq physical ids
    const int32_t* context_lens;  // keys per sequence
    int32_t num_seqs;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t block_size;
    int32_t max_context_len;      // upper clamp on context_lens
    int32_t max_blocks_per_seq;   // row length of block_tables
    float scale;                  // logit scale, normally 1/sqrt(head_dim)
    hipStream_t stream;
};

// PagedAttention forward pass: output += softmax(scale q.K^T).V per (seq, head).
// Aborts with a message on an unsupported shape or a HIP error.
void paged_attention_forward(const PagedAttentionParams& params);

}  // namespace vllm
