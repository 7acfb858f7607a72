// paged_attention.cpp — vllm::paged_attention_forward over the C ABI
// (reference launcher: src/attention/paged_attention.cu:85-93).
#include "vllm/attention/paged_attention.hpp"

#include "vllm/utils/hip_utils.hpp"
#include "vllm_kv_amd.h"

namespace vllm {

void paged_attention_forward(const PagedAttentionParams& params) {
    vkv_decode_params p{};
    p.output = params.output;
    p.query = params.query;
    p.key_cache = params.key_cache;
    p.value_cache = params.value_cache;
    p.block_tables = params.block_tables;
    p.context_lens = params.context_lens;
    p.num_seqs = params.num_seqs;
    p.num_heads = params.num_heads;
    p.num_kv_heads = params.num_kv_heads;
    p.head_dim = params.head_dim;
    p.block_size = params.block_size;
    p.max_context_len = params.max_context_len;
    p.max_blocks_per_seq = params.max_blocks_per_seq;
    p.scale = params.scale;
    p.io_dtype = VKV_DTYPE_F32;
    p.kv_dtype = VKV_DTYPE_F32;
    p.accumulate = 1;  // the reference kernel adds into the caller-zeroed output
    VLLM_KV_CHECK(vkv_paged_decode(&p, reinterpret_cast<vkv_stream_t>(params.stream)));
}

}  // namespace vllm
