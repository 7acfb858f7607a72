/*
 * kv_oracle.h — CPU restatement of the reference's paged KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY.  This code is the checker for the HIP path: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it, and never as the thing measured or shipped.  The product library
 * (vllm-cpp_amd/) does not link or call it.
 *
 * Each function cites the reference file:line whose behaviour it restates.
 * Pinning (what checks each function against something other than itself)
 * is listed per function; tests/test_oracle.py holds those checks.
 */
#ifndef VKV_ORACLE_H
#define VKV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes, equal to the product ABI's VKV_DTYPE_* */
enum { OR_F32 = 0, OR_F16 = 1, OR_FP8 = 2 };

/* IEEE binary16 <-> binary32 (round to nearest even).
 * Pinned: exhaustive comparison with numpy.float16 over all 65536 patterns. */
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);

/* OCP e4m3fn decode straight from the format definition (bias 7, 0x7F/0xFF NaN).
 * Pinned: all 256 codes against torch.float8_e4m3fn. */
float oracle_fp8_decode(uint8_t code);

/* e4m3fn encode by brute force: the nearest of the 127 finite magnitudes,
 * ties to the even code, |x| >= 448 saturates to 448, NaN -> 0x7F|sign.
 * Pinned: every fp16 input and a dense fp32 sweep against torch.float8_e4m3fn
 * (which rounds to nearest even) inside the finite range. */
uint8_t oracle_fp8_encode(float x);

/* Per-(token, kv head) FP8 scale: amax/448 in fp32, 1.0 for amax == 0.
 * No reference counterpart (FP8 KV is absent from the reference); the rule is
 * the one the product documents.  Pinned: closed forms in tests. */
float oracle_fp8_scale(float amax);

/* KV append.  Restates src/layers/attention.cpp:84-102 (slot = block_table[pos/bs]*bs
 * + pos%bs, K/V rows copied whole into [blk][slot][Hkv][D]) with the slot given
 * per token; slots < 0 or >= num_blocks*bs are skipped.  FP8 quantises as in
 * oracle_fp8_scale / oracle_fp8_encode.  Pinned: gather(append(x)) == x and a
 * numpy scatter in tests. */
void oracle_reshape_and_cache(const void* key, const void* value, int64_t key_stride,
                              int64_t value_stride, void* key_cache, void* value_cache,
                              float* key_scales, float* value_scales,
                              const int32_t* slot_mapping, int32_t num_tokens,
                              int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                              int32_t num_blocks, int32_t src_dtype, int32_t cache_dtype);

/* The FP8 quantisation of oracle_reshape_and_cache on a dense array of rows:
 * row r of head_dim source elements (src_dtype) -> codes[r * head_dim ..] and
 * scales[r], by the same per-row code (amax / 448 scale, nearest e4m3 code of
 * x / scale), on nthreads threads (rows are independent).  Pinned by
 * tests/test_oracle.py against oracle_reshape_and_cache and torch's e4m3. */
void oracle_fp8_quantise_rows(const void* src, int64_t num_rows, int32_t head_dim, int32_t src_dtype,
                              uint8_t* codes, float* scales, int32_t nthreads);

/* RoPE in place.  Restates src/kernels/rotary_embedding.cu:13-34 (pairs d and
 * d + D/2, interleaved [pos][D/2][cos, sin] table rows of head_dim floats,
 * q heads h < num_heads, k heads h < num_kv_heads) with pos = positions[t]
 * (NULL: start_pos + t, the reference's form) clamped to [0, max_position).
 * Each output is fmaf(x0, c, -(x1*s)) / fmaf(x0, s, x1*c) in fp32, rounded to
 * src_dtype (F32/F16).  Pinned: numpy fp64 rotation of the same inputs,
 * position 0 = identity, pair norms preserved, in tests. */
void oracle_rope(void* query, void* key, int64_t query_stride, int64_t key_stride,
                 const float* cos_sin, const int32_t* positions, int32_t start_pos,
                 int32_t max_position, int32_t num_tokens, int32_t num_heads,
                 int32_t num_kv_heads, int32_t head_dim, int32_t src_dtype);

/* Paged decode.  Restates src/attention/paged_attention.cu:13-82: GQA map
 * h/(H/Hkv), ctx = min(context_lens[s], max_context_len), 32-lane strided
 * partial dots (fused multiply-add) reduced by the shfl_down 16..1 tree,
 * m0 = -1e30, online max/sum with expf, second pass weight =
 * expf(dot*scale - m)/(l + 1e-10) and out += weight * V (fused multiply-add) in
 * token order.  out is accumulated into, as in the reference.  K/V of dtype
 * F16/FP8 are widened to fp32 first (FP8: decode(code) * scale in fp32).
 * query is fp32 [num_seqs][num_heads][head_dim].  nthreads > 1 splits the
 * (seq, head) pairs over that many POSIX threads.
 * Pinned: fp64 textbook softmax(qK^T s)V in numpy, closed forms (ctx 1 -> V0,
 * equal keys -> mean V, dominant logit -> that V, ctx 0 -> untouched output). */
void oracle_paged_decode(float* out, const float* query, const void* key_cache,
                         const void* value_cache, const float* key_scales,
                         const float* value_scales, const int32_t* block_tables,
                         const int32_t* context_lens, int32_t num_seqs, int32_t num_heads,
                         int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                         int32_t max_context_len, int32_t max_blocks_per_seq, float scale,
                         int32_t kv_dtype, int32_t nthreads);

/* Causal chunked prefill.  The reference prefills one token per forward
 * (src/core/engine.cpp:157-164), so row j of sequence s (q_len = qsl[s+1]-qsl[s])
 * is oracle_paged_decode of that row with context context_lens[s]-q_len+j+1.
 * out is overwritten (zeroed, then accumulated as the reference's caller does,
 * src/layers/attention.cpp:128).  Pinned: equals per-position decode by
 * construction of the definition; tests add the fp64 masked-softmax check. */
void oracle_paged_prefill(float* out, const float* query, const void* key_cache,
                          const void* value_cache, const float* key_scales,
                          const float* value_scales, const int32_t* block_tables,
                          const int32_t* context_lens, const int32_t* query_start_loc,
                          int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                          int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq,
                          float scale, int32_t kv_dtype, int32_t nthreads);

/* Block copy: memcpy of each plane/layer block, pairs applied in order (no
 * reference counterpart; the contract is distinct destinations that are not
 * sources).  Pinned: numpy fancy-index copy in tests. */
typedef struct oracle_plane {
    void* base;
    int64_t layer_stride_bytes;
    int64_t block_bytes;
} oracle_plane;

void oracle_copy_blocks(const oracle_plane* planes, int32_t num_planes, int32_t num_layers,
                        int32_t num_blocks, const int32_t* block_pairs, int32_t num_pairs);

/* Swap between device-layout planes and a block-major host buffer
 * ([host block][plane][layer][block bytes]); direction 0 = out, 1 = in.
 * Pinned: out-then-in round trip is the identity; numpy copy in tests. */
void oracle_swap_blocks(const oracle_plane* planes, int32_t num_planes, int32_t num_layers,
                        int32_t num_dev_blocks, void* host_base, int32_t num_host_blocks,
                        const int32_t* block_pairs, int32_t num_pairs, int32_t direction);

#ifdef __cplusplus
}
#endif

#endif
