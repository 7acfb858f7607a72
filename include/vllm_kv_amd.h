/*
 * vllm_kv_amd.h — C ABI of the MI355X (gfx950) paged KV-cache hot path.
 *
 * Every entry point takes plain pointers, sizes and a HIP stream, launches
 * hand-written HIP kernels on that stream and returns immediately (no host
 * synchronisation, no hidden allocation except where stated).  All device
 * pointers are owned by the caller.
 *
 * Status codes: 0 = success; > 0 = a hipError_t from the runtime;
 * < 0 = an argument error detected on the host before any launch
 * (see VKV_ERR_*).  vkv_last_error() returns a message for the last failing
 * call made on the calling thread.
 *
 * KV cache layout (the reference's, src/memory/kv_cache.cpp:27-51):
 *   key_cache / value_cache of one layer: [num_blocks][block_size][num_kv_heads][head_dim]
 *   slot id s = physical_block * block_size + offset_in_block; the K/V vector of
 *   (slot s, kv head h) starts at element (s * num_kv_heads + h) * head_dim.
 * FP8 caches add one fp32 scale per (slot, kv head):
 *   key_scales / value_scales of one layer: [num_blocks][block_size][num_kv_heads]
 */
#ifndef VLLM_KV_AMD_H
#define VLLM_KV_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same type as hipStream_t (struct ihipStream_t*); NULL is the null stream. */
typedef struct ihipStream_t* vkv_stream_t;

/* Element types. */
enum {
    VKV_DTYPE_F32 = 0,      /* IEEE binary32 */
    VKV_DTYPE_F16 = 1,      /* IEEE binary16 */
    VKV_DTYPE_FP8_E4M3 = 2  /* OCP 8-bit e4m3fn (bias 7, max 448, no inf); cache only */
};

/* Host-side argument errors (negative so they never collide with hipError_t). */
enum {
    VKV_OK = 0,
    VKV_ERR_NULL = -1,        /* a required pointer is NULL */
    VKV_ERR_SHAPE = -2,       /* a size is out of range or inconsistent */
    VKV_ERR_UNSUPPORTED = -3, /* dtype / head_dim / group size combination not built */
    VKV_ERR_WORKSPACE = -4,   /* caller workspace too small */
    VKV_ERR_ALIGN = -5,       /* pointer or stride not aligned as required */
    VKV_ERR_DEVICE = -6       /* no usable gfx950 device / kernel image */
};

/* Message describing the last failing call on this thread ("" if none). */
const char* vkv_last_error(void);

/* ABI version: bumped whenever a struct below changes layout. */
int vkv_abi_version(void);

/* -------------------------------------------------------------------------
 * KV append (reshape_and_cache).
 *
 * Replaces the per-token pair of cudaMemcpyAsync calls of the reference's
 * AttentionLayer::forward (src/layers/attention.cpp:84-102) with one launch:
 * token t's K and V rows (num_kv_heads * head_dim elements) are written to
 * slot slot_mapping[t]; slot_mapping[t] < 0 skips the token (padding) and so
 * does a slot >= num_blocks * block_size.  The reference computes the slot as
 * block_table[pos / block_size] * block_size + pos % block_size;
 * vkv_slot_mapping_host() builds exactly that on the host.
 *
 * Any head_dim and token stride; pointers aligned to their element size
 * (16-byte rows take the vector kernels, other rows an element kernel with
 * the same results).
 *
 * cache_dtype F32 requires src F32 (bit copy); F16 takes F16 (bit copy) or
 * F32 (round to nearest even); FP8_E4M3 takes F16 or F32 and quantises per
 * (token, kv head): amax = max|x| over head_dim, scale = amax / 448 (IEEE
 * fp32 division, 1.0 when amax == 0), q = e4m3fn_rne_saturate(x / scale),
 * scale stored to key_scales/value_scales[slot][kv_head].
 * ------------------------------------------------------------------------- */
typedef struct vkv_append_params {
    const void* key;            /* [num_tokens, num_kv_heads, head_dim] (token stride key_stride) */
    const void* value;          /* [num_tokens, num_kv_heads, head_dim] (token stride value_stride) */
    int64_t key_stride;         /* elements between consecutive tokens; 0 = num_kv_heads*head_dim */
    int64_t value_stride;
    void* key_cache;            /* [num_blocks, block_size, num_kv_heads, head_dim] */
    void* value_cache;
    float* key_scales;          /* FP8 only: [num_blocks, block_size, num_kv_heads] */
    float* value_scales;
    const int32_t* slot_mapping;/* [num_tokens] device */
    int32_t num_tokens;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t block_size;
    int32_t num_blocks;
    int32_t src_dtype;          /* VKV_DTYPE_F32 / F16 */
    int32_t cache_dtype;        /* VKV_DTYPE_F32 / F16 / FP8_E4M3 */
} vkv_append_params;

int vkv_reshape_and_cache(const vkv_append_params* p, vkv_stream_t stream);

/* Host helper: slot_mapping[t] = block_table[(ctx+t)/bs]*bs + (ctx+t)%bs for
 * t < num_tokens (the reference's placement, src/layers/attention.cpp:85-94).
 * Returns VKV_ERR_SHAPE if a position falls outside block_table (where the
 * reference aborts, :87-90).  Pure host code, no device access. */
int vkv_slot_mapping_host(const int32_t* block_table, int32_t table_len, int32_t block_size,
                          int32_t context_len, int32_t num_tokens, int32_t* slot_mapping);

/* Host helpers for sizing the KV pool with its element type.  The reference
 * sizes the pool in src/model/qwen.cpp:72-73 and 94-104 with sizeof(float)
 * hard-coded: kv_bytes_per_block = 2 * block_size * num_kv_heads * head_dim *
 * 4 * num_layers, and num_blocks = min(max_num_seqs * ceil(max_model_len /
 * block_size), (budget - non_kv) / kv_bytes_per_block).
 * vkv_kv_block_bytes is that per-block figure for kv_dtype (FP8 adds its two
 * fp32 scales per slot and kv head); vkv_kv_pool_num_blocks is the block count
 * (0 when budget_bytes <= non_kv_bytes, as the reference then refuses to
 * start).  Negative VKV_ERR_SHAPE / VKV_ERR_UNSUPPORTED on bad arguments. */
int64_t vkv_kv_block_bytes(int32_t num_layers, int32_t block_size, int32_t num_kv_heads, int32_t head_dim,
                           int32_t kv_dtype);
int64_t vkv_kv_pool_num_blocks(uint64_t budget_bytes, uint64_t non_kv_bytes, int32_t num_layers, int32_t block_size,
                               int32_t num_kv_heads, int32_t head_dim, int32_t kv_dtype, int32_t max_num_seqs,
                               int32_t max_model_len);

/* -------------------------------------------------------------------------
 * Rotary position embedding fused with the KV append.
 *
 * Replaces the reference's rope_forward (src/kernels/rotary_embedding.cu:37-45,
 * declared in include/vllm/kernels/rotary_embedding.cuh:9-12) followed by the
 * append loop of AttentionLayer::forward (src/layers/attention.cpp:79-102).
 * For token t at position pos = positions[t] (positions == NULL: start_pos + t,
 * the reference's form) and every dim pair (d, d + head_dim/2), d < head_dim/2,
 * with c = cos_sin[pos][d][0], s = cos_sin[pos][d][1]:
 *   x[d] <- fma(x[d], c, -(x[d+D/2] * s));  x[d+D/2] <- fma(x[d], s, x[d+D/2] * c)
 * in fp32, rounded to src_dtype.  Every query head is rotated in place.
 *   key_cache != NULL (fused): the rotated key and the value rows are stored to
 *     slot slot_mapping[t] exactly as vkv_reshape_and_cache stores its source
 *     (same skip rule, dtype rules and FP8 quantisation); key is not written.
 *   key_cache == NULL (rope only): key heads are rotated in place as well;
 *     value, slot_mapping and the cache fields are ignored.
 * Positions are clamped to [0, max_position) (the reference reads out of its
 * table there).  cos_sin is [max_position][head_dim/2][2] fp32, the
 * reference's table layout (src/model/qwen.cpp:119-128);
 * vkv_rope_cos_sin_host() fills it as the reference does.  head_dim 64, 128
 * or 256; query/key/value/cos_sin 16-byte aligned with 16-byte token strides.
 * ------------------------------------------------------------------------- */
typedef struct vkv_rope_append_params {
    void* query;                /* [num_tokens, num_heads, head_dim] src_dtype, rotated in place */
    void* key;                  /* [num_tokens, num_kv_heads, head_dim] src_dtype */
    const void* value;          /* [num_tokens, num_kv_heads, head_dim] src_dtype (fused only) */
    int64_t query_stride;       /* elements between tokens; 0 = dense */
    int64_t key_stride;
    int64_t value_stride;
    const float* cos_sin;       /* [max_position, head_dim/2, 2] */
    const int32_t* positions;   /* [num_tokens] device, or NULL */
    int32_t start_pos;          /* used when positions == NULL */
    int32_t max_position;
    void* key_cache;            /* NULL: rope only */
    void* value_cache;
    float* key_scales;          /* FP8 only */
    float* value_scales;
    const int32_t* slot_mapping;/* [num_tokens] device (fused only) */
    int32_t num_tokens;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t block_size;
    int32_t num_blocks;
    int32_t src_dtype;          /* VKV_DTYPE_F32 / F16 (query, key, value) */
    int32_t cache_dtype;        /* as vkv_append_params.cache_dtype (fused only) */
} vkv_rope_append_params;

int vkv_rope_reshape_and_cache(const vkv_rope_append_params* p, vkv_stream_t stream);

/* Host helper: the reference's RoPE table (src/model/qwen.cpp:119-128):
 * cos_sin[pos][d] = {cosf(f), sinf(f)}, f = pos / powf(theta, 2.0f*d/head_dim),
 * all in fp32 with the C library's powf/cosf/sinf, for pos < max_position and
 * d < head_dim/2.  Pure host code. */
int vkv_rope_cos_sin_host(float theta, int32_t head_dim, int32_t max_position, float* cos_sin);

/* -------------------------------------------------------------------------
 * Paged decode attention.
 *
 * Replaces vllm::paged_attention_forward (src/attention/paged_attention.cu:85-93,
 * include/vllm/attention/paged_attention.hpp:9-28).  For sequence s and query
 * head h: kv head = h / (num_heads / num_kv_heads); ctx = min(context_lens[s],
 * max_context_len, max_blocks_per_seq * block_size); the result is
 * softmax(scale * q . K[0:ctx]^T) . V[0:ctx] with K/V gathered through
 * block_tables[s][t / block_size]; ctx == 0 yields zeros.  accumulate = 1
 * adds the result into output (the reference's `out +=`, its caller zeroes
 * output first, src/layers/attention.cpp:128); accumulate = 0 overwrites.
 *
 * io_dtype (query and output): F32 or F16.  kv_dtype: F32 (io F32 only),
 * F16 or FP8_E4M3 (needs key_scales / value_scales).  Any group size
 * num_heads / num_kv_heads, head_dim 1..1024 and block_size >= 1 (the
 * reference kernel's domain); pointers aligned to their element size.  head_dim
 * 64/128/256 with groups up to 8, power-of-two blocks and 16-byte-aligned
 * caches run on the tuned kernels, everything else on a generic one.
 *
 * Long contexts are split into partitions of partition_size tokens that are
 * reduced by a second kernel; that needs vkv_paged_decode_workspace_size()
 * bytes of device workspace.  With partition_size 0 the kernels choose the
 * size per call from the device-side context lengths (3/4 to 2 times the
 * default; the workspace size covers the smallest), so results may differ in
 * the last bits from an explicit size.
 *
 * Workspace.  A caller workspace must have its first 1024 bytes zeroed before
 * its first use (work counters; every call leaves them zero again, apart from
 * int 1, the partition size the call chose), and calls that may run
 * concurrently need distinct workspaces.  workspace == NULL uses a buffer the
 * library keeps per (device, stream): calls on different streams never share
 * it (hipStreamPerThread: per (device, thread)).  It grows with hipMalloc
 * when a call needs more (an outgrown buffer is kept, not freed, so graphs
 * captured before stay valid); a call that would grow it while its stream is
 * being captured fails with VKV_ERR_WORKSPACE instead, so capture after one
 * eager call of the largest size, or pass a workspace.  The buffers live
 * until vkv_release_workspace(stream), which a caller runs before it destroys
 * the stream.  Calls over many sequences are split into consecutive ranges of
 * rows inside the library (same results).
 * ------------------------------------------------------------------------- */
typedef struct vkv_decode_params {
    void* output;               /* [num_seqs, num_heads, head_dim] io_dtype */
    const void* query;          /* [num_seqs, num_heads, head_dim] io_dtype (seq stride query_stride) */
    const void* key_cache;      /* [num_blocks, block_size, num_kv_heads, head_dim] kv_dtype */
    const void* value_cache;
    const float* key_scales;    /* FP8 only: [num_blocks, block_size, num_kv_heads] */
    const float* value_scales;
    const int32_t* block_tables;/* [num_seqs, max_blocks_per_seq] */
    const int32_t* context_lens;/* [num_seqs] */
    int64_t query_stride;       /* elements between sequences in query; 0 = num_heads*head_dim */
    int32_t num_seqs;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t block_size;
    int32_t max_context_len;
    int32_t max_blocks_per_seq;
    int32_t num_blocks;         /* >0: block ids outside [0,num_blocks) read block 0 instead of faulting */
    float scale;
    int32_t io_dtype;
    int32_t kv_dtype;
    int32_t accumulate;
    int32_t partition_size;     /* tokens per split-K partition; 0 = the library picks it per call on the device */
    void* workspace;            /* optional, see above */
    size_t workspace_bytes;
} vkv_decode_params;

size_t vkv_paged_decode_workspace_size(const vkv_decode_params* p);
int vkv_paged_decode(const vkv_decode_params* p, vkv_stream_t stream);

/* One decode step of the attention layer: the append of each sequence's new
 * token, then the decode, as in the reference's AttentionLayer::forward (the
 * per-token slot copies, src/layers/attention.cpp:81-101, then
 * paged_attention_forward, :103-127).  Results, cache contents and errors are
 * those of vkv_reshape_and_cache(ap) followed by vkv_paged_decode(dp) on the
 * same stream (workspace as for vkv_paged_decode).  When the two fit together
 * — token s of ap is sequence s's new token (ap->num_tokens == dp->num_seqs),
 * both name the same fp16 or fp32 caches with the same geometry and pool,
 * source rows of the cache's type, 16-byte aligned with token strides a
 * multiple of 16 bytes, and a shape the tuned decode kernels run — the append
 * is fused into the decode
 * launches (one launch fewer per step): each sequence's last position is read
 * from its new rows when ap's slot for the token is that position's slot, and
 * the merge kernel stores the rows.  The fused form assumes what a decode step
 * guarantees: the slot of an appended token is read in this call only as its
 * own sequence's last position (a slot of no other sequence's context).
 * Otherwise the two calls run as they are. */
int vkv_paged_decode_append(const vkv_append_params* ap, const vkv_decode_params* dp, vkv_stream_t stream);

/* Frees the workspace buffers the library keeps for `stream` on the current
 * device (the ones decode and prefill calls with workspace == NULL use), after
 * synchronising the stream; for hipStreamPerThread, the calling thread's.  No
 * counterpart in the reference, whose kernels use no workspace.  Call it
 * before destroying a stream the library was called on with workspace ==
 * NULL: a stream created later at the same handle value would otherwise
 * inherit the buffers, and they would stay allocated until the process ends.
 * Graphs captured from such calls on that stream must not be replayed after
 * it.  VKV_OK (nothing to do) for a stream without buffers. */
int vkv_release_workspace(vkv_stream_t stream);

/* Paged decode that allocates nothing.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results as vkv_paged_decode, except that workspace /
 * workspace_bytes are ignored: the split-K partials live in a fixed 64 MiB
 * device array of the library.  The array is part of the library's code
 * object: every process that runs any of this library's kernels on a device
 * holds those 64 MiB of HBM on it, from the library's first use there until
 * the process ends, whether or not it ever calls this entry point.  A call whose
 * vkv_paged_decode_workspace_size() exceeds 64 MiB fails with
 * VKV_ERR_WORKSPACE before any launch.  All calls on one device share the
 * array: calls that overlap on one device (other streams, other threads) race
 * and give wrong results; serialise them.  Calls no hipMalloc or hipFree. */
int vkv_paged_decode_noalloc(const vkv_decode_params* p, vkv_stream_t stream);

/* -------------------------------------------------------------------------
 * Chunked-prefill (and mixed) paged attention, causal.
 *
 * The reference runs a prompt one token at a time through the decode path
 * (src/core/engine.cpp:157-164), so query token j of sequence s, at absolute
 * position pos = context_lens[s] - q_len_s + j, attends keys 0..pos of that
 * sequence.  This entry point does all of a step's query tokens at once;
 * the chunk's own K/V must already be in the cache (vkv_reshape_and_cache).
 * query_start_loc[s]..query_start_loc[s+1] are sequence s's rows of query.
 * Rows with q_len 1 are plain decode.  max_query_len must bound every q_len
 * (rows past it are not computed).  fp16 queries at head_dim 64/128 over fp16
 * or FP8 caches run sequences with q_len >= 2 on the matrix cores and the
 * q_len 1 ones through split-K decode; other combinations decode every row
 * with its causal context.  max_context_len > 0 clamps every row's key count
 * as decode does (the reference's max_context_len, paged_attention.cu:20);
 * 0 leaves only the table clamp.  multi_token_only = 1 is the caller's
 * promise that no sequence has exactly one query token (known on the host,
 * e.g. a step of prompt chunks only): the split-K decode pass that serves
 * such sequences (two kernels) is then not launched, and a sequence of one
 * query token would get no output row; 0 (the default) launches it, and it
 * finds the single-token sequences on the device.  Workspace: as for decode, a caller buffer of
 * vkv_paged_prefill_workspace_size() bytes (first 1024 bytes zeroed before
 * its first use) or, with workspace == NULL, the library's buffer of the
 * stream.
 * ------------------------------------------------------------------------- */
typedef struct vkv_prefill_params {
    void* output;               /* [num_query_tokens, num_heads, head_dim] io_dtype */
    const void* query;          /* [num_query_tokens, num_heads, head_dim] io_dtype */
    const void* key_cache;
    const void* value_cache;
    const float* key_scales;
    const float* value_scales;
    const int32_t* block_tables;    /* [num_seqs, max_blocks_per_seq] */
    const int32_t* context_lens;    /* [num_seqs] total keys incl. this step's tokens */
    const int32_t* query_start_loc; /* [num_seqs + 1] device */
    int64_t query_stride;       /* elements between query rows; 0 = num_heads*head_dim */
    int32_t num_seqs;
    int32_t num_query_tokens;
    int32_t max_query_len;      /* host bound on q_len over sequences */
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t block_size;
    int32_t max_blocks_per_seq;
    int32_t num_blocks;
    float scale;
    int32_t io_dtype;
    int32_t kv_dtype;
    int32_t max_context_len;    /* > 0: clamp of every row's keys; 0: none */
    int32_t multi_token_only;   /* 1: no sequence has q_len 1 (see above); 0: not known */
    void* workspace;            /* optional, see above */
    size_t workspace_bytes;
    const int32_t* work_list;   /* optional device copy of vkv_prefill_work_list_host()'s words for this call */
    int32_t work_list_words;    /* its length; 0 with work_list NULL: the kernels order the work themselves */
} vkv_prefill_params;

size_t vkv_paged_prefill_workspace_size(const vkv_prefill_params* p);
int vkv_paged_prefill(const vkv_prefill_params* p, vkv_stream_t stream);

/* Host-built work list of the matrix-core prefill kernels.  No counterpart in
 * the reference, whose prefill is one decode per token (src/core/engine.cpp:
 * 157-164).  From host copies of the call's query_start_loc and context_lens
 * and the shape fields of *p, it deals the call's work items (blocks of query
 * rows of one sequence and kv head, with their sequence's query rows and
 * context) to one list per workgroup of the kernels' persistent grid (one per
 * CU of the current device, 256 without one), longest first, each to the list
 * with the least work so far: a workgroup then runs its list without claiming
 * items and knows its next item while it computes the current one.  With the words
 * copied to device memory and passed as p->work_list / work_list_words, the
 * kernels skip ordering the items themselves: an engine builds it once per
 * step beside its other metadata, for every layer of the step.  The list must
 * come from the same lengths and shape as the call (items outside the call's
 * sequences, kv heads and query rows are skipped, so a stale list gives wrong
 * rows but reads nothing out of bounds; a grid smaller than the number of
 * lists runs the extra lists in turn).  Returns the number of int32 words; writes them when out is not
 * NULL and capacity_words suffices (else returns -2); 0 when the call's shape
 * runs without a list (everything but fp16 queries at head_dim 64/128 over fp16
 * caches or FP8 caches at 128); -1 for a NULL argument. */
int64_t vkv_prefill_work_list_host(const vkv_prefill_params* p, const int32_t* host_query_start_loc,
                                   const int32_t* host_context_lens, int32_t* out, int64_t capacity_words);

/* -------------------------------------------------------------------------
 * Block copy (copy-on-write on fork) and swap (HBM <-> pinned host).
 *
 * No counterpart exists in the reference; the nearest hooks are
 * BlockManager::inc_ref (src/core/block_manager.cpp:37-41) and the
 * "for preemption / swap" BlockTable::to_id_list declaration
 * (include/vllm/core/block_manager.hpp:39-40).  A plane is one per-layer
 * array indexed by block id: K, V and, for FP8, the two scale arrays.  Block b
 * of layer l of plane p starts at base + l*layer_stride_bytes + b*block_bytes.
 * ------------------------------------------------------------------------- */
typedef struct vkv_block_plane {
    void* base;
    int64_t layer_stride_bytes;
    int64_t block_bytes;
} vkv_block_plane;

/* For every (src, dst) pair in block_pairs ([num_pairs][2], device memory) and
 * every layer and plane: block dst <- block src.  Destinations must be
 * distinct and no destination may appear as a source (then every copy reads
 * the pre-call contents); both are the caller's contract, checkable on the
 * host with vkv_check_block_pairs_host().  Ids outside [0,num_blocks) are
 * skipped.  At most 4 planes. */
int vkv_copy_blocks(const vkv_block_plane* planes, int32_t num_planes, int32_t num_layers,
                    int32_t num_blocks, const int32_t* block_pairs, int32_t num_pairs,
                    vkv_stream_t stream);

int vkv_check_block_pairs_host(const int32_t* block_pairs, int32_t num_pairs, int32_t num_blocks);

/* Swap.  host_base is pinned host memory from hipHostMalloc (device-accessible);
 * host block h occupies host_block_bytes = sum over planes of
 * num_layers*block_bytes at host_base + h*host_block_bytes, ordered
 * [plane][layer][block bytes].  direction 0 (out): host block pair.dst <- device
 * block pair.src; direction 1 (in): device block pair.dst <- host block pair.src.
 * block_pairs is device memory.  Ids out of range are skipped. */
enum { VKV_SWAP_OUT = 0, VKV_SWAP_IN = 1 };

size_t vkv_swap_host_block_bytes(const vkv_block_plane* planes, int32_t num_planes, int32_t num_layers);

int vkv_swap_blocks(const vkv_block_plane* dev_planes, int32_t num_planes, int32_t num_layers,
                    int32_t num_dev_blocks, void* host_base, int32_t num_host_blocks,
                    const int32_t* block_pairs, int32_t num_pairs, int32_t direction,
                    vkv_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VLLM_KV_AMD_H */
