// launch.hpp — internal launchers behind the C ABI.  Arguments reaching these
// functions have been validated by capi.cpp; each returns 0 or a negative
// VKV_ERR_* for a combination that has no compiled kernel.
#pragma once

#include <hip/hip_runtime.h>

#include "vllm_kv_amd.h"

namespace vkv {

// Argument checks and error reporting of the C ABI (capi.cpp), for entry
// points defined in other files: the decode argument check, setting the
// thread's last-error message (returns code), and the status after a launch
// (a non-zero launcher result or a pending HIP error).
int check_decode_args(const vkv_decode_params* p);
int report_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int report_launch(int rc, const char* what);

int launch_append(const vkv_append_params* p, hipStream_t st);
int launch_rope_append(const vkv_rope_append_params* p, hipStream_t st);

// Split-K decode: partition kernel + reduce kernel.  part_o / part_ml point into
// a workspace of decode_workspace_bytes(); partition_size already normalised.
// When the caller leaves the partition size to the library, num_candidates > 1
// sizes (ascending, partition_size among them) go to the kernels, which pick
// one per call from the device-side context lengths; max_parts then covers the
// smallest.
constexpr int kMaxPartitionCandidates = 6;
struct DecodePlan {
    int partition_size;
    int max_parts;
    size_t workspace_bytes;
    int num_candidates;
    int candidates[kMaxPartitionCandidates];
};
DecodePlan plan_decode(const vkv_decode_params* p);
int launch_decode(const vkv_decode_params* p, const DecodePlan& plan, void* workspace, hipStream_t st);
// An append of one new token per sequence fused into the decode (fp16 source
// and cache, fixed shapes, the same pool and geometry on both sides): the
// partition kernel reads each row's last position from the new rows when the
// append targets that position's slot, and the merge kernel stores the rows.
bool decode_append_fusable(const vkv_append_params* ap, const vkv_decode_params* p);
int launch_decode_append(const vkv_append_params* ap, const vkv_decode_params* p, const DecodePlan& plan,
                         void* workspace, hipStream_t st);

// Causal chunked prefill.  fp16 queries with fp16 or FP8 keys at head_dim 64
// or 128: sequences with >= 2 query tokens on the matrix-core kernel
// (prefill.hip), single-token sequences through split-K decode.  Otherwise
// every query row goes through the decode kernels with its causal context
// (workspace: partials plus the row -> (sequence, context) map).
DecodePlan plan_prefill(const vkv_prefill_params* p);
int launch_prefill(const vkv_prefill_params* p, const DecodePlan& plan, void* workspace, hipStream_t st);
vkv_decode_params prefill_as_decode(const vkv_prefill_params* p, bool per_sequence);
bool prefill_mfma_supported(const vkv_prefill_params* p);
size_t prefill_items_bytes(const vkv_prefill_params* p);
// item_space: prefill_items_bytes(p) bytes of workspace for the list kernel's
// items and counters.
int launch_prefill_mfma(const vkv_prefill_params* p, void* item_space, hipStream_t st);
// vkv_prefill_work_list_host
int64_t prefill_work_list_host(const vkv_prefill_params* p, const int32_t* host_qsl, const int32_t* host_cl,
                               int32_t* out, int64_t capacity);
// Decode workspace header ints (the claim counters use 0, 32, 64, ...).
constexpr int kChosenPartitionSlot = 1;  // partition size the partition kernel chose

struct PlaneSet {
    char* base[4];
    int64_t layer_stride[4];
    int64_t block_bytes[4];
    int32_t num_planes;
};
int launch_copy_blocks(const PlaneSet& planes, int32_t num_layers, int32_t num_blocks,
                       const int32_t* pairs, int32_t num_pairs, hipStream_t st);
int launch_swap_blocks(const PlaneSet& planes, int32_t num_layers, int32_t num_dev_blocks,
                       char* host_base, int64_t host_block_bytes, int32_t num_host_blocks,
                       const int32_t* pairs, int32_t num_pairs, int32_t direction, hipStream_t st);

}  // namespace vkv
