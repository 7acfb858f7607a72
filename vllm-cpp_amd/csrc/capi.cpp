// capi.cpp — the extern "C" boundary declared in include/vllm_kv_amd.h.
//
// Every entry point validates its arguments on the host (so that no kernel is
// launched with a shape it does not support), then calls the launcher.  No
// entry point synchronises the device.  The only allocation is the per-stream
// split-K workspace used when the caller passes none.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <thread>
#include <unordered_set>
#include <vector>

#include "launch.hpp"
#include "vllm_kv_amd.h"

namespace {

thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return VKV_OK;
    return fail(int(e), "%s: %s", what, hipGetErrorString(e));
}

// Launch errors (bad configuration, missing code object) surface here.
int after_launch(int rc, const char* what) {
    if (rc != 0) return fail(rc, "%s: no kernel compiled for this dtype/head_dim/group combination", what);
    return hip_status(hipGetLastError(), what);
}

bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

// Decode shape domain: any group size H / Hkv, head_dim and block_size up to
// these bounds (the reference kernel has none; these keep every per-lane
// register tile and partition size within the generic kernel's layout).
constexpr int kMaxHeadDim = 1024;
constexpr int kMaxBlockSize = 1 << 20;

// Library-owned workspaces, one per (device, stream): calls on different
// streams never share one, calls on one stream are ordered by it.  The
// per-thread stream handle (hipStreamPerThread) names a different stream in
// every thread, so its buffers are kept per (device, thread).  A buffer only
// grows.  An outgrown buffer is retired, not freed: queued work or a captured
// graph may still use it, and freeing would need a synchronisation.  Growth
// doubles, so the retired buffers of a stream never exceed its current one.
// A stream that is being captured cannot grow its buffer (that would allocate
// inside the capture): the call fails instead.  vkv_release_workspace frees a
// stream's buffers (the caller does so before destroying the stream, so that
// a new stream created at the same address starts with none).
struct StreamWorkspace {
    int device;
    hipStream_t stream;
    std::thread::id thread;  // hipStreamPerThread only; default otherwise
    void* ptr;
    size_t bytes;
    std::vector<void*> retired;
};
std::mutex g_ws_mutex;
std::vector<StreamWorkspace> g_ws;

std::thread::id stream_thread(hipStream_t stream) {
    return stream == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
}

int library_workspace(size_t need, hipStream_t stream, void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    const std::thread::id th = stream_thread(stream);
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    StreamWorkspace* w = nullptr;
    for (StreamWorkspace& x : g_ws)
        if (x.device == dev && x.stream == stream && x.thread == th) w = &x;
    if (!w) {
        g_ws.push_back(StreamWorkspace{dev, stream, th, nullptr, 0, {}});
        w = &g_ws.back();
    }
    if (w->bytes < need) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(stream, &cs);
        if (e != hipSuccess) return hip_status(e, "hipStreamIsCapturing");
        if (cs != hipStreamCaptureStatusNone)
            return fail(VKV_ERR_WORKSPACE,
                        "the library workspace of this stream must grow to %zu bytes, which cannot happen while "
                        "the stream is captured: make one eager call of this size first, or pass a workspace",
                        need);
        size_t sz = w->bytes * 2;
        if (sz < need) sz = need;
        if (sz < (size_t(1) << 20)) sz = size_t(1) << 20;
        void* p = nullptr;
        e = hipMalloc(&p, sz);
        if (e != hipSuccess) return hip_status(e, "hipMalloc (library workspace)");
        // The first 1 KiB holds the claim counters, which must start at zero;
        // the clear is ordered before the call's kernels on the same stream.
        e = hipMemsetAsync(p, 0, 1024, stream);
        if (e != hipSuccess) {
            (void)hipFree(p);
            return hip_status(e, "hipMemsetAsync (workspace header)");
        }
        if (w->ptr) w->retired.push_back(w->ptr);
        w->ptr = p;
        w->bytes = sz;
    }
    *out = w->ptr;
    return VKV_OK;
}

// A caller workspace: large enough, 16-byte aligned.
int check_workspace(void* ws, size_t have, size_t need) {
    if (have < need) return fail(VKV_ERR_WORKSPACE, "workspace %zu bytes < %zu needed", have, need);
    if (reinterpret_cast<uintptr_t>(ws) & 15u) return fail(VKV_ERR_ALIGN, "workspace must be 16-byte aligned");
    return VKV_OK;
}

int check_decode(const vkv_decode_params* p) {
    if (!p) return fail(VKV_ERR_NULL, "vkv_paged_decode: params is NULL");
    if (p->num_seqs < 0) return fail(VKV_ERR_SHAPE, "num_seqs < 0");
    if (p->num_seqs == 0) return VKV_OK;
    if (!p->output || !p->query || !p->key_cache || !p->value_cache || !p->block_tables || !p->context_lens)
        return fail(VKV_ERR_NULL, "vkv_paged_decode: a required pointer is NULL");
    if (p->num_heads <= 0 || p->num_kv_heads <= 0 || p->num_heads % p->num_kv_heads != 0)
        return fail(VKV_ERR_SHAPE, "num_heads (%d) must be a positive multiple of num_kv_heads (%d)", p->num_heads,
                    p->num_kv_heads);
    if (p->head_dim < 1 || p->head_dim > kMaxHeadDim)
        return fail(p->head_dim < 1 ? VKV_ERR_SHAPE : VKV_ERR_UNSUPPORTED, "head_dim %d outside 1..%d",
                    p->head_dim, kMaxHeadDim);
    if (p->block_size < 1 || p->block_size > kMaxBlockSize)
        return fail(VKV_ERR_SHAPE, "block_size %d outside 1..%d", p->block_size, kMaxBlockSize);
    if (p->max_blocks_per_seq <= 0) return fail(VKV_ERR_SHAPE, "max_blocks_per_seq must be > 0");
    if (p->num_blocks < 0) return fail(VKV_ERR_SHAPE, "num_blocks < 0");
    if (p->io_dtype != VKV_DTYPE_F32 && p->io_dtype != VKV_DTYPE_F16)
        return fail(VKV_ERR_UNSUPPORTED, "io_dtype %d unsupported", p->io_dtype);
    if (p->kv_dtype == VKV_DTYPE_F32 && p->io_dtype != VKV_DTYPE_F32)
        return fail(VKV_ERR_UNSUPPORTED, "fp32 KV requires fp32 query/output");
    if (p->kv_dtype != VKV_DTYPE_F32 && p->kv_dtype != VKV_DTYPE_F16 && p->kv_dtype != VKV_DTYPE_FP8_E4M3)
        return fail(VKV_ERR_UNSUPPORTED, "kv_dtype %d unsupported", p->kv_dtype);
    if (p->kv_dtype == VKV_DTYPE_FP8_E4M3 && (!p->key_scales || !p->value_scales))
        return fail(VKV_ERR_NULL, "FP8 KV needs key_scales and value_scales");
    if (p->query_stride < 0) return fail(VKV_ERR_SHAPE, "query_stride < 0");
    const int64_t qs = p->query_stride ? p->query_stride : int64_t(p->num_heads) * p->head_dim;
    if (qs < int64_t(p->num_heads) * p->head_dim)
        return fail(VKV_ERR_SHAPE, "query_stride smaller than num_heads*head_dim");
    const int io_eb = p->io_dtype == VKV_DTYPE_F32 ? 4 : 2;
    const int kv_eb = p->kv_dtype == VKV_DTYPE_F32 ? 4 : (p->kv_dtype == VKV_DTYPE_F16 ? 2 : 1);
    if ((reinterpret_cast<uintptr_t>(p->key_cache) | reinterpret_cast<uintptr_t>(p->value_cache)) &
        uintptr_t(kv_eb - 1))
        return fail(VKV_ERR_ALIGN, "key_cache/value_cache misaligned for their dtype");
    if ((reinterpret_cast<uintptr_t>(p->query) & uintptr_t(io_eb - 1)) ||
        (reinterpret_cast<uintptr_t>(p->output) & uintptr_t(io_eb - 1)))
        return fail(VKV_ERR_ALIGN, "query/output misaligned for their dtype");
    if (p->partition_size < 0) return fail(VKV_ERR_SHAPE, "partition_size < 0");
    return VKV_OK;
}

int check_prefill(const vkv_prefill_params* p) {
    if (!p) return fail(VKV_ERR_NULL, "vkv_paged_prefill: params is NULL");
    if (p->num_seqs < 0 || p->num_query_tokens < 0) return fail(VKV_ERR_SHAPE, "negative size");
    if (p->num_seqs == 0 || p->num_query_tokens == 0) return VKV_OK;
    if (!p->query_start_loc) return fail(VKV_ERR_NULL, "query_start_loc is NULL");
    if (p->max_query_len < 1) return fail(VKV_ERR_SHAPE, "max_query_len must be >= 1");
    if (p->max_context_len < 0) return fail(VKV_ERR_SHAPE, "max_context_len < 0");
    if (p->multi_token_only != 0 && p->multi_token_only != 1)
        return fail(VKV_ERR_SHAPE, "multi_token_only must be 0 or 1");
    if (p->work_list_words < 0 || (p->work_list_words > 0 && !p->work_list))
        return fail(VKV_ERR_SHAPE, "work_list_words must be >= 0, with a work_list when > 0");
    if (p->work_list && (reinterpret_cast<uintptr_t>(p->work_list) & 7u))
        return fail(VKV_ERR_ALIGN, "work_list must be 8-byte aligned");
    // Shape/dtype rules are those of decode; the decode rows are the
    // sequences (mixed matrix-core path) or the query tokens (row path).
    const vkv_decode_params d = vkv::prefill_as_decode(p, vkv::prefill_mfma_supported(p));
    return check_decode(&d);
}

int check_append(const vkv_append_params* p) {
    if (!p) return fail(VKV_ERR_NULL, "vkv_reshape_and_cache: params is NULL");
    if (p->num_tokens < 0) return fail(VKV_ERR_SHAPE, "num_tokens < 0");
    if (p->num_tokens == 0) return VKV_OK;
    if (!p->key || !p->value || !p->key_cache || !p->value_cache || !p->slot_mapping)
        return fail(VKV_ERR_NULL, "vkv_reshape_and_cache: a required pointer is NULL");
    if (p->num_kv_heads <= 0 || p->head_dim <= 0 || p->block_size <= 0 || p->num_blocks <= 0)
        return fail(VKV_ERR_SHAPE, "num_kv_heads, head_dim, block_size, num_blocks must be > 0");
    if (p->src_dtype != VKV_DTYPE_F32 && p->src_dtype != VKV_DTYPE_F16)
        return fail(VKV_ERR_UNSUPPORTED, "src_dtype %d unsupported", p->src_dtype);
    const int src_eb = p->src_dtype == VKV_DTYPE_F32 ? 4 : 2;
    const int64_t row = int64_t(p->num_kv_heads) * p->head_dim;
    if (p->key_stride < 0 || p->value_stride < 0) return fail(VKV_ERR_SHAPE, "negative stride");
    const int64_t ks = p->key_stride ? p->key_stride : row;
    const int64_t vs = p->value_stride ? p->value_stride : row;
    if (ks < row || vs < row) return fail(VKV_ERR_SHAPE, "token stride smaller than num_kv_heads*head_dim");
    const int dst_eb = p->cache_dtype == VKV_DTYPE_F32 ? 4 : (p->cache_dtype == VKV_DTYPE_F16 ? 2 : 1);
    if ((reinterpret_cast<uintptr_t>(p->key) | reinterpret_cast<uintptr_t>(p->value)) & uintptr_t(src_eb - 1))
        return fail(VKV_ERR_ALIGN, "key/value misaligned for their dtype");
    if ((reinterpret_cast<uintptr_t>(p->key_cache) | reinterpret_cast<uintptr_t>(p->value_cache)) &
        uintptr_t(dst_eb - 1))
        return fail(VKV_ERR_ALIGN, "caches misaligned for their dtype");
    switch (p->cache_dtype) {
        case VKV_DTYPE_F32:
            if (p->src_dtype != VKV_DTYPE_F32) return fail(VKV_ERR_UNSUPPORTED, "fp32 cache needs fp32 source");
            break;
        case VKV_DTYPE_F16:
            break;
        case VKV_DTYPE_FP8_E4M3:
            if (!p->key_scales || !p->value_scales) return fail(VKV_ERR_NULL, "FP8 cache needs scale arrays");
            break;
        default:
            return fail(VKV_ERR_UNSUPPORTED, "cache_dtype %d unsupported", p->cache_dtype);
    }
    return VKV_OK;
}

int check_rope(const vkv_rope_append_params* p) {
    if (!p) return fail(VKV_ERR_NULL, "vkv_rope_reshape_and_cache: params is NULL");
    if (p->num_tokens < 0) return fail(VKV_ERR_SHAPE, "num_tokens < 0");
    if (p->num_tokens == 0) return VKV_OK;
    const bool fused = p->key_cache != nullptr;
    if (!p->query || !p->key || !p->cos_sin || (fused && (!p->value || !p->value_cache || !p->slot_mapping)))
        return fail(VKV_ERR_NULL, "vkv_rope_reshape_and_cache: a required pointer is NULL");
    if (p->num_heads <= 0 || p->num_kv_heads <= 0 || p->max_position <= 0)
        return fail(VKV_ERR_SHAPE, "num_heads, num_kv_heads and max_position must be > 0");
    if (p->head_dim != 64 && p->head_dim != 128 && p->head_dim != 256)
        return fail(VKV_ERR_UNSUPPORTED, "head_dim %d not built (64, 128, 256)", p->head_dim);
    if (p->src_dtype != VKV_DTYPE_F32 && p->src_dtype != VKV_DTYPE_F16)
        return fail(VKV_ERR_UNSUPPORTED, "src_dtype %d unsupported", p->src_dtype);
    if (p->query_stride < 0 || p->key_stride < 0 || p->value_stride < 0) return fail(VKV_ERR_SHAPE, "negative stride");
    const int seb = p->src_dtype == VKV_DTYPE_F32 ? 4 : 2;
    const int64_t qrow = int64_t(p->num_heads) * p->head_dim, kvrow = int64_t(p->num_kv_heads) * p->head_dim;
    const int64_t qs = p->query_stride ? p->query_stride : qrow;
    const int64_t ks = p->key_stride ? p->key_stride : kvrow;
    const int64_t vs = p->value_stride ? p->value_stride : kvrow;
    if (qs < qrow || ks < kvrow || (fused && vs < kvrow))
        return fail(VKV_ERR_SHAPE, "token stride smaller than the token's heads * head_dim");
    uintptr_t bits = reinterpret_cast<uintptr_t>(p->query) | reinterpret_cast<uintptr_t>(p->key) |
                     reinterpret_cast<uintptr_t>(p->cos_sin) | uintptr_t(qs * seb) | uintptr_t(ks * seb);
    if (fused)
        bits |= reinterpret_cast<uintptr_t>(p->value) | uintptr_t(vs * seb) |
                reinterpret_cast<uintptr_t>(p->key_cache) | reinterpret_cast<uintptr_t>(p->value_cache);
    if (bits & 15u) return fail(VKV_ERR_ALIGN, "query/key/value/cos_sin/caches and token strides must be 16-byte aligned");
    if (!fused) return VKV_OK;
    if (p->block_size <= 0 || p->num_blocks <= 0) return fail(VKV_ERR_SHAPE, "block_size and num_blocks must be > 0");
    switch (p->cache_dtype) {
        case VKV_DTYPE_F32:
            if (p->src_dtype != VKV_DTYPE_F32) return fail(VKV_ERR_UNSUPPORTED, "fp32 cache needs fp32 source");
            break;
        case VKV_DTYPE_F16:
            break;
        case VKV_DTYPE_FP8_E4M3:
            if (!p->key_scales || !p->value_scales) return fail(VKV_ERR_NULL, "FP8 cache needs scale arrays");
            break;
        default:
            return fail(VKV_ERR_UNSUPPORTED, "cache_dtype %d unsupported", p->cache_dtype);
    }
    return VKV_OK;
}

int fill_planes(const vkv_block_plane* planes, int32_t num_planes, vkv::PlaneSet* out) {
    if (!planes) return fail(VKV_ERR_NULL, "planes is NULL");
    if (num_planes < 1 || num_planes > 4) return fail(VKV_ERR_SHAPE, "num_planes must be 1..4");
    std::memset(out, 0, sizeof(*out));
    out->num_planes = num_planes;
    for (int i = 0; i < num_planes; ++i) {
        if (!planes[i].base) return fail(VKV_ERR_NULL, "plane %d base is NULL", i);
        if (planes[i].block_bytes <= 0 || planes[i].layer_stride_bytes < 0)
            return fail(VKV_ERR_SHAPE, "plane %d has block_bytes <= 0 or negative layer stride", i);
        out->base[i] = static_cast<char*>(planes[i].base);
        out->layer_stride[i] = planes[i].layer_stride_bytes;
        out->block_bytes[i] = planes[i].block_bytes;
    }
    return VKV_OK;
}

}  // namespace

namespace vkv {

int check_decode_args(const vkv_decode_params* p) { return check_decode(p); }

int report_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int report_launch(int rc, const char* what) { return after_launch(rc, what); }

}  // namespace vkv

extern "C" {

const char* vkv_last_error(void) { return g_last_error; }

int vkv_abi_version(void) { return 4; }

int64_t vkv_prefill_work_list_host(const vkv_prefill_params* p, const int32_t* host_query_start_loc,
                                   const int32_t* host_context_lens, int32_t* out, int64_t capacity_words) {
    return vkv::prefill_work_list_host(p, host_query_start_loc, host_context_lens, out, capacity_words);
}

int vkv_release_workspace(vkv_stream_t stream_handle) {
    const hipStream_t stream = reinterpret_cast<hipStream_t>(stream_handle);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    const std::thread::id th = stream_thread(stream);
    std::vector<void*> bufs;
    {
        std::lock_guard<std::mutex> lock(g_ws_mutex);
        for (size_t i = 0; i < g_ws.size(); ++i) {
            StreamWorkspace& x = g_ws[i];
            if (x.device != dev || x.stream != stream || x.thread != th) continue;
            bufs = std::move(x.retired);
            if (x.ptr) bufs.push_back(x.ptr);
            g_ws.erase(g_ws.begin() + long(i));
            break;
        }
    }
    if (bufs.empty()) return VKV_OK;
    // the stream's queued calls may still use the buffers
    e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return hip_status(e, "hipStreamSynchronize (vkv_release_workspace)");
    for (void* b : bufs) {
        e = hipFree(b);
        if (e != hipSuccess) return hip_status(e, "hipFree (vkv_release_workspace)");
    }
    return VKV_OK;
}

int vkv_reshape_and_cache(const vkv_append_params* p, vkv_stream_t stream) {
    int rc = check_append(p);
    if (rc != VKV_OK || p->num_tokens == 0) return rc;
    return after_launch(vkv::launch_append(p, reinterpret_cast<hipStream_t>(stream)), "vkv_reshape_and_cache");
}

int64_t vkv_kv_block_bytes(int32_t num_layers, int32_t block_size, int32_t num_kv_heads, int32_t head_dim,
                           int32_t kv_dtype) {
    if (num_layers <= 0 || block_size <= 0 || num_kv_heads <= 0 || head_dim <= 0)
        return fail(VKV_ERR_SHAPE, "vkv_kv_block_bytes: sizes must be > 0");
    int64_t per_slot_head;  // bytes of one (slot, kv head) for K or V
    switch (kv_dtype) {
        case VKV_DTYPE_F32: per_slot_head = int64_t(head_dim) * 4; break;
        case VKV_DTYPE_F16: per_slot_head = int64_t(head_dim) * 2; break;
        case VKV_DTYPE_FP8_E4M3: per_slot_head = int64_t(head_dim) + 4; break;  // codes + scale
        default: return fail(VKV_ERR_UNSUPPORTED, "vkv_kv_block_bytes: kv_dtype %d", kv_dtype);
    }
    return 2 * int64_t(block_size) * num_kv_heads * per_slot_head * num_layers;
}

int64_t vkv_kv_pool_num_blocks(uint64_t budget_bytes, uint64_t non_kv_bytes, int32_t num_layers, int32_t block_size,
                               int32_t num_kv_heads, int32_t head_dim, int32_t kv_dtype, int32_t max_num_seqs,
                               int32_t max_model_len) {
    const int64_t per_block = vkv_kv_block_bytes(num_layers, block_size, num_kv_heads, head_dim, kv_dtype);
    if (per_block < 0) return per_block;
    if (max_num_seqs <= 0 || max_model_len <= 0)
        return fail(VKV_ERR_SHAPE, "vkv_kv_pool_num_blocks: max_num_seqs and max_model_len must be > 0");
    if (budget_bytes <= non_kv_bytes) return 0;
    const int64_t per_seq = (int64_t(max_model_len) + block_size - 1) / block_size;
    const int64_t by_seqs = per_seq * max_num_seqs;
    const int64_t by_memory = int64_t((budget_bytes - non_kv_bytes) / uint64_t(per_block));
    return by_seqs < by_memory ? by_seqs : by_memory;
}

int vkv_rope_reshape_and_cache(const vkv_rope_append_params* p, vkv_stream_t stream) {
    int rc = check_rope(p);
    if (rc != VKV_OK || p->num_tokens == 0) return rc;
    return after_launch(vkv::launch_rope_append(p, reinterpret_cast<hipStream_t>(stream)),
                        "vkv_rope_reshape_and_cache");
}

int vkv_rope_cos_sin_host(float theta, int32_t head_dim, int32_t max_position, float* cos_sin) {
    if (!cos_sin) return fail(VKV_ERR_NULL, "vkv_rope_cos_sin_host: cos_sin is NULL");
    if (head_dim <= 0 || head_dim % 2 || max_position < 0 || !(theta > 0.0f))
        return fail(VKV_ERR_SHAPE, "vkv_rope_cos_sin_host: bad theta/head_dim/max_position");
    const int half = head_dim / 2;
    for (int32_t pos = 0; pos < max_position; ++pos) {
        for (int d = 0; d < half; ++d) {
            const float f = float(pos) / powf(theta, 2.0f * float(d) / float(head_dim));
            cos_sin[int64_t(pos) * head_dim + 2 * d] = cosf(f);
            cos_sin[int64_t(pos) * head_dim + 2 * d + 1] = sinf(f);
        }
    }
    return VKV_OK;
}

int vkv_slot_mapping_host(const int32_t* block_table, int32_t table_len, int32_t block_size, int32_t context_len,
                          int32_t num_tokens, int32_t* slot_mapping) {
    if ((!block_table && table_len > 0) || (!slot_mapping && num_tokens > 0))
        return fail(VKV_ERR_NULL, "vkv_slot_mapping_host: NULL pointer");
    if (block_size <= 0 || table_len < 0 || context_len < 0 || num_tokens < 0)
        return fail(VKV_ERR_SHAPE, "vkv_slot_mapping_host: bad sizes");
    for (int32_t t = 0; t < num_tokens; ++t) {
        const int64_t pos = int64_t(context_len) + t;
        const int64_t logical = pos / block_size;
        if (logical >= table_len)
            return fail(VKV_ERR_SHAPE, "KV block table missing position %lld", static_cast<long long>(pos));
        slot_mapping[t] = int32_t(int64_t(block_table[logical]) * block_size + pos % block_size);
    }
    return VKV_OK;
}

size_t vkv_paged_decode_workspace_size(const vkv_decode_params* p) {
    if (check_decode(p) != VKV_OK || p->num_seqs == 0) return 0;
    return vkv::plan_decode(p).workspace_bytes;
}

int vkv_paged_decode(const vkv_decode_params* p, vkv_stream_t stream) {
    int rc = check_decode(p);
    if (rc != VKV_OK || p->num_seqs == 0) return rc;
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const vkv::DecodePlan plan = vkv::plan_decode(p);
    void* ws = p->workspace;
    rc = ws ? check_workspace(ws, p->workspace_bytes, plan.workspace_bytes)
            : library_workspace(plan.workspace_bytes, st, &ws);
    if (rc != VKV_OK) return rc;
    return after_launch(vkv::launch_decode(p, plan, ws, st), "vkv_paged_decode");
}

int vkv_paged_decode_append(const vkv_append_params* ap, const vkv_decode_params* dp, vkv_stream_t stream) {
    int rc = check_append(ap);
    if (rc != VKV_OK) return rc;
    rc = check_decode(dp);
    if (rc != VKV_OK) return rc;
    if (ap->num_tokens == 0 || dp->num_seqs == 0 || !vkv::decode_append_fusable(ap, dp)) {
        rc = vkv_reshape_and_cache(ap, stream);
        return rc != VKV_OK ? rc : vkv_paged_decode(dp, stream);
    }
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const vkv::DecodePlan plan = vkv::plan_decode(dp);
    void* ws = dp->workspace;
    rc = ws ? check_workspace(ws, dp->workspace_bytes, plan.workspace_bytes)
            : library_workspace(plan.workspace_bytes, st, &ws);
    if (rc != VKV_OK) return rc;
    return after_launch(vkv::launch_decode_append(ap, dp, plan, ws, st), "vkv_paged_decode_append");
}

size_t vkv_paged_prefill_workspace_size(const vkv_prefill_params* p) {
    if (check_prefill(p) != VKV_OK || p->num_seqs == 0 || p->num_query_tokens == 0) return 0;
    return vkv::plan_prefill(p).workspace_bytes;
}

int vkv_paged_prefill(const vkv_prefill_params* p, vkv_stream_t stream) {
    int rc = check_prefill(p);
    if (rc != VKV_OK || p->num_seqs == 0 || p->num_query_tokens == 0) return rc;
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const vkv::DecodePlan plan = vkv::plan_prefill(p);
    void* ws = p->workspace;
    rc = ws ? check_workspace(ws, p->workspace_bytes, plan.workspace_bytes)
            : library_workspace(plan.workspace_bytes, st, &ws);
    if (rc != VKV_OK) return rc;
    return after_launch(vkv::launch_prefill(p, plan, ws, st), "vkv_paged_prefill");
}

int vkv_check_block_pairs_host(const int32_t* block_pairs, int32_t num_pairs, int32_t num_blocks) {
    if (num_pairs < 0) return fail(VKV_ERR_SHAPE, "num_pairs < 0");
    if (num_pairs > 0 && !block_pairs) return fail(VKV_ERR_NULL, "block_pairs is NULL");
    std::unordered_set<int32_t> dsts;
    dsts.reserve(size_t(num_pairs) * 2);
    for (int32_t i = 0; i < num_pairs; ++i) {
        const int32_t s = block_pairs[2 * i], d = block_pairs[2 * i + 1];
        if (s < 0 || s >= num_blocks || d < 0 || d >= num_blocks)
            return fail(VKV_ERR_SHAPE, "pair %d (%d -> %d) outside [0, %d)", i, s, d, num_blocks);
        if (!dsts.insert(d).second) return fail(VKV_ERR_SHAPE, "destination block %d repeated", d);
    }
    for (int32_t i = 0; i < num_pairs; ++i)
        if (dsts.count(block_pairs[2 * i]))
            return fail(VKV_ERR_SHAPE, "block %d is both a source and a destination", block_pairs[2 * i]);
    return VKV_OK;
}

int vkv_copy_blocks(const vkv_block_plane* planes, int32_t num_planes, int32_t num_layers, int32_t num_blocks,
                    const int32_t* block_pairs, int32_t num_pairs, vkv_stream_t stream) {
    if (num_pairs < 0 || num_layers < 0 || num_blocks < 0) return fail(VKV_ERR_SHAPE, "negative size");
    if (num_pairs == 0 || num_layers == 0) return VKV_OK;
    if (!block_pairs) return fail(VKV_ERR_NULL, "block_pairs is NULL");
    vkv::PlaneSet ps;
    int rc = fill_planes(planes, num_planes, &ps);
    if (rc != VKV_OK) return rc;
    return after_launch(vkv::launch_copy_blocks(ps, num_layers, num_blocks, block_pairs, num_pairs,
                                                reinterpret_cast<hipStream_t>(stream)),
                        "vkv_copy_blocks");
}

size_t vkv_swap_host_block_bytes(const vkv_block_plane* planes, int32_t num_planes, int32_t num_layers) {
    if (!planes || num_planes < 1 || num_planes > 4 || num_layers < 0) return 0;
    size_t total = 0;
    for (int i = 0; i < num_planes; ++i) total += size_t(planes[i].block_bytes) * size_t(num_layers);
    return total;
}

int vkv_swap_blocks(const vkv_block_plane* dev_planes, int32_t num_planes, int32_t num_layers, int32_t num_dev_blocks,
                    void* host_base, int32_t num_host_blocks, const int32_t* block_pairs, int32_t num_pairs,
                    int32_t direction, vkv_stream_t stream) {
    if (num_pairs < 0 || num_layers < 0 || num_dev_blocks < 0 || num_host_blocks < 0)
        return fail(VKV_ERR_SHAPE, "negative size");
    if (direction != VKV_SWAP_OUT && direction != VKV_SWAP_IN) return fail(VKV_ERR_SHAPE, "bad direction");
    if (num_pairs == 0 || num_layers == 0) return VKV_OK;
    if (!block_pairs || !host_base) return fail(VKV_ERR_NULL, "block_pairs or host_base is NULL");
    vkv::PlaneSet ps;
    int rc = fill_planes(dev_planes, num_planes, &ps);
    if (rc != VKV_OK) return rc;
    // The kernel addresses host memory through its device mapping.
    void* dev_view = nullptr;
    hipError_t e = hipHostGetDevicePointer(&dev_view, host_base, 0);
    if (e != hipSuccess) return hip_status(e, "hipHostGetDevicePointer (host_base must come from hipHostMalloc)");
    const int64_t hbb = int64_t(vkv_swap_host_block_bytes(dev_planes, num_planes, num_layers));
    return after_launch(vkv::launch_swap_blocks(ps, num_layers, num_dev_blocks, static_cast<char*>(dev_view), hbb,
                                                num_host_blocks, block_pairs, num_pairs, direction,
                                                reinterpret_cast<hipStream_t>(stream)),
                        "vkv_swap_blocks");
}

}  // extern "C"
