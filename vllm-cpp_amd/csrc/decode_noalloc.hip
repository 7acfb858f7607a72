// decode_noalloc.hip — vkv_paged_decode_noalloc: paged decode whose split-K
// workspace is a fixed device array of the library, for callers that cannot
// allocate (code under HIP graph capture, serving loops that forbid
// hipMalloc).  Same kernels and results as vkv_paged_decode.
//
// The array `scratch` is one per device (each device holds its own copy from
// the first call until the process ends).  Host code never passes its name to
// a kernel: the name is a host-side stand-in, not a device address.  The
// device address comes from hipGetSymbolAddress, once per device with that
// device current, and is kept per device.  Every call on a device shares the
// array, so calls that overlap on one device (two streams, two threads) race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "launch.hpp"
#include "vllm_kv_amd.h"

// Split-K partials of one call: 64 MiB covers, e.g., 256
// sequences x 32 query heads at head_dim 128 with contexts up to ~8k tokens.
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxDevices] = {};

int scratch_address(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return vkv::report_error(int(e), "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return vkv::report_error(VKV_ERR_DEVICE, "device %d >= %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return vkv::report_error(e != hipSuccess ? int(e) : VKV_ERR_DEVICE, "hipGetSymbolAddress (scratch): %s",
                                     hipGetErrorString(e));
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return VKV_OK;
}

}  // namespace

extern "C" int vkv_paged_decode_noalloc(const vkv_decode_params* p, vkv_stream_t stream) {
    int rc = vkv::check_decode_args(p);
    if (rc != VKV_OK || p->num_seqs == 0) return rc;
    const vkv::DecodePlan plan = vkv::plan_decode(p);
    if (plan.workspace_bytes > kScratchBytes)
        return vkv::report_error(VKV_ERR_WORKSPACE,
                                 "vkv_paged_decode_noalloc: the call needs %zu bytes of split-K scratch, more than "
                                 "the %zu the library holds; use vkv_paged_decode with a workspace",
                                 plan.workspace_bytes, kScratchBytes);
    void* ws = nullptr;
    rc = scratch_address(&ws);
    if (rc != VKV_OK) return rc;
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    // (the array keeps the last call's contents: its claim counters start
    // zeroed, as device memory of a code object does, and every call's merge
    // kernel returns them to zero)
    return vkv::report_launch(vkv::launch_decode(p, plan, ws, st), "vkv_paged_decode_noalloc");
}
