// step_loop.cpp — a native caller's loop of decode steps, for timing the
// launch-bound configurations (bench.py --suite c1) without the Python
// wrapper's per-call cost.  Measurement code only; links the library.
//
//   vkvb_step_loop      n eager steps on `stream`: vkv_reshape_and_cache then
//                       vkv_paged_decode, or (fused != 0) vkv_paged_decode_append.
//   vkvb_graph_create   one step captured into a HIP graph (on a side stream
//                       whose library workspace an eager step sizes first).
//   vkvb_graph_launch   n launches of that graph on `stream`.
//   vkvb_graph_destroy
//
// Every entry point returns 0, a hipError_t or a library status.
#include <hip/hip_runtime.h>

#include "vllm_kv_amd.h"

namespace {

struct StepGraph {
    hipStream_t capture = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

int step(const vkv_append_params* ap, const vkv_decode_params* dp, int fused, hipStream_t st) {
    if (fused) return vkv_paged_decode_append(ap, dp, st);
    int rc = vkv_reshape_and_cache(ap, st);
    return rc ? rc : vkv_paged_decode(dp, st);
}

}  // namespace

extern "C" {

int vkvb_step_loop(const vkv_append_params* ap, const vkv_decode_params* dp, int n, int fused, hipStream_t stream) {
    for (int i = 0; i < n; ++i) {
        const int rc = step(ap, dp, fused, stream);
        if (rc) return rc;
    }
    return 0;
}

int vkvb_graph_create(const vkv_append_params* ap, const vkv_decode_params* dp, int fused, void** handle) {
    if (!handle) return int(hipErrorInvalidValue);
    *handle = nullptr;
    StepGraph* g = new StepGraph;
    int rc = int(hipStreamCreateWithFlags(&g->capture, hipStreamNonBlocking));
    if (!rc) rc = step(ap, dp, fused, g->capture);  // sizes the capture stream's workspace
    if (!rc) rc = int(hipStreamSynchronize(g->capture));
    if (!rc) rc = int(hipStreamBeginCapture(g->capture, hipStreamCaptureModeThreadLocal));
    if (!rc) {
        const int step_rc = step(ap, dp, fused, g->capture);
        rc = int(hipStreamEndCapture(g->capture, &g->graph));
        if (!rc) rc = step_rc;
    }
    if (!rc) rc = int(hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0));
    if (rc) {
        if (g->exec) (void)hipGraphExecDestroy(g->exec);
        if (g->graph) (void)hipGraphDestroy(g->graph);
        if (g->capture) (void)hipStreamDestroy(g->capture);
        delete g;
        return rc;
    }
    *handle = g;
    return 0;
}

int vkvb_graph_launch(void* handle, int n, hipStream_t stream) {
    StepGraph* g = static_cast<StepGraph*>(handle);
    if (!g) return int(hipErrorInvalidValue);
    for (int i = 0; i < n; ++i) {
        const int rc = int(hipGraphLaunch(g->exec, stream));
        if (rc) return rc;
    }
    return 0;
}

int vkvb_graph_destroy(void* handle) {
    StepGraph* g = static_cast<StepGraph*>(handle);
    if (!g) return 0;
    (void)hipStreamSynchronize(g->capture);
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(g->graph);
    (void)vkv_release_workspace(g->capture);
    (void)hipStreamDestroy(g->capture);
    delete g;
    return 0;
}

}  // extern "C"
