// hip_utils.hpp — error handling for the HIP calls of the paged KV path.
//
// Mirrors the reference's VLLM_CUDA_CHECK (include/vllm/utils/cuda_utils.hpp:13-21):
// a failing call prints file:line and the runtime's message, then aborts.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>

#include "vllm_kv_amd.h"

#define VLLM_HIP_CHECK(call)                                                                  \
    do {                                                                                      \
        hipError_t _err = (call);                                                             \
        if (_err != hipSuccess) {                                                             \
            std::fprintf(stderr, "HIP error at %s:%d: %s (%s)\n", __FILE__, __LINE__,         \
                         hipGetErrorString(_err), hipGetErrorName(_err));                     \
            std::abort();                                                                     \
        }                                                                                     \
    } while (0)

// For the C ABI of vllm_kv_amd.h: non-zero status aborts with vkv_last_error().
#define VLLM_KV_CHECK(call)                                                                   \
    do {                                                                                      \
        int _rc = (call);                                                                     \
        if (_rc != 0) {                                                                       \
            std::fprintf(stderr, "vllm_kv_amd error %d at %s:%d: %s\n", _rc, __FILE__, __LINE__, \
                         vkv_last_error());                                                   \
            std::abort();                                                                     \
        }                                                                                     \
    } while (0)
