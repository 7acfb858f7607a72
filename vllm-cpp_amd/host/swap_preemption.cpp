// swap_preemption.cpp — vllm::SwapPreemption (include/vllm/core/swap_preemption.hpp).
#include "vllm/core/swap_preemption.hpp"

#include <algorithm>
#include <stdexcept>

#include "vllm/utils/hip_utils.hpp"
#include "vllm_kv_amd.h"

namespace vllm {

SwapPreemption::SwapPreemption(BlockManager& bm, KVCache& cache, void* host_pool)
    : bm_(bm), cache_(cache), host_pool_(host_pool) {
    if (!host_pool) throw std::invalid_argument("SwapPreemption needs a host pool");
    dev_pairs_cap_ = 2 * std::max<size_t>(std::max(bm.num_total_gpu_blocks(), bm.num_total_cpu_blocks()), 1);
    VLLM_HIP_CHECK(hipMalloc(&dev_pairs_, dev_pairs_cap_ * sizeof(int32_t)));
    VLLM_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&host_pairs_), dev_pairs_cap_ * sizeof(int32_t)));
    VLLM_HIP_CHECK(hipEventCreateWithFlags(&uploaded_, hipEventDisableTiming));
    VLLM_HIP_CHECK(hipEventCreateWithFlags(&swapped_, hipEventDisableTiming));
}

SwapPreemption::~SwapPreemption() {
    // the swap kernels read dev_pairs_: let them finish before it is freed
    if (swap_enqueued_) (void)hipEventSynchronize(swapped_);
    if (upload_pending_) (void)hipEventSynchronize(uploaded_);
    (void)hipEventDestroy(swapped_);
    (void)hipEventDestroy(uploaded_);
    (void)hipHostFree(host_pairs_);
    (void)hipFree(dev_pairs_);
}

int SwapPreemption::pick_victim(const std::vector<SwappableSequence*>& running, const SwappableSequence* except) {
    for (size_t i = running.size(); i > 0; --i) {
        const SwappableSequence* s = running[i - 1];
        if (s == except || s->finished || s->block_table.empty()) continue;
        return int(i - 1);
    }
    return -1;
}

void SwapPreemption::enqueue_swap(const std::vector<int32_t>& pairs, int32_t direction, hipStream_t stream) {
    const size_t n = pairs.size() / 2;
    if (n == 0) return;
    if (pairs.size() > dev_pairs_cap_) throw std::length_error("SwapPreemption: more pairs than the pool has blocks");
    // The pinned staging buffer may still feed the previous upload.
    if (upload_pending_) VLLM_HIP_CHECK(hipEventSynchronize(uploaded_));
    // The previous swap (perhaps on another stream) may still read dev_pairs_
    // and the blocks this one reuses: order this one after it.
    if (swap_enqueued_) VLLM_HIP_CHECK(hipStreamWaitEvent(stream, swapped_, 0));
    std::copy(pairs.begin(), pairs.end(), host_pairs_);
    VLLM_HIP_CHECK(
        hipMemcpyAsync(dev_pairs_, host_pairs_, pairs.size() * sizeof(int32_t), hipMemcpyHostToDevice, stream));
    VLLM_HIP_CHECK(hipEventRecord(uploaded_, stream));
    upload_pending_ = true;
    // the swap kernel after the upload on the same stream reads the list
    cache_.swap_blocks(host_pool_, int32_t(bm_.num_total_cpu_blocks()), dev_pairs_, int32_t(n), direction, stream);
    VLLM_HIP_CHECK(hipEventRecord(swapped_, stream));
    swap_enqueued_ = true;
}

void SwapPreemption::wait_swaps(hipStream_t stream) {
    if (swap_enqueued_) VLLM_HIP_CHECK(hipStreamWaitEvent(stream, swapped_, 0));
}

bool SwapPreemption::preempt_one(std::vector<SwappableSequence*>& running, std::deque<SwappableSequence*>& waiting,
                                 const SwappableSequence* except, hipStream_t stream) {
    const int v = pick_victim(running, except);
    if (v < 0) return false;
    SwappableSequence* victim = running[size_t(v)];
    std::vector<int32_t> pairs;
    if (!bm_.swap_out(victim->block_table, pairs)) return false;
    enqueue_swap(pairs, VKV_SWAP_OUT, stream);
    victim->swapped_out = true;
    running.erase(running.begin() + v);
    waiting.push_back(victim);
    return true;
}

bool SwapPreemption::swap_in(SwappableSequence& seq, hipStream_t stream) {
    if (!seq.swapped_out) return true;
    std::vector<int32_t> pairs;
    if (!bm_.swap_in(seq.block_table, pairs)) return false;
    enqueue_swap(pairs, VKV_SWAP_IN, stream);
    seq.swapped_out = false;
    return true;
}

}  // namespace vllm
