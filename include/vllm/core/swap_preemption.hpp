// swap_preemption.hpp — preemption by swapping a sequence's KV blocks to
// pinned host memory instead of recomputing them.
//
// The reference preempts by recompute (src/core/scheduler.cpp:168-188): it
// walks the running groups from the back, skips the group it is making room
// for, finished groups and groups without blocks, frees the victim's blocks,
// marks it for recompute and moves it to the back of the waiting queue; on
// re-admission (promote_to_running, :147-166) it gets fresh blocks and replays
// its tokens.  SwapPreemption keeps that victim order and queue position, but
// the victim's blocks go to host memory (BlockManager::swap_out, then
// vkv_swap_blocks on the caller's stream) and come back into fresh GPU blocks
// on re-admission (BlockManager::swap_in, vkv_swap_blocks): no token is
// recomputed.  Single-threaded, like BlockManager.
//
// Stream ordering.  The block ids a swap gives up return to BlockManager's
// free lists when the swap is enqueued, before its kernel has copied them:
// preempt_one frees the victim's GPU blocks while the swap-out still reads
// them, swap_in frees its CPU blocks while the swap-in still reads them.  So:
//   - swaps of one instance are ordered among themselves by the instance (each
//     swap's stream waits for the previous swap, whatever streams they use);
//   - every other write into the KV cache (append, copy_blocks, a prefill's
//     cache writes) that runs on a stream other than the swap's must be
//     ordered after it: call wait_swaps(that_stream) after preempt_one /
//     swap_in and before enqueuing the write.  Running all KV writes on the
//     swap's stream orders them too.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <deque>
#include <vector>

#include "vllm/core/block_manager.hpp"
#include "vllm/memory/kv_cache.hpp"

namespace vllm {

// A sequence as the preemption policy sees it.
struct SwappableSequence {
    int64_t seq_id = 0;
    std::vector<int32_t> block_table;  // GPU ids while resident, CPU ids while swapped out
    bool finished = false;
    bool swapped_out = false;
};

class SwapPreemption {
  public:
    // host_pool: hipHostMalloc memory of at least
    // bm.num_total_cpu_blocks() * cache.host_block_bytes() bytes, holding CPU
    // block c at c * host_block_bytes().  Allocates a small device buffer for
    // the pair lists and a pinned host buffer they are uploaded from (one each
    // per instance).
    SwapPreemption(BlockManager& bm, KVCache& cache, void* host_pool);
    ~SwapPreemption();
    SwapPreemption(const SwapPreemption&) = delete;
    SwapPreemption& operator=(const SwapPreemption&) = delete;

    // The reference's victim: the last entry of running that is not `except`,
    // not finished and holds blocks; -1 if there is none.
    static int pick_victim(const std::vector<SwappableSequence*>& running, const SwappableSequence* except);

    // Swap the victim out (enqueued on stream), erase it from running and
    // append it to waiting.  False, with nothing changed, when there is no
    // victim or the CPU pool cannot hold its blocks.
    bool preempt_one(std::vector<SwappableSequence*>& running, std::deque<SwappableSequence*>& waiting,
                     const SwappableSequence* except, hipStream_t stream);

    // Re-admission of a swapped-out sequence: its blocks are swapped back into
    // fresh GPU blocks (enqueued on stream) and its table holds their ids.
    // False, with nothing changed, when the GPU pool lacks free blocks.
    bool swap_in(SwappableSequence& seq, hipStream_t stream);

    // Makes `stream` wait (on the device, no host sync) until every swap this
    // instance has enqueued so far has finished; a no-op before the first one.
    void wait_swaps(hipStream_t stream);

  private:
    void enqueue_swap(const std::vector<int32_t>& pairs, int32_t direction, hipStream_t stream);

    BlockManager& bm_;
    KVCache& cache_;
    void* host_pool_;
    int32_t* dev_pairs_ = nullptr;  // capacity: 2 * max(GPU blocks, CPU blocks) ids
    size_t dev_pairs_cap_ = 0;
    // Pinned staging of the pair list: the upload is asynchronous, so the
    // buffer is rewritten only after the previous upload's event completed.
    int32_t* host_pairs_ = nullptr;
    hipEvent_t uploaded_ = nullptr;
    bool upload_pending_ = false;
    // Recorded after each swap kernel: the next swap and wait_swaps wait on it.
    hipEvent_t swapped_ = nullptr;
    bool swap_enqueued_ = false;
};

}  // namespace vllm
