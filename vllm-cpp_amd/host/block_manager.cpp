// block_manager.cpp — BlockManager with the reference's id semantics
// (src/core/block_manager.cpp:7-108): ids 0..N-1, free list used as a stack
// (the initial list is 0..N-1, so a fresh pool hands out N-1 first), ref
// count 1 on acquire, all-or-nothing sequence allocation.
//
// One deliberate difference: releasing or dec_ref-ing a block that is already
// free does nothing.  The reference pushes such an id onto the free list a
// second time, after which two sequences can be handed the same block.
#include "vllm/core/block_manager.hpp"

#include <stdexcept>

namespace vllm {

BlockManager::BlockManager(size_t block_size, size_t num_gpu_blocks, size_t num_cpu_blocks)
    : block_size_(block_size), num_gpu_blocks_(num_gpu_blocks), num_cpu_blocks_(num_cpu_blocks) {
    if (block_size_ == 0) throw std::invalid_argument("KV block size must be greater than zero");
    gpu_blocks_.assign(num_gpu_blocks_, PhysicalBlock{});
    cpu_blocks_.assign(num_cpu_blocks_, PhysicalBlock{});
    gpu_free_list_.reserve(num_gpu_blocks_);
    for (size_t id = 0; id < num_gpu_blocks_; ++id) gpu_free_list_.push_back(int32_t(id));
    cpu_free_list_.reserve(num_cpu_blocks_);
    for (size_t id = 0; id < num_cpu_blocks_; ++id) cpu_free_list_.push_back(int32_t(id));
}

std::optional<int32_t> BlockManager::acquire_block() {
    if (gpu_free_list_.empty()) return std::nullopt;
    const int32_t id = gpu_free_list_.back();
    gpu_free_list_.pop_back();
    PhysicalBlock& b = gpu_blocks_[size_t(id)];
    b.is_free = false;
    b.ref_count = 1;
    return id;
}

void BlockManager::release_block(int32_t physical_id) {
    if (physical_id < 0 || size_t(physical_id) >= num_gpu_blocks_) return;
    PhysicalBlock& b = gpu_blocks_[size_t(physical_id)];
    if (b.is_free) return;
    b.is_free = true;
    b.ref_count = 0;
    gpu_free_list_.push_back(physical_id);
}

void BlockManager::inc_ref(int32_t physical_id) {
    if (physical_id < 0 || size_t(physical_id) >= num_gpu_blocks_) return;
    ++gpu_blocks_[size_t(physical_id)].ref_count;
}

bool BlockManager::dec_ref(int32_t physical_id) {
    if (physical_id < 0 || size_t(physical_id) >= num_gpu_blocks_) return false;
    PhysicalBlock& b = gpu_blocks_[size_t(physical_id)];
    if (b.is_free) return false;
    if (--b.ref_count > 0) return false;
    b.ref_count = 0;
    b.is_free = true;
    gpu_free_list_.push_back(physical_id);
    return true;
}

size_t BlockManager::num_free_gpu_blocks() const { return gpu_free_list_.size(); }

size_t BlockManager::num_free_cpu_blocks() const { return cpu_free_list_.size(); }

bool BlockManager::can_allocate(size_t num_blocks) const { return gpu_free_list_.size() >= num_blocks; }

static size_t blocks_for(size_t tokens, size_t block_size) { return (tokens + block_size - 1) / block_size; }

std::vector<int32_t> BlockManager::allocate_for_sequence(size_t num_tokens) {
    const size_t need = blocks_for(num_tokens, block_size_);
    std::vector<int32_t> table;
    table.reserve(need);
    while (table.size() < need) {
        std::optional<int32_t> id = acquire_block();
        if (!id) {
            free_sequence(table);  // give back what this call took, in table order
            return {};
        }
        table.push_back(*id);
    }
    return table;
}

bool BlockManager::ensure_sequence_capacity(std::vector<int32_t>& block_table, size_t num_tokens) {
    const size_t need = blocks_for(num_tokens, block_size_);
    const size_t had = block_table.size();
    while (block_table.size() < need) {
        std::optional<int32_t> id = acquire_block();
        if (!id) {
            // undo newest first, so the free list ends as it started
            while (block_table.size() > had) {
                release_block(block_table.back());
                block_table.pop_back();
            }
            return false;
        }
        block_table.push_back(*id);
    }
    return true;
}

void BlockManager::free_sequence(const std::vector<int32_t>& block_table) {
    for (int32_t id : block_table) dec_ref(id);
}

std::vector<int32_t> BlockManager::find_prefix_blocks(const std::vector<int32_t>&, size_t) const { return {}; }

int32_t BlockManager::ref_count(int32_t physical_id) const {
    if (physical_id < 0 || size_t(physical_id) >= num_gpu_blocks_) return 0;
    return gpu_blocks_[size_t(physical_id)].ref_count;
}

}  // namespace vllm
