// block_manager.cpp — BlockManager with the reference's id semantics
// (src/core/block_manager.cpp:7-108): ids 0..N-1, free list used as a stack
// (the initial list is 0..N-1, so a fresh pool hands out N-1 first), ref
// count 1 on acquire, all-or-nothing sequence allocation.
//
// One deliberate difference: releasing or dec_ref-ing a block that is already
// free does nothing.  The reference pushes such an id onto the free list a
// second time, after which two sequences can be handed the same block.
#include "vllm/core/block_manager.hpp"

#include <algorithm>
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
    forget_prefix(physical_id);
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
    forget_prefix(physical_id);
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

// ---------------------------------------------------------------- prefix cache

uint64_t BlockManager::prefix_key(uint64_t parent, const int32_t* tokens, size_t n) {
    // FNV-1a over the parent key and the block's token ids; 0 is reserved for "none".
    uint64_t h = 1469598103934665603ull;
    auto mix = [&h](uint64_t x) {
        for (int i = 0; i < 8; ++i) {
            h ^= (x >> (8 * i)) & 0xFFu;
            h *= 1099511628211ull;
        }
    };
    mix(parent);
    for (size_t i = 0; i < n; ++i) mix(uint64_t(uint32_t(tokens[i])));
    return h ? h : 1;
}

void BlockManager::forget_prefix(int32_t physical_id) {
    PhysicalBlock& b = gpu_blocks_[size_t(physical_id)];
    if (!b.prefix_key) return;
    auto it = prefix_.find(b.prefix_key);
    if (it != prefix_.end() && it->second.block == physical_id) prefix_.erase(it);
    b.prefix_key = 0;
}

void BlockManager::cache_prefix_blocks(const std::vector<int32_t>& token_ids, const std::vector<int32_t>& block_table) {
    const size_t full = std::min(token_ids.size() / block_size_, block_table.size());
    uint64_t parent = 0;
    for (size_t i = 0; i < full; ++i) {
        const int32_t* tok = token_ids.data() + i * block_size_;
        const uint64_t key = prefix_key(parent, tok, block_size_);
        const int32_t id = block_table[i];
        if (id < 0 || size_t(id) >= num_gpu_blocks_ || gpu_blocks_[size_t(id)].is_free) break;
        auto it = prefix_.find(key);
        const bool taken = it != prefix_.end() && it->second.block != id &&
                           !gpu_blocks_[size_t(it->second.block)].is_free;
        if (!taken) {  // the first live holder of a prefix keeps it
            if (gpu_blocks_[size_t(id)].prefix_key != key) forget_prefix(id);
            prefix_[key] = PrefixEntry{parent, std::vector<int32_t>(tok, tok + block_size_), id};
            gpu_blocks_[size_t(id)].prefix_key = key;
        }
        parent = key;
    }
}

std::vector<int32_t> BlockManager::find_prefix_blocks(const std::vector<int32_t>& token_ids, size_t max_blocks) const {
    std::vector<int32_t> out;
    const size_t full = std::min(token_ids.size() / block_size_, max_blocks);
    uint64_t parent = 0;
    for (size_t i = 0; i < full; ++i) {
        const int32_t* tok = token_ids.data() + i * block_size_;
        const uint64_t key = prefix_key(parent, tok, block_size_);
        auto it = prefix_.find(key);
        if (it == prefix_.end()) break;
        const PrefixEntry& e = it->second;
        const PhysicalBlock& b = gpu_blocks_[size_t(e.block)];
        if (e.parent != parent || b.is_free || b.ref_count <= 0 ||
            !std::equal(e.tokens.begin(), e.tokens.end(), tok))
            break;  // a hash collision or a block no longer holding the prefix
        out.push_back(e.block);
        parent = key;
    }
    return out;
}

// ---------------------------------------------------------------- fork / copy-on-write

std::vector<int32_t> BlockManager::fork_sequence(const std::vector<int32_t>& parent_table) {
    for (int32_t id : parent_table) inc_ref(id);
    return parent_table;
}

bool BlockManager::make_writable(std::vector<int32_t>& block_table, size_t position, std::vector<int32_t>& copy_pairs) {
    const size_t logical = position / block_size_;
    if (logical >= block_table.size()) return false;
    const int32_t old = block_table[logical];
    if (ref_count(old) <= 1) return true;  // already exclusive
    std::optional<int32_t> fresh = acquire_block();
    if (!fresh) return false;
    dec_ref(old);  // still held by the other sharers
    block_table[logical] = *fresh;
    copy_pairs.push_back(old);
    copy_pairs.push_back(*fresh);
    return true;
}

// ---------------------------------------------------------------- swap

std::optional<int32_t> BlockManager::acquire_cpu_block() {
    if (cpu_free_list_.empty()) return std::nullopt;
    const int32_t id = cpu_free_list_.back();
    cpu_free_list_.pop_back();
    cpu_blocks_[size_t(id)].is_free = false;
    cpu_blocks_[size_t(id)].ref_count = 1;
    return id;
}

void BlockManager::release_cpu_block(int32_t id) {
    if (id < 0 || size_t(id) >= num_cpu_blocks_ || cpu_blocks_[size_t(id)].is_free) return;
    cpu_blocks_[size_t(id)].is_free = true;
    cpu_blocks_[size_t(id)].ref_count = 0;
    cpu_free_list_.push_back(id);
}

bool BlockManager::swap_out(std::vector<int32_t>& block_table, std::vector<int32_t>& swap_pairs) {
    if (cpu_free_list_.size() < block_table.size()) return false;
    for (int32_t& id : block_table) {
        const int32_t cpu = *acquire_cpu_block();
        swap_pairs.push_back(id);
        swap_pairs.push_back(cpu);
        dec_ref(id);
        id = cpu;
    }
    return true;
}

bool BlockManager::swap_in(std::vector<int32_t>& block_table, std::vector<int32_t>& swap_pairs) {
    if (gpu_free_list_.size() < block_table.size()) return false;
    for (int32_t& id : block_table) {
        const int32_t gpu = *acquire_block();
        swap_pairs.push_back(id);
        swap_pairs.push_back(gpu);
        release_cpu_block(id);
        id = gpu;
    }
    return true;
}

int32_t BlockManager::ref_count(int32_t physical_id) const {
    if (physical_id < 0 || size_t(physical_id) >= num_gpu_blocks_) return 0;
    return gpu_blocks_[size_t(physical_id)].ref_count;
}

}  // namespace vllm
