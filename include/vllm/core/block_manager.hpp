// block_manager.hpp — physical KV block pool, API kept as in the reference
// (include/vllm/core/block_manager.hpp:8-104 of jiamumuzhao/vllm-cpp): int32
// block ids, LIFO free list, reference counts.  LogicalBlock and BlockTable are
// declared, as there, but have no definition in either code base.
#pragma once

#include <cstdint>
#include <memory>
#include <optional>
#include <vector>

namespace vllm {

class Sequence;

struct LogicalBlock {
    int32_t block_id;     // position of the block inside its sequence
    int32_t physical_id;  // id in the pool, -1 while none is assigned
    int32_t ref_count;    // sequences sharing this block
    bool is_committed;    // K/V of all its slots written
};

class BlockTable {
  public:
    explicit BlockTable(size_t block_size, size_t max_blocks);
    int32_t allocate_block(int32_t logical_idx);
    int32_t physical_id(int32_t logical_idx) const;
    void release_all();
    size_t num_blocks() const { return blocks_.size(); }
    size_t block_size() const { return block_size_; }
    std::vector<int32_t> to_id_list() const;

  private:
    size_t block_size_;
    std::vector<LogicalBlock> blocks_;
};

class BlockManager {
  public:
    // Throws std::invalid_argument for block_size == 0.
    BlockManager(size_t block_size, size_t num_gpu_blocks, size_t num_cpu_blocks);

    // Reserve a free physical block (the most recently freed first; a fresh
    // pool hands out num_gpu_blocks-1, -2, ...).  nullopt if none is free.
    std::optional<int32_t> acquire_block();

    // Return a block to the free pool.  Out-of-range ids are ignored; a block
    // that is already free is ignored too (the reference would list it twice).
    void release_block(int32_t physical_id);

    // Reference counting for blocks shared between sequences.
    void inc_ref(int32_t physical_id);
    // Returns true if the count reached zero and the block was freed.
    bool dec_ref(int32_t physical_id);

    // ceil(num_tokens / block_size) fresh blocks, or {} (nothing held) if the
    // pool runs out.
    std::vector<int32_t> allocate_for_sequence(size_t num_tokens);

    // Grow block_table to ceil(num_tokens / block_size) blocks; on failure the
    // blocks added by this call are released and false is returned.
    bool ensure_sequence_capacity(std::vector<int32_t>& block_table, size_t num_tokens);

    // dec_ref every block of the table.
    void free_sequence(const std::vector<int32_t>& block_table);

    size_t block_size() const { return block_size_; }
    size_t num_total_gpu_blocks() const { return num_gpu_blocks_; }
    size_t num_free_gpu_blocks() const;
    size_t num_total_cpu_blocks() const { return num_cpu_blocks_; }
    size_t num_free_cpu_blocks() const;
    bool can_allocate(size_t num_blocks) const;

    // Prefix caching is not implemented (as in the reference): always {}.
    std::vector<int32_t> find_prefix_blocks(const std::vector<int32_t>& token_ids, size_t max_blocks) const;

    // Current reference count of a block (0 when free or out of range).
    int32_t ref_count(int32_t physical_id) const;

  private:
    struct PhysicalBlock {
        int32_t ref_count = 0;
        bool is_free = true;
    };

    size_t block_size_;
    size_t num_gpu_blocks_;
    size_t num_cpu_blocks_;
    std::vector<PhysicalBlock> gpu_blocks_;
    std::vector<PhysicalBlock> cpu_blocks_;
    std::vector<int32_t> gpu_free_list_;
    std::vector<int32_t> cpu_free_list_;
};

}  // namespace vllm
