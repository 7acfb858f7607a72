// block_manager.hpp — physical KV block pool, API kept as in the reference
// (include/vllm/core/block_manager.hpp:8-104 of jiamumuzhao/vllm-cpp): int32
// block ids, LIFO free list, reference counts.  LogicalBlock and BlockTable are
// declared, as there, but have no definition in either code base.
#pragma once

#include <cstdint>
#include <memory>
#include <optional>
#include <unordered_map>
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

    // Prefix cache.  The reference declares find_prefix_blocks and returns {}
    // (src/core/block_manager.cpp:105-108); here it returns the live blocks
    // (ref_count > 0) that hold the longest run of full leading blocks of
    // token_ids registered by cache_prefix_blocks, at most max_blocks.  With
    // nothing registered it returns {} as the reference does.  A caller that
    // adopts the blocks takes a reference with inc_ref.
    std::vector<int32_t> find_prefix_blocks(const std::vector<int32_t>& token_ids, size_t max_blocks) const;
    // Registers the full blocks of a sequence (block i holds tokens
    // [i*block_size, (i+1)*block_size)); a block leaves the cache when freed.
    void cache_prefix_blocks(const std::vector<int32_t>& token_ids, const std::vector<int32_t>& block_table);

    // --- sharing, copy-on-write and swap.  No counterpart in the reference:
    // its hooks are LogicalBlock::ref_count ("for prefix caching / sharing"),
    // BlockTable::to_id_list ("for preemption / swap") and the CPU free list,
    // all unused there (include/vllm/core/block_manager.hpp:17,39-40;
    // src/core/block_manager.cpp:11,15-17).  Pair lists are flat
    // [src, dst, src, dst, ...] int32, the layout vkv_copy_blocks and
    // vkv_swap_blocks take once uploaded.  The caller enqueues the copy or swap
    // before any later write to the blocks on the same stream.

    // A child sequence sharing every block of the parent (each ref_count + 1).
    std::vector<int32_t> fork_sequence(const std::vector<int32_t>& parent_table);

    // Copy-on-write before the token at `position` is written: when the block
    // holding it is shared (ref_count > 1), a fresh block replaces it in the
    // table, the shared one loses this sequence's reference and (old, new) is
    // appended to copy_pairs.  False (nothing changed) if no block is free or
    // the table does not reach position.
    bool make_writable(std::vector<int32_t>& block_table, size_t position, std::vector<int32_t>& copy_pairs);

    // Preemption by swapping instead of recompute (the reference recomputes,
    // src/core/scheduler.cpp:168-188).  swap_out gives every GPU block of the
    // table a CPU block, appends (gpu, cpu) pairs, drops the GPU references and
    // leaves CPU ids in the table; swap_in is the reverse with (cpu, gpu)
    // pairs.  False (nothing changed) when the other pool lacks free blocks.
    bool swap_out(std::vector<int32_t>& block_table, std::vector<int32_t>& swap_pairs);
    bool swap_in(std::vector<int32_t>& block_table, std::vector<int32_t>& swap_pairs);
    bool can_swap_in(size_t num_blocks) const { return can_allocate(num_blocks); }

    // Current reference count of a block (0 when free or out of range).
    int32_t ref_count(int32_t physical_id) const;

  private:
    struct PhysicalBlock {
        int32_t ref_count = 0;
        bool is_free = true;
        uint64_t prefix_key = 0;  // prefix-cache entry naming this block, 0 = none
    };
    struct PrefixEntry {
        uint64_t parent;
        std::vector<int32_t> tokens;
        int32_t block;
    };

    static uint64_t prefix_key(uint64_t parent, const int32_t* tokens, size_t n);
    void forget_prefix(int32_t physical_id);
    std::optional<int32_t> acquire_cpu_block();
    void release_cpu_block(int32_t id);

    size_t block_size_;
    size_t num_gpu_blocks_;
    size_t num_cpu_blocks_;
    std::vector<PhysicalBlock> gpu_blocks_;
    std::vector<PhysicalBlock> cpu_blocks_;
    std::vector<int32_t> gpu_free_list_;
    std::vector<int32_t> cpu_free_list_;
    std::unordered_map<uint64_t, PrefixEntry> prefix_;
};

}  // namespace vllm
