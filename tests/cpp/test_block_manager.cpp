// test_block_manager.cpp — BlockManager behaviour pinned by the reference's own
// unit tests (tests/unit/test_block_manager.cpp:4-26 and the block accounting of
// tests/unit/test_scheduler.cpp:27-36, 91-93), restated without gtest, plus the
// LIFO closed form of the id order (src/core/block_manager.cpp:12-14, 20-26).
#include <optional>
#include <stdexcept>
#include <vector>

#include "check.hpp"
#include "vllm/core/block_manager.hpp"

using vllm::BlockManager;

TEST_CASE(acquire_release) {  // reference test_block_manager.cpp:4-12
    BlockManager bm(16, 10, 0);
    CHECK_EQ(bm.num_free_gpu_blocks(), 10u);
    auto blk = bm.acquire_block();
    CHECK(blk.has_value());
    CHECK_EQ(bm.num_free_gpu_blocks(), 9u);
    bm.release_block(*blk);
    CHECK_EQ(bm.num_free_gpu_blocks(), 10u);
}

TEST_CASE(ref_counting) {  // reference test_block_manager.cpp:14-20
    BlockManager bm(16, 5, 0);
    auto blk = bm.acquire_block();
    bm.inc_ref(*blk);
    CHECK(!bm.dec_ref(*blk));
    CHECK(bm.dec_ref(*blk));
}

TEST_CASE(can_allocate) {  // reference test_block_manager.cpp:22-26
    BlockManager bm(16, 3, 0);
    CHECK(bm.can_allocate(2));
    CHECK(!bm.can_allocate(5));
}

TEST_CASE(zero_block_size_throws) {  // reference test_scheduler.cpp:91-93
    bool threw = false;
    try {
        BlockManager bm(0, 4, 0);
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    CHECK(threw);
}

TEST_CASE(prompt_of_one_block) {  // block accounting of reference test_scheduler.cpp:27-36
    BlockManager bm(16, 4, 0);
    auto table = bm.allocate_for_sequence(16);
    CHECK_EQ(table.size(), 1u);
    CHECK_EQ(bm.num_free_gpu_blocks(), 3u);
    CHECK(bm.ensure_sequence_capacity(table, 17));  // decode crosses into a second block
    CHECK_EQ(table.size(), 2u);
    CHECK_EQ(bm.num_free_gpu_blocks(), 2u);
}

TEST_CASE(lifo_id_order) {  // free list starts 0..N-1 and is popped from the back
    const int N = 7;
    BlockManager bm(16, N, 0);
    for (int i = 0; i < N; ++i) CHECK_EQ(*bm.acquire_block(), N - 1 - i);
    CHECK(!bm.acquire_block().has_value());
    bm.release_block(2);
    bm.release_block(5);
    CHECK_EQ(*bm.acquire_block(), 5);  // most recently freed first
    CHECK_EQ(*bm.acquire_block(), 2);
}

TEST_CASE(allocate_for_sequence_all_or_nothing) {
    BlockManager bm(16, 3, 0);
    auto t = bm.allocate_for_sequence(16 * 4);  // needs 4 of 3
    CHECK(t.empty());
    CHECK_EQ(bm.num_free_gpu_blocks(), 3u);
    // The failed call took 2, 1, 0 and gave them back in table order, so the
    // stack now pops 0, 1, 2 (the reference's own build does the same).
    auto ok = bm.allocate_for_sequence(33);
    CHECK_EQ(ok.size(), 3u);
    CHECK_EQ(ok[0], 0);
    CHECK_EQ(ok[2], 2);
}

TEST_CASE(ensure_capacity_rolls_back) {
    BlockManager bm(16, 4, 0);
    auto t = bm.allocate_for_sequence(16);  // id 3
    auto other = bm.allocate_for_sequence(16);  // id 2
    CHECK(!bm.ensure_sequence_capacity(t, 16 * 4));  // needs 3 more, 2 free
    CHECK_EQ(t.size(), 1u);
    CHECK_EQ(bm.num_free_gpu_blocks(), 2u);
    // the rolled-back blocks return in reverse, so the next acquire sees the same order
    CHECK_EQ(*bm.acquire_block(), 1);
    (void)other;
}

TEST_CASE(free_sequence_and_sharing) {
    BlockManager bm(16, 4, 0);
    auto a = bm.allocate_for_sequence(32);  // ids 3, 2
    for (int id : a) bm.inc_ref(id);       // a fork shares both blocks
    bm.free_sequence(a);                    // parent done: still held by the fork
    CHECK_EQ(bm.num_free_gpu_blocks(), 2u);
    CHECK_EQ(bm.ref_count(3), 1);
    bm.free_sequence(a);                    // fork done
    CHECK_EQ(bm.num_free_gpu_blocks(), 4u);
}

TEST_CASE(double_free_is_ignored) {  // documented divergence from the reference
    BlockManager bm(16, 3, 0);
    auto id = *bm.acquire_block();
    bm.release_block(id);
    bm.release_block(id);
    CHECK_EQ(bm.num_free_gpu_blocks(), 3u);
    CHECK(!bm.dec_ref(id));
    CHECK_EQ(bm.num_free_gpu_blocks(), 3u);
    // three distinct ids come back out
    int a = *bm.acquire_block(), b = *bm.acquire_block(), c = *bm.acquire_block();
    CHECK(a != b && b != c && a != c);
}

TEST_CASE(out_of_range_ids_ignored) {
    BlockManager bm(16, 3, 2);
    bm.release_block(-1);
    bm.release_block(3);
    bm.inc_ref(7);
    CHECK(!bm.dec_ref(-4));
    CHECK_EQ(bm.num_free_gpu_blocks(), 3u);
    CHECK_EQ(bm.num_free_cpu_blocks(), 2u);
    CHECK(bm.find_prefix_blocks({1, 2, 3}, 4).empty());
}

// ---- sharing, copy-on-write, swap and the prefix cache (no reference counterpart)

TEST_CASE(fork_shares_every_block) {
    BlockManager bm(4, 8, 0);
    auto parent = bm.allocate_for_sequence(10);  // 3 blocks: 7, 6, 5
    auto child = bm.fork_sequence(parent);
    CHECK(child == parent);
    for (int32_t id : parent) CHECK_EQ(bm.ref_count(id), 2);
    CHECK_EQ(bm.num_free_gpu_blocks(), 5u);
    bm.free_sequence(parent);  // the child keeps them
    for (int32_t id : child) CHECK_EQ(bm.ref_count(id), 1);
    CHECK_EQ(bm.num_free_gpu_blocks(), 5u);
}

TEST_CASE(copy_on_write_of_the_shared_tail) {
    BlockManager bm(4, 8, 0);
    auto parent = bm.allocate_for_sequence(10);  // ids 7, 6, 5; tokens 8..9 in block 5
    auto child = bm.fork_sequence(parent);
    std::vector<int32_t> pairs;
    CHECK(bm.make_writable(child, 10, pairs));   // token 10 goes into the shared block 5
    CHECK_EQ(pairs.size(), 2u);
    CHECK_EQ(pairs[0], 5);
    CHECK_EQ(pairs[1], 4);                       // the next fresh id (LIFO)
    CHECK_EQ(child[2], 4);
    CHECK_EQ(parent[2], 5);
    CHECK_EQ(bm.ref_count(5), 1);
    CHECK_EQ(bm.ref_count(4), 1);
    CHECK_EQ(bm.ref_count(7), 2);                // full blocks stay shared
    pairs.clear();
    CHECK(bm.make_writable(child, 11, pairs));   // now exclusive: no copy
    CHECK(pairs.empty());
    CHECK(!bm.make_writable(child, 12, pairs));  // past the table
    // no free block: nothing changes
    BlockManager small(4, 2, 0);
    auto a = small.allocate_for_sequence(8);
    auto b = small.fork_sequence(a);
    CHECK(!small.make_writable(b, 5, pairs));
    CHECK(b == a);
    CHECK_EQ(small.ref_count(a[1]), 2);
}

TEST_CASE(swap_out_and_back_in) {
    BlockManager bm(4, 6, 4);
    auto seq = bm.allocate_for_sequence(12);  // gpu 5, 4, 3
    auto other = bm.fork_sequence(seq);       // shared: swap-out drops one reference
    std::vector<int32_t> pairs;
    CHECK(bm.swap_out(seq, pairs));
    CHECK_EQ(pairs.size(), 6u);
    CHECK_EQ(pairs[0], 5);
    CHECK_EQ(pairs[1], 3);  // cpu ids LIFO from 3
    CHECK_EQ(pairs[3], 2);
    CHECK_EQ(pairs[5], 1);
    CHECK_EQ(seq[0], 3);
    CHECK_EQ(bm.num_free_cpu_blocks(), 1u);
    for (int32_t id : other) CHECK_EQ(bm.ref_count(id), 1);
    bm.free_sequence(other);
    CHECK_EQ(bm.num_free_gpu_blocks(), 6u);
    std::vector<int32_t> back;
    CHECK(bm.swap_in(seq, back));
    CHECK_EQ(back.size(), 6u);
    CHECK_EQ(back[0], 3);
    CHECK_EQ(back[1], 3);   // gpu ids LIFO: 3 was freed last
    CHECK_EQ(bm.num_free_cpu_blocks(), 4u);
    CHECK_EQ(bm.num_free_gpu_blocks(), 3u);
    // not enough CPU blocks: nothing changes
    auto big = bm.allocate_for_sequence(12);
    auto copy = big;
    std::vector<int32_t> p2;
    BlockManager tiny(4, 6, 2);
    auto t = tiny.allocate_for_sequence(12);
    auto t0 = t;
    CHECK(!tiny.swap_out(t, p2));
    CHECK(t == t0 && p2.empty());
    CHECK(big == copy);
}

TEST_CASE(prefix_cache_hits_live_blocks_only) {
    BlockManager bm(4, 8, 0);
    std::vector<int32_t> tokens = {1, 2, 3, 4, 5, 6, 7, 8, 9, 10};
    CHECK(bm.find_prefix_blocks(tokens, 8).empty());  // nothing registered: the reference's {}
    auto table = bm.allocate_for_sequence(tokens.size());
    bm.cache_prefix_blocks(tokens, table);            // 2 full blocks registered
    std::vector<int32_t> same = {1, 2, 3, 4, 5, 6, 7, 8, 42};
    auto hit = bm.find_prefix_blocks(same, 8);
    CHECK_EQ(hit.size(), 2u);
    CHECK_EQ(hit[0], table[0]);
    CHECK_EQ(hit[1], table[1]);
    CHECK_EQ(bm.find_prefix_blocks(same, 1).size(), 1u);
    std::vector<int32_t> diverge = {1, 2, 3, 4, 5, 6, 0, 8};
    CHECK_EQ(bm.find_prefix_blocks(diverge, 8).size(), 1u);
    std::vector<int32_t> shifted = {5, 6, 7, 8};      // same block content, other parent
    CHECK(bm.find_prefix_blocks(shifted, 8).empty());
    bm.free_sequence(table);                          // freed blocks leave the cache
    CHECK(bm.find_prefix_blocks(same, 8).empty());
}

int main() { return check::run_all(); }
