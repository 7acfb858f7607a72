// bm_trace_driver.cpp — TEST INFRASTRUCTURE ONLY.
//
// Runs a script of BlockManager operations read from stdin and prints one line
// per result.  The same source is compiled twice by oracle/Makefile: against
// the reference's src/core/block_manager.cpp (-> _ref/bm_trace_ref) and against
// this repository's vllm-cpp_amd/host/block_manager.cpp (-> _build/bm_trace_ours),
// so the two implementations can be compared on identical operation sequences.
//
// Script lines:  new BS NGPU NCPU | acquire | release ID | inc ID | dec ID |
//                alloc NTOK | ensure T NTOK | free T | can N | nfree
// "alloc" appends a new table (index = number of tables so far); tables are
// referenced by that index in ensure/free.
#include <iostream>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "vllm/core/block_manager.hpp"

static void print_table(const std::vector<int32_t>& t) {
    std::cout << t.size();
    for (int32_t id : t) std::cout << ' ' << id;
    std::cout << '\n';
}

int main() {
    std::unique_ptr<vllm::BlockManager> bm;
    std::vector<std::vector<int32_t>> tables;
    std::string line;
    while (std::getline(std::cin, line)) {
        std::istringstream in(line);
        std::string op;
        if (!(in >> op)) continue;
        if (op == "new") {
            size_t bs, ng, nc;
            in >> bs >> ng >> nc;
            tables.clear();
            try {
                bm.reset(new vllm::BlockManager(bs, ng, nc));
                std::cout << "ok\n";
            } catch (const std::invalid_argument&) {
                bm.reset();
                std::cout << "invalid_argument\n";
            }
        } else if (op == "acquire") {
            auto id = bm->acquire_block();
            std::cout << (id ? std::to_string(*id) : std::string("none")) << '\n';
        } else if (op == "release") {
            int32_t id;
            in >> id;
            bm->release_block(id);
            std::cout << bm->num_free_gpu_blocks() << '\n';
        } else if (op == "inc") {
            int32_t id;
            in >> id;
            bm->inc_ref(id);
            std::cout << bm->num_free_gpu_blocks() << '\n';
        } else if (op == "dec") {
            int32_t id;
            in >> id;
            std::cout << (bm->dec_ref(id) ? 1 : 0) << ' ' << bm->num_free_gpu_blocks() << '\n';
        } else if (op == "alloc") {
            size_t n;
            in >> n;
            tables.push_back(bm->allocate_for_sequence(n));
            print_table(tables.back());
        } else if (op == "ensure") {
            size_t t, n;
            in >> t >> n;
            const bool ok = bm->ensure_sequence_capacity(tables.at(t), n);
            std::cout << (ok ? 1 : 0) << ' ';
            print_table(tables.at(t));
        } else if (op == "free") {
            size_t t;
            in >> t;
            bm->free_sequence(tables.at(t));
            tables.at(t).clear();
            std::cout << bm->num_free_gpu_blocks() << '\n';
        } else if (op == "can") {
            size_t n;
            in >> n;
            std::cout << (bm->can_allocate(n) ? 1 : 0) << '\n';
        } else if (op == "nfree") {
            std::cout << bm->num_free_gpu_blocks() << ' ' << bm->num_free_cpu_blocks() << ' '
                      << bm->num_total_gpu_blocks() << ' ' << bm->num_total_cpu_blocks() << '\n';
        } else {
            std::cout << "?\n";
        }
    }
    return 0;
}
