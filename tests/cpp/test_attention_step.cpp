// test_attention_step.cpp — AttentionMetadata + PagedAttentionLayer on a GPU
// against the reference's per-sequence, per-token semantics restated by the
// CPU oracle (oracle/kv_oracle.h; test infrastructure, linked only here).
//
// Four sequences get block tables from vllm::BlockManager and go through a
// prefill step (prompts of 5, 33, 1 and 18 tokens: chunks plus a one-token
// row), two decode steps, and a mixed step (one sequence appends a 7-token
// chunk while the others decode), on two layers.  After every step:
//   - the rotated queries and both layers' cache bytes (K, V, FP8 scales) are
//     bit-identical to oracle_rope + oracle_reshape_and_cache of the same tokens;
//   - the attention output is within the tolerance of oracle_paged_prefill,
//     which is one reference decode per query position (src/core/engine.cpp:157-164).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <deque>
#include <random>
#include <vector>

#include "check.hpp"
#include "kv_oracle.h"
#include "vllm/attention/attention_step.hpp"
#include "vllm/core/block_manager.hpp"
#include "vllm/core/swap_preemption.hpp"
#include "vllm/memory/kv_cache.hpp"
#include "vllm/utils/hip_utils.hpp"

namespace {

struct Geometry {
    int L, N, bs, H, Hkv, D;
    vllm::KVDtype io, kv;
};

size_t eb(vllm::KVDtype t) { return vllm::kv_dtype_bytes(t); }

// fp16 bits of x (the oracle's rounding) or the float itself.
void put(std::vector<uint8_t>& buf, size_t i, float x, vllm::KVDtype t) {
    if (t == vllm::KVDtype::kF16) {
        const uint16_t h = oracle_f32_to_f16(x);
        std::memcpy(buf.data() + 2 * i, &h, 2);
    } else {
        std::memcpy(buf.data() + 4 * i, &x, 4);
    }
}

float get(const std::vector<uint8_t>& buf, size_t i, vllm::KVDtype t) {
    if (t == vllm::KVDtype::kF16) {
        uint16_t h;
        std::memcpy(&h, buf.data() + 2 * i, 2);
        return oracle_f16_to_f32(h);
    }
    float x;
    std::memcpy(&x, buf.data() + 4 * i, 4);
    return x;
}

// The GPU cache and layer plus a host mirror of every layer's cache bytes,
// kept equal to the oracle's view of the same history.
struct Harness {
    Geometry g;
    bool fp8;
    vllm::KVCache cache;
    vllm::BlockManager bm;
    vllm::PagedAttentionLayer layer;
    vllm::AttentionMetadata md;
    static constexpr int P = 256;   // RoPE positions
    static constexpr int MB = 8;    // block-table row length
    static constexpr int MS = 8;    // sequences per step
    std::vector<float> cs;
    float* dcs = nullptr;
    size_t row, layer_elems;
    std::vector<std::vector<uint8_t>> hk, hv;
    std::vector<std::vector<float>> hks, hvs;
    std::mt19937 gen;
    std::normal_distribution<float> nd{0.f, 0.6f};
    hipStream_t st = nullptr;  // the stream the layer's kernels (appends included) run on

    Harness(const Geometry& geo, uint32_t seed, int cpu_blocks = 0)
        : g(geo),
          fp8(geo.kv == vllm::KVDtype::kFP8E4M3),
          cache(geo.L, geo.N, geo.bs, geo.Hkv, geo.D, nullptr, nullptr, geo.kv),
          bm(geo.bs, geo.N, cpu_blocks),
          layer(geo.H, geo.Hkv, geo.D, P),
          md(MS, 128, MB, geo.bs),
          cs(size_t(P) * geo.D),
          gen(seed) {
        std::printf("  scenario H%d Hkv%d D%d bs%d io %zuB kv %zuB\n", g.H, g.Hkv, g.D, g.bs, eb(g.io), eb(g.kv));
        VLLM_KV_CHECK(vkv_rope_cos_sin_host(10000.0f, g.D, P, cs.data()));
        VLLM_HIP_CHECK(hipMalloc(&dcs, cs.size() * 4));
        VLLM_HIP_CHECK(hipMemcpy(dcs, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
        layer.attach_rope_table(dcs, P);
        row = size_t(g.Hkv) * g.D;
        layer_elems = size_t(g.N) * g.bs * row;
        hk.resize(g.L);
        hv.resize(g.L);
        hks.resize(g.L);
        hvs.resize(g.L);
        for (int l = 0; l < g.L; ++l) {
            hk[l].assign(layer_elems * eb(g.kv), 0);
            hv[l].assign(layer_elems * eb(g.kv), 0);
            if (fp8) {
                hks[l].assign(size_t(g.N) * g.bs * g.Hkv, 0.f);
                hvs[l].assign(size_t(g.N) * g.bs * g.Hkv, 0.f);
            }
        }
    }
    ~Harness() { (void)hipFree(dcs); }

    size_t block_elems() const { return size_t(g.bs) * row; }

    // Host mirror of a device block move (copy-on-write or a swap round trip).
    void mirror_copy(int32_t src, int32_t dst) {
        const size_t be = block_elems() * eb(g.kv), se = size_t(g.bs) * g.Hkv;
        for (int l = 0; l < g.L; ++l) {
            std::memcpy(hk[l].data() + size_t(dst) * be, hk[l].data() + size_t(src) * be, be);
            std::memcpy(hv[l].data() + size_t(dst) * be, hv[l].data() + size_t(src) * be, be);
            if (fp8) {
                std::memcpy(hks[l].data() + size_t(dst) * se, hks[l].data() + size_t(src) * se, se * 4);
                std::memcpy(hvs[l].data() + size_t(dst) * se, hvs[l].data() + size_t(src) * se, se * 4);
            }
        }
    }

    // One step: new[s] tokens for sequence s on top of ctx[s] cached ones;
    // every layer runs and is checked against the oracle.
    void step(const std::vector<std::vector<int32_t>*>& tables, const std::vector<int>& ctx, const std::vector<int>& nnew,
              const char* what) {
        using vllm::KVDtype;
        const int S = int(tables.size());
        std::vector<vllm::StepSequence> ss;
        std::vector<int32_t> qsl = {0};
        for (int s = 0; s < S; ++s) {
            ss.push_back({tables[s]->data(), int32_t(tables[s]->size()), ctx[s], nnew[s]});
            qsl.push_back(qsl.back() + nnew[s]);
        }
        const int T = qsl.back();
        md.build(ss, st);
        CHECK_EQ(md.num_tokens(), T);
        CHECK_EQ(md.single_token_seqs(), int32_t(std::count(nnew.begin(), nnew.end(), 1)));
        CHECK_EQ(md.max_query_len(), *std::max_element(nnew.begin(), nnew.end()));
        std::vector<int32_t> slots(T), pos(T), cl(S);
        for (int s = 0, t = 0; s < S; ++s) {
            for (int j = 0; j < nnew[s]; ++j, ++t) {
                pos[t] = ctx[s] + j;
                slots[t] = (*tables[s])[pos[t] / g.bs] * g.bs + pos[t] % g.bs;  // attention.cpp:85-94
            }
            cl[s] = ctx[s] + nnew[s];
        }
        std::vector<int32_t> bt(size_t(S) * MB, 0);
        for (int s = 0; s < S; ++s) std::copy(tables[s]->begin(), tables[s]->end(), bt.begin() + s * MB);

        for (int l = 0; l < g.L; ++l) {
            std::vector<uint8_t> q(size_t(T) * g.H * g.D * eb(g.io)), k(size_t(T) * row * eb(g.io)),
                v(size_t(T) * row * eb(g.io));
            for (size_t i = 0; i < q.size() / eb(g.io); ++i) put(q, i, nd(gen), g.io);
            for (size_t i = 0; i < k.size() / eb(g.io); ++i) put(k, i, nd(gen), g.io);
            for (size_t i = 0; i < v.size() / eb(g.io); ++i) put(v, i, nd(gen), g.io);
            void *dq, *dk, *dv, *dout;
            VLLM_HIP_CHECK(hipMalloc(&dq, q.size()));
            VLLM_HIP_CHECK(hipMalloc(&dk, k.size()));
            VLLM_HIP_CHECK(hipMalloc(&dv, v.size()));
            VLLM_HIP_CHECK(hipMalloc(&dout, q.size()));
            VLLM_HIP_CHECK(hipMemcpy(dq, q.data(), q.size(), hipMemcpyHostToDevice));
            VLLM_HIP_CHECK(hipMemcpy(dk, k.data(), k.size(), hipMemcpyHostToDevice));
            VLLM_HIP_CHECK(hipMemcpy(dv, v.data(), v.size(), hipMemcpyHostToDevice));
            layer.forward(dout, dq, dk, dv, g.io, cache, md, size_t(l), st);
            VLLM_HIP_CHECK(hipDeviceSynchronize());

            // oracle: the reference's rope then row copies, then one decode per query position
            const int32_t sdt = int32_t(g.io);
            oracle_rope(q.data(), k.data(), 0, 0, cs.data(), pos.data(), 0, P, T, g.H, g.Hkv, g.D, sdt);
            oracle_reshape_and_cache(k.data(), v.data(), 0, 0, hk[l].data(), hv[l].data(),
                                     fp8 ? hks[l].data() : nullptr, fp8 ? hvs[l].data() : nullptr, slots.data(), T,
                                     g.Hkv, g.D, g.bs, g.N, sdt, int32_t(g.kv));
            std::vector<float> qf(size_t(T) * g.H * g.D), ref(qf.size());
            for (size_t i = 0; i < qf.size(); ++i) qf[i] = get(q, i, g.io);
            oracle_paged_prefill(ref.data(), qf.data(), hk[l].data(), hv[l].data(), fp8 ? hks[l].data() : nullptr,
                                 fp8 ? hvs[l].data() : nullptr, bt.data(), cl.data(), qsl.data(), S, g.H, g.Hkv, g.D,
                                 g.bs, MB, 1.0f / std::sqrt(float(g.D)), int32_t(g.kv), 1);

            std::vector<uint8_t> gq(q.size()), gout(q.size()), gk(hk[l].size()), gv(hv[l].size());
            VLLM_HIP_CHECK(hipMemcpy(gq.data(), dq, q.size(), hipMemcpyDeviceToHost));
            VLLM_HIP_CHECK(hipMemcpy(gout.data(), dout, q.size(), hipMemcpyDeviceToHost));
            VLLM_HIP_CHECK(hipMemcpy(gk.data(), cache.k_ptr(size_t(l), 0), gk.size(), hipMemcpyDeviceToHost));
            VLLM_HIP_CHECK(hipMemcpy(gv.data(), cache.v_ptr(size_t(l), 0), gv.size(), hipMemcpyDeviceToHost));
            CHECK(gq == q);
            CHECK(gk == hk[l]);
            CHECK(gv == hv[l]);
            if (fp8) {
                std::vector<float> gks(hks[l].size()), gvs(hvs[l].size());
                VLLM_HIP_CHECK(hipMemcpy(gks.data(), cache.k_scale_ptr(size_t(l), 0), gks.size() * 4,
                                         hipMemcpyDeviceToHost));
                VLLM_HIP_CHECK(hipMemcpy(gvs.data(), cache.v_scale_ptr(size_t(l), 0), gvs.size() * 4,
                                         hipMemcpyDeviceToHost));
                CHECK(gks == hks[l]);
                CHECK(gvs == hvs[l]);
            }
            const double atol = g.io == KVDtype::kF16 ? 2e-3 : 2e-5, rtol = g.io == KVDtype::kF16 ? 1e-2 : 1e-4;
            double worst = 0;
            for (size_t i = 0; i < ref.size(); ++i)
                worst = std::max(worst, std::fabs(double(get(gout, i, g.io)) - ref[i]) / (atol + rtol * std::fabs(ref[i])));
            if (worst > 1.0) std::printf("    %s layer %d: worst error ratio %.3f\n", what, l, worst);
            CHECK(worst <= 1.0);
            (void)hipFree(dq);
            (void)hipFree(dk);
            (void)hipFree(dv);
            (void)hipFree(dout);
        }
    }
};

void run_scenario(const Geometry& g, uint32_t seed) {
    Harness h(g, seed);
    std::vector<int> ctx = {0, 0, 0, 0};
    std::vector<int> prompt = {5, 33, 1, 18};
    std::vector<std::vector<int32_t>> tables(4);
    for (int s = 0; s < 4; ++s) {
        tables[s] = h.bm.allocate_for_sequence(size_t(prompt[s]));
        CHECK(!tables[s].empty());
    }
    std::vector<std::vector<int32_t>*> tp = {&tables[0], &tables[1], &tables[2], &tables[3]};
    // prompts (one of them a single token), decodes, a step where every
    // sequence has >= 2 new tokens (the prefill call then skips its decode
    // pass), a mixed step
    const std::vector<std::vector<int>> steps = {{5, 33, 1, 18}, {1, 1, 1, 1}, {3, 2, 2, 4}, {1, 1, 1, 1}, {1, 7, 1, 1}};
    for (size_t st = 0; st < steps.size(); ++st) {
        for (int s = 0; s < 4; ++s) CHECK(h.bm.ensure_sequence_capacity(tables[s], size_t(ctx[s] + steps[st][s])));
        h.step(tp, ctx, steps[st], "step");
        for (int s = 0; s < 4; ++s) ctx[s] += steps[st][s];
    }
}

// Fork (copy-on-write through KVCache::copy_blocks) and preemption by swap
// (KVCache::swap_blocks to pinned host memory and back into other block ids),
// driven by BlockManager; attention stays equal to the oracle's on the
// mirrored history throughout.
void run_fork_swap_scenario(const Geometry& g, uint32_t seed) {
    Harness h(g, seed, 16);
    std::vector<int32_t> a = h.bm.allocate_for_sequence(20);  // 2 blocks, the second partial
    std::vector<int> ctx = {0};
    h.step({&a}, ctx, {20}, "prefill A");
    std::vector<int32_t> b = h.bm.fork_sequence(a);  // B shares A's 20 tokens
    CHECK_EQ(h.bm.ref_count(a[1]), 2);

    // both append at position 20, inside the shared partial block
    std::vector<int32_t> pairs;
    CHECK(h.bm.make_writable(a, 20, pairs));
    CHECK(h.bm.make_writable(b, 20, pairs));
    CHECK_EQ(pairs.size(), 2u);  // only the first writer copies; B then owns the old block
    CHECK(a[1] != b[1]);
    int32_t* dpairs;
    VLLM_HIP_CHECK(hipMalloc(&dpairs, pairs.size() * 4));
    VLLM_HIP_CHECK(hipMemcpy(dpairs, pairs.data(), pairs.size() * 4, hipMemcpyHostToDevice));
    h.cache.copy_blocks(dpairs, int32_t(pairs.size() / 2), nullptr);
    h.mirror_copy(pairs[0], pairs[1]);
    std::vector<int> c2 = {20, 20};
    for (int i = 0; i < 3; ++i) {  // three decode steps of the two branches
        CHECK(h.bm.ensure_sequence_capacity(a, size_t(c2[0] + 1)));
        CHECK(h.bm.ensure_sequence_capacity(b, size_t(c2[1] + 1)));
        h.step({&a, &b}, c2, {1, 1}, "fork decode");
        c2[0] += 1;
        c2[1] += 1;
    }

    // preempt A by swapping it out; B runs a 9-token chunk meanwhile (the
    // freed ids are reused), then A comes back into fresh ids and decodes.
    const size_t hbb = h.cache.host_block_bytes();
    void* host = nullptr;
    VLLM_HIP_CHECK(hipHostMalloc(&host, hbb * 16, hipHostMallocDefault));
    std::vector<int32_t> out_pairs;
    const std::vector<int32_t> a_gpu = a;
    CHECK(h.bm.swap_out(a, out_pairs));
    CHECK_EQ(out_pairs.size(), 2 * a_gpu.size());
    int32_t* dswap;
    VLLM_HIP_CHECK(hipMalloc(&dswap, out_pairs.size() * 4));
    VLLM_HIP_CHECK(hipMemcpy(dswap, out_pairs.data(), out_pairs.size() * 4, hipMemcpyHostToDevice));
    h.cache.swap_blocks(host, 16, dswap, int32_t(out_pairs.size() / 2), VKV_SWAP_OUT, nullptr);
    VLLM_HIP_CHECK(hipDeviceSynchronize());
    // host mirror: remember A's blocks by CPU id
    std::vector<std::vector<uint8_t>> saved_k(a_gpu.size() * size_t(g.L)), saved_v(saved_k.size());
    const size_t be = h.block_elems() * eb(g.kv);
    for (size_t i = 0; i < a_gpu.size(); ++i)
        for (int l = 0; l < g.L; ++l) {
            const uint8_t* sk = h.hk[l].data() + size_t(a_gpu[i]) * be;
            const uint8_t* sv = h.hv[l].data() + size_t(a_gpu[i]) * be;
            saved_k[i * g.L + l].assign(sk, sk + be);
            saved_v[i * g.L + l].assign(sv, sv + be);
        }
    CHECK(h.bm.ensure_sequence_capacity(b, size_t(c2[1] + 9)));
    h.step({&b}, {c2[1]}, {9}, "chunk while A is swapped out");
    c2[1] += 9;
    std::vector<int32_t> in_pairs;
    CHECK(h.bm.swap_in(a, in_pairs));
    VLLM_HIP_CHECK(hipMemcpy(dswap, in_pairs.data(), in_pairs.size() * 4, hipMemcpyHostToDevice));
    h.cache.swap_blocks(host, 16, dswap, int32_t(in_pairs.size() / 2), VKV_SWAP_IN, nullptr);
    for (size_t i = 0; i < a.size(); ++i)
        for (int l = 0; l < g.L; ++l) {
            std::memcpy(h.hk[l].data() + size_t(a[i]) * be, saved_k[i * g.L + l].data(), be);
            std::memcpy(h.hv[l].data() + size_t(a[i]) * be, saved_v[i * g.L + l].data(), be);
        }
    CHECK(h.bm.ensure_sequence_capacity(a, size_t(c2[0] + 1)));
    CHECK(h.bm.ensure_sequence_capacity(b, size_t(c2[1] + 1)));
    h.step({&a, &b}, c2, {1, 1}, "decode after swap-in");
    (void)hipFree(dpairs);
    (void)hipFree(dswap);
    (void)hipHostFree(host);
}

// The reference's preemption pressure test (tests/unit/test_scheduler.cpp:47-89)
// with swap instead of recompute: a 3-block pool of 16-token blocks; A's
// 16-token prompt takes one block and its first decode a second; B's 16-token
// prompt takes the last one; when A reaches 32 tokens and needs a third block
// the victim is the last running sequence other than A, which is B; B is
// swapped out (not freed) and requeued, A grows to 3 blocks and decodes; when
// A finishes B is swapped back in, its blocks' bytes equal those it had before
// (every layer, K and V), and it decodes on.  Attention is checked against the
// oracle at every step.
//
// With side_stream, the swaps run on a side stream behind 1 GiB of unrelated
// work (a memset), while the layer's appends and attention run on a compute
// stream: the swap-out is still queued when A's next append is enqueued into
// the block B gave up, so only SwapPreemption::wait_swaps(compute) keeps that
// append from overwriting B's bytes before they are copied to the host.
void run_swap_preemption_scenario(const Geometry& g, uint32_t seed, bool side_stream = false) {
    Harness h(g, seed, 3);
    hipStream_t compute = nullptr, side = nullptr;
    void* busy = nullptr;
    const size_t busy_bytes = size_t(1) << 30;
    if (side_stream) {
        VLLM_HIP_CHECK(hipStreamCreateWithFlags(&compute, hipStreamNonBlocking));
        VLLM_HIP_CHECK(hipStreamCreateWithFlags(&side, hipStreamNonBlocking));
        VLLM_HIP_CHECK(hipMalloc(&busy, busy_bytes));
        h.st = compute;
    }
    CHECK_EQ(h.bm.num_total_gpu_blocks(), 3u);
    const size_t hbb = h.cache.host_block_bytes();
    void* host = nullptr;
    VLLM_HIP_CHECK(hipHostMalloc(&host, hbb * 3, hipHostMallocDefault));
    vllm::SwapPreemption swap(h.bm, h.cache, host);
    vllm::SwappableSequence a, b;
    a.seq_id = 1;
    b.seq_id = 2;
    std::vector<vllm::SwappableSequence*> running;
    std::deque<vllm::SwappableSequence*> waiting;

    a.block_table = h.bm.allocate_for_sequence(16);  // the prompt: one block
    running.push_back(&a);
    h.step({&a.block_table}, {0}, {16}, "prefill A");
    CHECK(h.bm.ensure_sequence_capacity(a.block_table, 17));
    CHECK_EQ(a.block_table.size(), 2u);
    h.step({&a.block_table}, {16}, {1}, "decode A");

    b.block_table = h.bm.allocate_for_sequence(16);
    CHECK_EQ(b.block_table.size(), 1u);
    running.push_back(&b);
    h.step({&b.block_table}, {0}, {16}, "prefill B");
    CHECK_EQ(h.bm.num_free_gpu_blocks(), 0u);
    h.step({&a.block_table}, {17}, {15}, "A runs to 32 tokens");

    // A needs a third block for position 33: preempt (scheduler.cpp:107-118)
    const int32_t b_gpu = b.block_table[0];
    const size_t be = h.block_elems() * eb(g.kv);
    std::vector<std::vector<uint8_t>> b_k(g.L), b_v(g.L);
    for (int l = 0; l < g.L; ++l) {
        b_k[l].resize(be);
        b_v[l].resize(be);
        VLLM_HIP_CHECK(hipMemcpy(b_k[l].data(), h.cache.k_ptr(size_t(l), size_t(b_gpu)), be, hipMemcpyDeviceToHost));
        VLLM_HIP_CHECK(hipMemcpy(b_v[l].data(), h.cache.v_ptr(size_t(l), size_t(b_gpu)), be, hipMemcpyDeviceToHost));
    }
    CHECK(!h.bm.ensure_sequence_capacity(a.block_table, 33));
    CHECK_EQ(vllm::SwapPreemption::pick_victim(running, &a), 1);
    if (side_stream) VLLM_HIP_CHECK(hipMemsetAsync(busy, 0x5a, busy_bytes, side));
    CHECK(swap.preempt_one(running, waiting, &a, side));
    swap.wait_swaps(compute);
    CHECK(h.bm.ensure_sequence_capacity(a.block_table, 33));
    CHECK_EQ(a.block_table.size(), 3u);
    CHECK(b.swapped_out);
    CHECK_EQ(b.block_table.size(), 1u);  // now a CPU block id
    CHECK_EQ(waiting.size(), 1u);
    CHECK_EQ(running.size(), 1u);
    CHECK(running[0] == &a);
    CHECK(!swap.preempt_one(running, waiting, &a, side));  // A alone: no victim
    h.step({&a.block_table}, {32}, {1}, "decode A in the third block");  // may overwrite B's old block

    // A finishes; B is re-admitted by swap-in, not replay
    h.bm.free_sequence(a.block_table);
    a.block_table.clear();
    a.finished = true;
    running.clear();
    if (side_stream) VLLM_HIP_CHECK(hipMemsetAsync(busy, 0xa5, busy_bytes, side));
    CHECK(swap.swap_in(b, side));
    swap.wait_swaps(compute);
    waiting.pop_front();
    running.push_back(&b);
    CHECK(!b.swapped_out);
    VLLM_HIP_CHECK(hipDeviceSynchronize());
    const int32_t b_new = b.block_table[0];
    for (int l = 0; l < g.L; ++l) {
        std::vector<uint8_t> k(be), v(be);
        VLLM_HIP_CHECK(hipMemcpy(k.data(), h.cache.k_ptr(size_t(l), size_t(b_new)), be, hipMemcpyDeviceToHost));
        VLLM_HIP_CHECK(hipMemcpy(v.data(), h.cache.v_ptr(size_t(l), size_t(b_new)), be, hipMemcpyDeviceToHost));
        CHECK(k == b_k[l]);
        CHECK(v == b_v[l]);
        std::memcpy(h.hk[l].data() + size_t(b_new) * be, b_k[l].data(), be);  // the oracle's mirror follows
        std::memcpy(h.hv[l].data() + size_t(b_new) * be, b_v[l].data(), be);
    }
    CHECK(h.bm.ensure_sequence_capacity(b.block_table, 17));
    CHECK_EQ(b.block_table.size(), 2u);
    h.step({&b.block_table}, {16}, {1}, "decode B after swap-in");
    VLLM_HIP_CHECK(hipDeviceSynchronize());
    (void)hipHostFree(host);
    if (side_stream) {
        (void)hipFree(busy);
        (void)hipStreamDestroy(side);
        (void)hipStreamDestroy(compute);
    }
}

}  // namespace

TEST_CASE(preemption_by_swap_reference_pressure_test) {
    run_swap_preemption_scenario({2, 3, 16, 14, 2, 64, vllm::KVDtype::kF16, vllm::KVDtype::kF16}, 6);
}

TEST_CASE(preemption_by_swap_on_a_side_stream) {
    run_swap_preemption_scenario({2, 3, 16, 14, 2, 64, vllm::KVDtype::kF16, vllm::KVDtype::kF16}, 7, true);
}

TEST_CASE(attention_step_f16_qwen05b_shape) {
    run_scenario({2, 48, 16, 14, 2, 64, vllm::KVDtype::kF16, vllm::KVDtype::kF16}, 1);
}

TEST_CASE(attention_step_f16_llama_shape_fp8_cache) {
    run_scenario({2, 48, 16, 32, 8, 128, vllm::KVDtype::kF16, vllm::KVDtype::kFP8E4M3}, 2);
}

TEST_CASE(attention_step_f32_reference_types) {
    run_scenario({2, 64, 8, 8, 2, 64, vllm::KVDtype::kF32, vllm::KVDtype::kF32}, 3);
}

TEST_CASE(attention_step_f16_qwen7b_shape_bs32) {
    run_scenario({1, 24, 32, 28, 4, 128, vllm::KVDtype::kF16, vllm::KVDtype::kF16}, 4);
}

TEST_CASE(fork_copy_on_write_and_swap_f16) {
    run_fork_swap_scenario({2, 24, 16, 14, 2, 64, vllm::KVDtype::kF16, vllm::KVDtype::kF16}, 5);
}

int main() { return check::run_all(); }
