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
#include <random>
#include <vector>

#include "check.hpp"
#include "kv_oracle.h"
#include "vllm/attention/attention_step.hpp"
#include "vllm/core/block_manager.hpp"
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

void run_scenario(const Geometry& g, uint32_t seed) {
    using vllm::KVDtype;
    std::printf("  scenario H%d Hkv%d D%d bs%d io %zuB kv %zuB\n", g.H, g.Hkv, g.D, g.bs, eb(g.io), eb(g.kv));
    const bool fp8 = g.kv == KVDtype::kFP8E4M3;
    vllm::KVCache cache(g.L, g.N, g.bs, g.Hkv, g.D, nullptr, nullptr, g.kv);
    vllm::BlockManager bm(g.bs, g.N, 0);
    const int P = 256;  // RoPE positions
    std::vector<float> cs(size_t(P) * g.D);
    VLLM_KV_CHECK(vkv_rope_cos_sin_host(10000.0f, g.D, P, cs.data()));
    float* dcs;
    VLLM_HIP_CHECK(hipMalloc(&dcs, cs.size() * 4));
    VLLM_HIP_CHECK(hipMemcpy(dcs, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    vllm::PagedAttentionLayer layer(g.H, g.Hkv, g.D, P);
    layer.attach_rope_table(dcs, P);
    const int max_mb = 8;
    vllm::AttentionMetadata md(8, 128, max_mb, g.bs);

    // host mirror of both layers' caches
    const size_t row = size_t(g.Hkv) * g.D;
    const size_t layer_elems = size_t(g.N) * g.bs * row;
    std::vector<std::vector<uint8_t>> hk(g.L), hv(g.L);
    std::vector<std::vector<float>> hks(g.L), hvs(g.L);
    for (int l = 0; l < g.L; ++l) {
        hk[l].assign(layer_elems * eb(g.kv), 0);
        hv[l].assign(layer_elems * eb(g.kv), 0);
        if (fp8) {
            hks[l].assign(size_t(g.N) * g.bs * g.Hkv, 0.f);
            hvs[l].assign(size_t(g.N) * g.bs * g.Hkv, 0.f);
        }
    }

    std::vector<int> ctx = {0, 0, 0, 0};
    std::vector<int> prompt = {5, 33, 1, 18};
    std::vector<std::vector<int32_t>> tables(4);
    for (int s = 0; s < 4; ++s) {
        tables[s] = bm.allocate_for_sequence(size_t(prompt[s]));
        CHECK(!tables[s].empty());
    }
    const std::vector<std::vector<int>> steps = {{5, 33, 1, 18}, {1, 1, 1, 1}, {1, 1, 1, 1}, {1, 7, 1, 1}};
    std::mt19937 gen(seed);
    std::normal_distribution<float> nd(0.f, 0.6f);
    for (size_t step = 0; step < steps.size(); ++step) {
        std::vector<vllm::StepSequence> ss;
        std::vector<int32_t> qsl = {0};
        for (int s = 0; s < 4; ++s) {
            const int n = steps[step][s];
            CHECK(bm.ensure_sequence_capacity(tables[s], size_t(ctx[s] + n)));
            ss.push_back({tables[s].data(), int32_t(tables[s].size()), ctx[s], n});
            qsl.push_back(qsl.back() + n);
        }
        const int T = qsl.back();
        md.build(ss, nullptr);
        CHECK_EQ(md.num_tokens(), T);
        CHECK_EQ(md.max_query_len(), *std::max_element(steps[step].begin(), steps[step].end()));
        std::vector<int32_t> slots(T), pos(T), cl(4);
        for (int s = 0, t = 0; s < 4; ++s) {
            for (int j = 0; j < steps[step][s]; ++j, ++t) {
                pos[t] = ctx[s] + j;
                slots[t] = tables[s][pos[t] / g.bs] * g.bs + pos[t] % g.bs;  // attention.cpp:85-94
            }
            cl[s] = ctx[s] + steps[step][s];
        }
        std::vector<int32_t> bt(4 * max_mb, 0);
        for (int s = 0; s < 4; ++s) std::copy(tables[s].begin(), tables[s].end(), bt.begin() + s * max_mb);

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
            layer.forward(dout, dq, dk, dv, g.io, cache, md, size_t(l), nullptr);
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
                                 fp8 ? hvs[l].data() : nullptr, bt.data(), cl.data(), qsl.data(), 4, g.H, g.Hkv, g.D,
                                 g.bs, max_mb, 1.0f / std::sqrt(float(g.D)), int32_t(g.kv), 1);

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
            if (worst > 1.0) std::printf("    step %zu layer %d: worst error ratio %.3f\n", step, l, worst);
            CHECK(worst <= 1.0);
            (void)hipFree(dq);
            (void)hipFree(dk);
            (void)hipFree(dv);
            (void)hipFree(dout);
        }
        for (int s = 0; s < 4; ++s) ctx[s] += steps[step][s];
    }
    (void)hipFree(dcs);
}

}  // namespace

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

int main() { return check::run_all(); }
